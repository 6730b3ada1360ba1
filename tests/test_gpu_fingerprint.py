"""The layer-0 dump_kv_fingerprint records (main.c:1829-1836, 1880-1951:
attn_norm, K_pre_norm, K_pre_rope, K_store, K_read0, K_readN, q_out, each
sum / l2 / max and v0..v3) from the engine's decode step and prompt chunks,
against the oracle's records of the same position run from the engine's
layer inputs and Q8_K (so only fp32 order differs).  With a real model file
(G4_GGUF), the reference's published K_store fingerprint of the --think
prompt at pos 1 (doc/design.md:988-993) is checked to its printed digits."""
import os

import numpy as np
import pytest

import synth
from engine_check import StepCheck, as_q8

pytestmark = pytest.mark.gpu

TAGS = ("attn_norm", "K_pre_norm", "K_pre_rope", "K_store", "K_read0", "K_readN", "q_out")


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_model_gguf(p, synth.tiny_shape(rope_freqs=True), seed=4)
    return p


def _close(a, b, have_a, have_b, what):
    assert np.array_equal(have_a, have_b), (what, have_a, have_b)
    for t in np.flatnonzero(have_a):
        e, o = a[t].astype(np.float64), b[t].astype(np.float64)
        scale = max(abs(o[1]), 1e-30)                    # the vector's l2 norm
        # sum: up to 1e-5 of l2 * sqrt(n) in cancellation; l2, max, values: 1e-5 relative
        assert abs(e[0] - o[0]) <= 1e-4 * scale, (what, TAGS[t], e, o)
        assert np.all(np.abs(e[1:] - o[1:]) <= 1e-5 * np.maximum(np.abs(o[2]), 1e-30)), (what, TAGS[t], e, o)


def test_decode_fingerprints(model_path, orc):
    import g4
    from oracle import OracleModel
    em = g4.Engine(model_path, max_seq=64)
    om = OracleModel(orc, model_path, max_seq=64)
    try:
        em.set_trace(True)
        toks = [2, 105, 9, 107, 77, 31, 8, 200, 17, 3, 99, 150]
        for dump_at in (0, 1, 5, 11):                    # 11: the 8-slot ring no longer holds position 0
            em.set_dump_hidden_at(dump_at)
            for pos in range(dump_at + 1):
                em.forward(toks[pos], pos, 0)
                StepCheck.engine(em, om, toks[pos], pos, 0)
            fe, he = em.kv_fingerprint()
            fo, ho = om.kv_fingerprint()
            if dump_at >= 8:
                assert not he[4]                         # K_read0 gone from the ring
                ho = ho.copy()
                ho[4] = False
            _close(fe, fo, he, ho, f"decode pos {dump_at}")
    finally:
        em.close()
        om.close()


def test_prefill_fingerprints(model_path, orc):
    """positions inside the first chunk and inside a later one (K_read0 then
    comes from the cache)"""
    import g4
    from oracle import OracleModel
    om = OracleModel(orc, model_path, max_seq=64)
    toks = np.array([2, 105, 9, 107, 77, 31, 8, 200, 17], np.int32)
    for dump_at in (1, 6):
        em = g4.Engine(model_path, max_seq=64)
        try:
            em.set_prefill_chunk(4)
            em.set_dump_hidden_at(dump_at)
            tr, qt = em.prefill_trace(toks, 0, q8=True)
            fe, he = em.kv_fingerprint()
        finally:
            em.close()
        for p in range(dump_at + 1):
            StepCheck(om, tr[:, p, :], as_q8(qt[:, p]), int(toks[p]), p, 0)
        fo, ho = om.kv_fingerprint()
        _close(fe, fo, he, ho, f"prefill pos {dump_at}")
    om.close()


GOLDEN_K_STORE_POS1 = (1.6829, 2.8726, 0.8384, -0.006941, -0.041012, -0.043630, -0.057859)
THINK_PROMPT = [2, 105, 9731, 107, 98, 107, 106, 107, 105, 2364, 107, 51953, 169845, 237457, 236881, 106, 107, 105,
                4368, 107]


@pytest.mark.skipif(not os.environ.get("G4_GGUF"), reason="set G4_GGUF to the gemma-4-E4B-it Q4_K_M GGUF to check "
                                                          "the published fingerprint")
def test_published_k_store_fingerprint():
    import g4
    em = g4.Engine(os.environ["G4_GGUF"], max_seq=64)
    try:
        em.set_dump_hidden_at(1)
        em.prefill(THINK_PROMPT, 0)
        fe, he = em.kv_fingerprint()
    finally:
        em.close()
    assert he[3]
    got = fe[3]
    assert np.allclose(got[:3], GOLDEN_K_STORE_POS1[:3], atol=1e-4) and \
        np.allclose(got[3:], GOLDEN_K_STORE_POS1[3:], atol=1e-6), got
