"""The engine with the tensor types as found in a GGUF: every matrix goes
through mm() (main.c:1669-1694) and may be F32, F16, BF16, Q4_K, Q5_K or
Q6_K; the token tables go through emb_lookup (main.c:1696-1723) and the tied
LM head through mm() and the soft-cap (main.c:1780-1796).  A synthetic model
mixes them so that every route of the decode step and the prompt chunks
runs: dense attention outputs, FFN down and PLE projections, gate and up of
different types (no fused gate|up kernel), Q projections without Q8_K
activations beside a Q8_K V, a Q4_K token table for both the lookup and the
LM head.  And the reference's --f32-matmul switch (main.c:1680-1683): Q4_K /
Q5_K through dequantized fp32 weights.

Parity as tests/test_gpu_engine.py: each layer teacher-forced against the
oracle's forward with its own and with the engine's Q8_K (engine_check.py),
same bars.
"""
import dataclasses

import numpy as np
import pytest

import synth
from engine_check import StepCheck, assert_bars, prefill_checks, rel

pytestmark = pytest.mark.gpu

MEDIAN_TOL = 2e-6      # per-layer, oracle's own Q8_K
Q8_TOL = 1e-4          # per-layer, engine's Q8_K injected: the dense and --f32-matmul GEMVs sum
                       # up to 2560 fp32 products in another order (observed <= 4e-5)
LOGIT_TOL = 1e-5

MIXED = (
    ("token_embd.weight", synth.Q4_K),
    ("per_layer_token_embd.weight", synth.F16),
    ("per_layer_model_proj.weight", synth.F16),
    ("blk.1*.attn_output.weight", synth.F16),
    ("blk.2*.ffn_down.weight", synth.BF16),
    ("blk.3.ffn_gate.weight", synth.Q6_K), ("blk.3.ffn_up.weight", synth.F32),
    ("blk.4.ffn_gate.weight", synth.Q5_K), ("blk.4.ffn_up.weight", synth.Q4_K),
    ("blk.5.attn_q.weight", synth.Q6_K),
    ("blk.6.attn_q.weight", synth.F16), ("blk.6.attn_k.weight", synth.F32), ("blk.6.attn_v.weight", synth.Q5_K),
    ("blk.7.inp_gate.weight", synth.F32), ("blk.8.inp_gate.weight", synth.Q6_K),
    ("blk.9.proj.weight", synth.F16), ("blk.1?.proj.weight", synth.Q5_K),
    ("blk.2*.attn_q.weight", synth.Q5_K),
)


def _model(tmp_path_factory, types, name):
    s = dataclasses.replace(synth.tiny_shape(rope_freqs=True), types=types)
    p = str(tmp_path_factory.mktemp("gguf") / name)
    synth.write_model_gguf(p, s, seed=4)
    return p


@pytest.fixture(scope="module")
def mixed_path(tmp_path_factory):
    return _model(tmp_path_factory, MIXED, "mixed.gguf")


@pytest.fixture(scope="module")
def plain_path(tmp_path_factory):
    return _model(tmp_path_factory, (), "plain.gguf")


def _decode_and_prefill(path, orc, f32_matmul=False):
    """teacher-forced decode (24 positions, logits at each) and a batched
    prefill of the same tokens, both against the oracle"""
    import g4
    from oracle import OracleModel
    om = OracleModel(orc, path, max_seq=64)
    em = g4.Engine(path, max_seq=64)
    orc.L.or_set_f32_matmul(int(f32_matmul))
    try:
        em.set_f32_matmul(f32_matmul)
        toks = np.random.default_rng(11).integers(0, om.vocab, 24)
        em.set_trace(True)
        checks, lerr = [], []
        for pos, t in enumerate(toks):
            em.forward(int(t), pos, 1)
            sc = StepCheck.engine(em, om, int(t), pos, 1)
            checks.append(sc)
            lerr.append(rel(em.logits(), sc.logits_q8))
        em.set_trace(False)
        assert_bars(checks, "decode", MEDIAN_TOL, Q8_TOL)
        assert max(lerr) < LOGIT_TOL, max(lerr)
        em.set_prefill_chunk(9)
        tr, qt = em.prefill_trace(toks, 0, q8=True)
        assert_bars(prefill_checks(om, toks, tr, qt), "prefill", MEDIAN_TOL, Q8_TOL)
    finally:
        orc.L.or_set_f32_matmul(0)
        em.close()
        om.close()


def test_mixed_types(mixed_path, orc):
    _decode_and_prefill(mixed_path, orc)


def test_f32_matmul(plain_path, orc):
    _decode_and_prefill(plain_path, orc, f32_matmul=True)


def test_mixed_graph_equals_eager(mixed_path):
    """One captured graph per decode step equals the eager launches on the
    mixed model, greedy and sampled, and after switching to --f32-matmul (the
    graphs are recaptured)."""
    import g4
    em = g4.Engine(mixed_path, max_seq=64)
    prompt = [5, 77, 301, 12, 9, 400, 31]
    try:
        for f32 in (False, True):
            em.set_f32_matmul(f32)
            a = em.generate_greedy(prompt, 16, use_graph=True)[0]
            b = em.generate_greedy(prompt, 16, use_graph=False)[0]
            assert np.array_equal(a, b), (f32, a, b)
            a = em.generate(prompt, 16, 0.8, 0.9, 40, 1.2, 16, 5, use_graph=True)[0]
            b = em.generate(prompt, 16, 0.8, 0.9, 40, 1.2, 16, 5, use_graph=False)[0]
            assert np.array_equal(a, b), (f32, a, b)
    finally:
        em.close()
