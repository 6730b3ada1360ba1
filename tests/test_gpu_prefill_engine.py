"""Batched prompt prefill of the C engine (g4e_prefill: chunks of tokens
layer by layer, batched GEMMs, attention over the chunk's query rows) against
the CPU oracle's token-by-token forward() (main.c:2366-2384 runs the prompt
that way), on the small synthetic Gemma 4 model of test_gpu_engine.py.

Each layer is checked in isolation, teacher-forced (engine_check.py): the
engine records every layer's input rows and Q8_K rows (g4e_prefill_trace_q8),
the oracle runs the same layer per token from those inputs with its own and
with the engine's Q8_K (which also fills its KV cache), and the outputs are
compared with the decode test's bars.  Without teacher forcing the two paths
drift apart with depth on this random model: a flip moves a row by ~1e-3 and
20 further layers amplify it, so an end-to-end cache comparison tests nothing
but that amplification.
"""
import numpy as np
import pytest

import synth
from engine_check import StepCheck, assert_bars, prefill_checks, rel

pytestmark = pytest.mark.gpu

MEDIAN_TOL = 2e-6      # per-layer, oracle's own Q8_K
Q8_TOL = 1e-5          # engine's Q8_K injected (observed <= 1e-6: fp32 order only)
LOGIT_TOL = 1e-5


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    s = synth.tiny_shape(rope_freqs=True)
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_model_gguf(p, s, seed=4)
    return p


@pytest.fixture(scope="module")
def orc_model(model_path, orc):
    from oracle import OracleModel
    om = OracleModel(orc, model_path, max_seq=64)
    yield om
    om.close()


def _engine(model_path, chunk):
    import g4
    em = g4.Engine(model_path, max_seq=64)
    em.set_prefill_chunk(chunk)
    return em


def test_prefill_one_chunk(model_path, orc_model):
    """24 prompt tokens in one chunk: the window-8 ring wraps 3 times, so the
    chunk's queries read positions that its own K/V rows overwrite in the ring,
    and layers 24..29 read donors 22/23 from the chunk buffers."""
    om = orc_model
    toks = np.random.default_rng(1).integers(0, om.vocab, 24)
    em = _engine(model_path, 64)
    try:
        tr, qt = em.prefill_trace(toks, 0, q8=True)
    finally:
        em.close()
    assert_bars(prefill_checks(om, toks, tr, qt), "one chunk", MEDIAN_TOL, Q8_TOL)


def test_prefill_chunks_and_calls(model_path, orc_model):
    """Chunks of 7 tokens over two calls (13 then 18 tokens at position 13):
    queries read earlier positions from the cache and their own chunk from the
    chunk buffers, across ring wraps and chunk boundaries."""
    om = orc_model
    toks = np.random.default_rng(2).integers(0, om.vocab, 31)
    em = _engine(model_path, 7)
    try:
        a = em.prefill_trace(toks[:13], 0, q8=True)
        b = em.prefill_trace(toks[13:], 13, q8=True)
    finally:
        em.close()
    tr, qt = np.concatenate([a[0], b[0]], axis=1), np.concatenate([a[1], b[1]], axis=1)
    assert_bars(prefill_checks(om, toks, tr, qt), "chunks of 7, two calls", MEDIAN_TOL, Q8_TOL)


def test_decode_after_prefill(model_path, orc_model):
    """Decode steps after a batched prefill read the caches it wrote: each
    step is teacher-forced against the oracle, whose cache holds the same
    positions computed from the engine's layer inputs, and the logits of the
    engine's final hidden state agree."""
    om = orc_model
    toks = np.random.default_rng(3).integers(0, om.vocab, 30)
    n_pre = 21
    em = _engine(model_path, 8)
    lerr = []
    try:
        tr, qt = em.prefill_trace(toks[:n_pre], 0, q8=True)
        checks = prefill_checks(om, toks[:n_pre], tr, qt)
        em.set_trace(True)
        for pos in range(n_pre, len(toks)):
            em.forward(int(toks[pos]), pos, 1)
            sc = StepCheck.engine(em, om, int(toks[pos]), pos, 1)
            checks.append(sc)
            lerr.append(rel(em.logits(), sc.logits_q8))
        em.set_trace(False)
    finally:
        em.close()
    assert_bars(checks, "prefill then decode", MEDIAN_TOL, Q8_TOL)
    assert max(lerr) < LOGIT_TOL


def test_prefill_chunk_setting(model_path):
    """The chunk length is bounded by 512 and, once the chunk buffers are
    sized, by what they hold; 0 selects the token-by-token prompt loop."""
    import g4
    em = _engine(model_path, 16)
    try:
        em.prefill([1, 2, 3], 0)
        em.set_prefill_chunk(0)
        em.set_prefill_chunk(16)
        with pytest.raises(g4.G4Error):
            em.set_prefill_chunk(17)
        with pytest.raises(g4.G4Error):
            em.set_prefill_chunk(-1)
        with pytest.raises(g4.G4Error):
            em.prefill([1, 2, 3], 62)        # positions past max_seq
    finally:
        em.close()


def test_prefill_chunking_bit_exact(model_path):
    """Each row of a chunk is computed with the same reduction order whatever
    the chunk length and wherever the call boundaries fall, so the caches
    after chunks of 3, of 8 and of 64 tokens, and after two calls, are
    bit-identical."""
    toks = np.random.default_rng(4).integers(0, 512, 26)
    caches = []
    for chunk, split in ((3, None), (8, None), (64, None), (64, 11)):
        em = _engine(model_path, chunk)
        try:
            if split:
                em.prefill(toks[:split], 0)
                em.prefill(toks[split:], split)
            else:
                em.prefill(toks, 0)
            kv = {}
            for l in range(em.n_layers):
                try:
                    _, slots = em.kv_info(l)
                except Exception:
                    continue
                kv[l] = em.kv(l, 0, min(slots, len(toks)))
            caches.append(kv)
        finally:
            em.close()
    for other in caches[1:]:
        for l, (k, v) in caches[0].items():
            assert np.array_equal(k, other[l][0]) and np.array_equal(v, other[l][1]), l


def test_unwritten_memory_reaches_no_result(model_path, monkeypatch):
    """Device buffers filled with NaN bytes when allocated (G4E_POISON=0xff)
    give bit-identical layer inputs to a normal engine, token by token and in
    prompt chunks: no kernel lets memory that nothing has written reach a
    result (the decode attention loads ring slots before it knows the
    position and must drop the ones no position has written)."""
    prompt = [5, 77, 301, 12, 9, 400, 31, 8, 200, 17, 3, 99, 150]
    runs = []
    for poison in (None, "0xff"):
        if poison:
            monkeypatch.setenv("G4E_POISON", poison)
        else:
            monkeypatch.delenv("G4E_POISON", raising=False)
        em = _engine(model_path, 5)
        try:
            em.set_trace(True)                   # token by token on unwritten caches first
            X = []
            for pos, t in enumerate(prompt):
                em.forward(t, pos, 1 if pos == len(prompt) - 1 else 0)
                X.append(em.layer_x())
            em.set_trace(False)
            lg = em.logits()
            runs.append((np.stack(X, 1), lg, em.prefill_trace(prompt, 0)))
        finally:
            em.close()
    monkeypatch.delenv("G4E_POISON", raising=False)
    for a, b in zip(runs[0], runs[1]):
        assert np.isfinite(b).all()
        assert np.array_equal(a, b)


def test_generate_uses_batched_prompt(model_path):
    """generate_greedy with a prompt chunk set prefills in chunks; its tokens
    equal a host loop of prefill() + forward() + argmax."""
    prompt = [5, 77, 301, 12, 9, 400, 31, 8, 200, 17, 3]
    em = _engine(model_path, 4)
    try:
        g, _, _ = em.generate_greedy(prompt, 10, use_graph=False)
        em.prefill(prompt[:-1], 0)
        seq, host = list(prompt), []
        for pos in range(len(prompt) - 1, len(prompt) + 9):
            em.forward(seq[pos], pos, 1)
            nxt = int(np.argmax(em.logits()))
            if nxt == 106:
                break
            host.append(nxt)
            seq.append(nxt)
    finally:
        em.close()
    assert np.array_equal(np.array(host, np.int32), g), (host, g)


def test_prefill_images_bit_exact(model_path, monkeypatch):
    """The chunk GEMMs on fp16 weight images (the default) and on the
    quantized tensors (G4E_PREFILL_IMAGES=0) give bit-identical layer inputs
    and caches: the images hold the same integers sc * q the quantized
    kernel forms in registers."""
    prompt = np.random.default_rng(9).integers(0, 512, 21)
    runs = []
    for flag in (None, "0"):
        if flag:
            monkeypatch.setenv("G4E_PREFILL_IMAGES", flag)
        else:
            monkeypatch.delenv("G4E_PREFILL_IMAGES", raising=False)
        em = _engine(model_path, 8)
        try:
            tr = em.prefill_trace(prompt, 0)
            kv = []
            for l in range(2):
                _, slots = em.kv_info(l)
                kv.append(em.kv(l, 0, min(slots, len(prompt))))
            runs.append((tr, kv))
        finally:
            em.close()
    monkeypatch.delenv("G4E_PREFILL_IMAGES", raising=False)
    assert np.array_equal(runs[0][0], runs[1][0])
    for (k0, v0), (k1, v1) in zip(runs[0][1], runs[1][1]):
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
