"""Parity of the engine at the shape the decode benchmark runs: the synthetic
E4B GGUF (42 layers, hidden 2560, FFN 10240, 8 q / 2 kv heads, head_dim
256/512, window 512, layers 24..41 reading donors 22/23, vocab 262144 with
the tied Q6_K head, Q4_K_M mix, seed 4).  At this width the fused paths the
benchmark times are the ones that run: the Q|K|V launch with the residual
step as its prologue and the x / x_alt ping-pong (engine.c enqueue_step),
the streaming gate|up GEMV, the K-slice Q6_K FFN down, the PLE inp_gate
launch with its prologue, and the 262144-row soft-capped LM head.

Phase 1, the prompt: 511 tokens prefilled in one chunk (batched GEMMs,
attention over the chunk's rows) with each layer's input rows and Q8_K rows
traced.  The oracle fills its KV cache position by position from those
inputs and Q8_K (or_forward_inject_kv) and runs whole layers at sampled
positions (engine_check.StepCheck: its own Q8_K, then the engine's).  The
engine's K/V cache rows are compared with the oracle's.

Phase 2, decode: graph-replayed decode steps at positions 511..516 (the
512-slot rings wrap at 512) are traced and checked the same way, with the
K/V rows each step appends, the full 262144 soft-capped logits and the
greedy token.

Bars (relative, max |diff| / max |ref| per vector):
  MEDIAN_TOL  layers, oracle's own Q8_K (median);
  Q8_TOL      every layer with the engine's Q8_K injected, and every K/V
              cache row; a layer above it with the oracle's own Q8_K must
              show single-step Q8_K differences;
  LOGIT_TOL   logits (the LM head GEMV bar, 1e-5).
"""
import numpy as np
import pytest

import synth
from engine_check import StepCheck, as_q8, assert_bars, rel

pytestmark = pytest.mark.gpu

N_PROMPT = 512                     # prompt tokens; the last one starts decode
SAMPLE = (0, 1, 7, 255, 509, 510)  # prompt positions checked layer by layer
DECODE_STEPS = 6                   # positions 511..516
MAX_SEQ = 1024

MEDIAN_TOL = 2e-6
Q8_TOL = 1e-5          # engine's Q8_K injected (observed <= 1e-6: fp32 order only)
LOGIT_TOL = 1e-5


@pytest.fixture(scope="module")
def e4b(orc):
    import g4
    from oracle import OracleModel
    path = synth.e4b_gguf(4)
    print(f"E4B GGUF: {path}", flush=True)
    em = g4.Engine(path, max_seq=MAX_SEQ)
    om = OracleModel(orc, path, max_seq=MAX_SEQ)
    assert (em.dim, em.hidden, em.n_layers, em.n_heads, em.n_kv, em.vocab, em.window) == \
        (2560, 10240, 42, 8, 2, 262144, 512)
    yield em, om
    em.close()
    om.close()


def _prompt(vocab):
    return np.random.default_rng(4).integers(0, vocab, N_PROMPT).astype(np.int32)


@pytest.fixture(scope="module")
def prefill_run(e4b):
    em, om = e4b
    prompt = _prompt(em.vocab)
    m = N_PROMPT - 1
    print("prefill 511 tokens (one chunk), traced", flush=True)
    tr, qt = em.prefill_trace(prompt[:m], 0, q8=True)      # (L + 1, m, dim), (L, m, slots, blocks, 292)
    checks = []
    for p in range(m):
        X, Q = tr[:, p, :], as_q8(qt[:, p])
        if p in SAMPLE:
            checks.append(StepCheck(om, X, Q, int(prompt[p]), p, 0))
        else:
            om.forward_inject_kv(int(prompt[p]), p, X, Q)
    del tr, qt
    print("oracle filled 511 positions", flush=True)
    kv_err = []
    for l in range(min(em.n_layers, 24)):
        kvd, _ = em.kv_info(l)
        ke, ve = em.kv(l, 0, m)
        ko, vo = om.kv(l)
        kv_err += [rel(ke[p], ko[p, :kvd]) for p in range(m)] + [rel(ve[p], vo[p, :kvd]) for p in range(m)]
    return {"prompt": prompt, "checks": checks, "kv_err": np.array(kv_err)}


@pytest.fixture(scope="module")
def decode_run(e4b, prefill_run):
    em, om = e4b
    tok = int(prefill_run["prompt"][-1])
    steps = []
    em.set_trace(True)
    try:
        for s in range(DECODE_STEPS):
            pos = N_PROMPT - 1 + s
            toks, _ = em.decode_steps(tok, pos, 1, use_graph=True, record=True)
            lg = em.logits()
            sc = StepCheck.engine(em, om, tok, pos, 1)
            kv = []
            for l in range(24):
                kvd, slots = em.kv_info(l)
                ke, ve = em.kv(l, pos % slots, 1)
                ko, vo = om.kv(l)
                kv += [rel(ke[0], ko[pos, :kvd]), rel(ve[0], vo[pos, :kvd])]
            steps.append({"check": sc, "tok": int(toks[0]), "logits": lg, "kv_err": max(kv)})
            print(sc.summary(), flush=True)
            tok = int(toks[0])
    finally:
        em.set_trace(False)
    return steps


def test_e4b_prefill_layers(prefill_run):
    assert_bars(prefill_run["checks"], f"E4B prefill positions {SAMPLE}", MEDIAN_TOL, Q8_TOL)


def test_e4b_prefill_kv_cache(prefill_run):
    e = prefill_run["kv_err"]
    print(f"prefill K/V rows: median {np.median(e):.2e} p99 {np.percentile(e, 99):.2e} max {e.max():.2e}")
    assert e.max() < Q8_TOL


def test_e4b_decode_layers(decode_run):
    """Every layer of every graph-replayed step, and the K/V rows it appended."""
    assert_bars([st["check"] for st in decode_run], "E4B graph decode 511..516", MEDIAN_TOL, Q8_TOL)
    for st in decode_run:
        assert st["kv_err"] < Q8_TOL, (st["check"].pos, st["kv_err"])


def test_e4b_decode_logits_and_greedy(decode_run):
    """The 262144 soft-capped logits of each step (the LM head kernel's
    grid-stride instantiation at this row count) and the first-index argmax."""
    for st in decode_run:
        sc = st["check"]
        ref = sc.logits_q8
        print(f"pos {sc.pos}: logits rel err {rel(st['logits'], ref):.2e}, token {st['tok']}")
        assert rel(st["logits"], ref) < LOGIT_TOL, (sc.pos, rel(st["logits"], ref))
        best = int(np.argmax(ref))
        top2 = np.sort(ref)[-2:]
        if top2[1] - top2[0] > 2 * LOGIT_TOL * np.max(np.abs(ref)):
            assert st["tok"] == best, (sc.pos, st["tok"], best)
