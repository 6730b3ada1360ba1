"""Decode at a long context through the engine: max_seq 8192 gives the
full-attention layers 128 time chunks (engine.c attn_chunks: 128 for any
capacity of 4096 or more, so g4run's default context of 8192 runs this), and
with 4 q heads per kv head the fused decode attention (norms, RoPE, K/V
append and attention in one launch, main.c:1886-1950) takes its eight-wave
chunk kernel (attn.hip launch_chunk: 4 q heads per kv head and 64 or more
chunks) on every full layer.

A 4199-token prompt is prefilled in chunks of 512; the oracle's KV cache is
then loaded with the engine's cache rows (full layers: every position;
sliding layers: the last window), so the graph-replayed decode steps at
positions 4199..4201 -- past 4096 -- are checked layer by layer,
teacher-forced (engine_check.py), with attention over more than 4096 cached
positions, plus the K/V rows each step appends and the logits.
"""
import numpy as np
import pytest

import synth
from engine_check import StepCheck, assert_bars, rel

pytestmark = pytest.mark.gpu

MAX_SEQ = 8192
N_PROMPT = 4200
STEPS = 3
MEDIAN_TOL = 2e-6
Q8_TOL = 1e-5
LOGIT_TOL = 1e-5


def test_decode_long_context_g128(tmp_path, orc):
    import g4
    from oracle import OracleModel
    shape = synth.tiny_shape(rope_freqs=True, n_heads=4, n_kv=1, context=MAX_SEQ)
    path = str(tmp_path / "tiny_long.gguf")
    synth.write_model_gguf(path, shape, seed=6)
    em = g4.Engine(path, max_seq=MAX_SEQ)
    om = OracleModel(orc, path, max_seq=MAX_SEQ)
    prompt = np.random.default_rng(6).integers(0, em.vocab, N_PROMPT).astype(np.int32)
    m = N_PROMPT - 1
    checks, lerr, kverr = [], [], []
    try:
        print(f"prefill {m} tokens", flush=True)
        em.set_prefill_chunk(512)
        em.prefill(prompt[:m], 0)
        n_store = min(em.n_layers, 24)
        full = 0
        for l in range(n_store):
            kvd, slots = em.kv_info(l)
            ko, vo = om.kv(l)
            if slots >= MAX_SEQ:                     # a full layer: every position
                full += 1
                ke, ve = em.kv(l, 0, m)
                ko[:m, :kvd], vo[:m, :kvd] = ke, ve
            else:                                     # a ring of `slots` positions
                ke, ve = em.kv(l, 0, slots)
                for p in range(max(0, m - slots), m):
                    ko[p, :kvd], vo[p, :kvd] = ke[p % slots], ve[p % slots]
        assert full >= 4
        print("oracle cache loaded from the engine's", flush=True)
        em.set_trace(True)
        tok = int(prompt[-1])
        for s in range(STEPS):
            pos = m + s
            toks, _ = em.decode_steps(tok, pos, 1, use_graph=True, record=True)
            sc = StepCheck.engine(em, om, tok, pos, 1)
            checks.append(sc)
            lerr.append(rel(em.logits(), sc.logits_q8))
            for l in range(n_store):
                kvd, slots = em.kv_info(l)
                ke, ve = em.kv(l, pos % slots, 1)
                ko, vo = om.kv(l)
                kverr += [rel(ke[0], ko[pos, :kvd]), rel(ve[0], vo[pos, :kvd])]
            print(sc.summary(), flush=True)
            tok = int(toks[0])
        em.set_trace(False)
    finally:
        em.close()
        om.close()
    assert_bars(checks, f"long context, positions {m}..{m + STEPS - 1}", MEDIAN_TOL, Q8_TOL)
    assert max(lerr) < LOGIT_TOL
    assert max(kverr) < Q8_TOL
