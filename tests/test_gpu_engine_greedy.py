"""The greedy step's LM head with the argmax in the same pass
(g4_mm_argmax_row through the engine's lm_mode 2): the reference's
fast_argmax route, taken when temp <= 0, repeat penalty <= 1 and the model
has no logit soft-cap (main.c:2348; logits_tied lm_mode 2 -> mm_argmax_row,
main.c:1570-1667, 1784-1786).  mm_argmax_row computes each row's value with
the same loop as mm_quant_rows (Q6_K) or the same Q8_K dot (Q4_K / Q5_K), so
its token is the first-index argmax of the logits logits_tied would produce;
the engine uses the fused pass for every greedy step (soft-capped models
take the argmax of the soft-capped values, as generate's greedy pick does).

Small synthetic Gemma 4 models with softcap 0: every graph-replayed decode
step is teacher-forced layer by layer against the oracle (engine_check.py),
its logits (written by the fused pass) against the oracle's logits of the
engine's final hidden state, and its token against the first-index argmax of
both (the oracle's may differ only where its top two logits lie within the
logit bar of each other).
"""
import numpy as np
import pytest

import synth
from engine_check import StepCheck, assert_bars, rel

pytestmark = pytest.mark.gpu

MEDIAN_TOL = 2e-6
Q8_TOL = 1e-5
LOGIT_TOL = 1e-5


def _run(tmp_path, orc, types=()):
    import g4
    from oracle import OracleModel
    shape = synth.tiny_shape(rope_freqs=True, softcap=0.0, types=types)
    path = str(tmp_path / "tiny_nocap.gguf")
    synth.write_model_gguf(path, shape, seed=8)
    em = g4.Engine(path, max_seq=64)
    om = OracleModel(orc, path, max_seq=64)
    prompt = [2, 105, 9, 77, 301, 12, 400]
    checks, steps = [], []
    try:
        em.set_trace(True)
        for pos, t in enumerate(prompt[:-1]):
            em.forward(t, pos, 0)
            checks.append(StepCheck.engine(em, om, t, pos, 0))
        tok = prompt[-1]
        for pos in range(len(prompt) - 1, len(prompt) + 11):
            toks, _ = em.decode_steps(tok, pos, 1, use_graph=True, record=True)
            sc = StepCheck.engine(em, om, tok, pos, 1)
            checks.append(sc)
            steps.append((int(toks[0]), em.logits(), sc.logits_q8))
            tok = int(toks[0])
        em.set_trace(False)
        # the same sequence from the untraced generate (graph replay; the
        # prompt token by token, as above)
        em.set_prefill_chunk(0)
        gen, _, _ = em.generate_greedy(prompt, len(steps), use_graph=True)
    finally:
        em.close()
        om.close()
    return checks, steps, gen


@pytest.mark.parametrize("head", ["q6k", "q4k", "f16"])
def test_greedy_fast_argmax_softcap0(tmp_path, orc, head):
    """Q6_K: the fused LM-head pass; Q4_K (mm_argmax_row's Q8_K dot route)
    and F16: g4_mm into the logits, then the argmax passes."""
    types = {"q6k": (), "q4k": (("token_embd.weight", synth.Q4_K),),
             "f16": (("token_embd.weight", synth.F16),)}[head]
    checks, steps, gen = _run(tmp_path, orc, types)
    assert_bars(checks, f"softcap 0, {head} head", MEDIAN_TOL, Q8_TOL)
    for i, (tok, lg, ref) in enumerate(steps):
        assert rel(lg, ref) < LOGIT_TOL, i
        assert tok == int(np.argmax(lg)), i                  # first index of the engine's own logits
        top = np.sort(ref.astype(np.float64))[-2:]
        if top[1] - top[0] > LOGIT_TOL * np.max(np.abs(ref)):
            assert tok == int(np.argmax(ref)), i
    want = [t for t, _, _ in steps]
    eos = 106
    n = want.index(eos) if eos in want else len(want)
    assert list(gen) == want[:n]
