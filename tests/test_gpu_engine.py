"""End-to-end parity of the C engine (libg4engine.so over libg4hip.so) with
the CPU oracle's forward() on a small synthetic Gemma 4 model: 30 layers (so
layers 24..29 read the shared KV of donors 22/23), sliding window 8 (so the
ring buffer wraps), full layers with head_dim 512 and p-RoPE factors.

Every layer is checked in isolation: the engine records each layer's input
(trace), the oracle runs the same layer from that input (or_forward_inject,
which also fills its KV cache from those inputs), and the outputs are
compared.  Most layers agree to a few ulps (tree vs sequential fp32 sums).
A Q8_K rounding that lands on the other side of .5 because its input moved by
one ulp changes one quantized activation by one step, which at this model's
width (256) moves a GEMV output by up to ~(amax/127)/(rms*sqrt(256)), a few
1e-3; such layers are rare, so the bars are on the median, the 90th
percentile, the share of layers with such a flip (under 5 %) and the
maximum.  Which layers flip depends on the GPU's summation order: two
attention kernels with the same error against the oracle (median 2e-7,
max 1.5e-5 over 40 random cases each) gave worst layers of 5.6e-3 and
1.6e-2 on this model, so the maximum allows a few flips (3e-2).  Logits are
computed from the engine's final hidden state on both sides and must agree
to 1e-5.
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

MEDIAN_TOL = 2e-6      # per-layer relative error (max |diff| / max |ref|)
P90_TOL = 2e-5
FLIP_TOL = 1e-3        # a layer above this has had a Q8_K rounding flip
FLIP_SHARE = 0.05      # ... and such layers are rare
MAX_TOL = 3e-2         # a few flips at width 256
LOGIT_TOL = 1e-5


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    s = synth.tiny_shape(rope_freqs=True)
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_model_gguf(p, s, seed=4)
    return p


@pytest.fixture(scope="module")
def pair(model_path, orc):
    import g4
    from oracle import OracleModel
    om = OracleModel(orc, model_path, max_seq=64)
    em = g4.Engine(model_path, max_seq=64)
    yield om, em
    em.close()
    om.close()


def _rel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def test_config(pair):
    om, em = pair
    assert (em.dim, em.hidden, em.n_layers, em.n_heads, em.n_kv, em.vocab, em.max_seq, em.ple_dim, em.window) == \
        (om.dim, om.hidden, om.n_layers, om.n_heads, om.n_kv, om.vocab, om.max_seq, om.ple_dim, om.window)


def test_layerwise_teacher_forced(pair):
    om, em = pair
    rng = np.random.default_rng(1)
    toks = rng.integers(0, om.vocab, 24)      # 24 positions: the window-8 ring wraps 3 times
    em.set_trace(True)
    errs, lerr = [], []
    try:
        for pos, t in enumerate(toks):
            em.forward(int(t), pos, 1)
            X = em.layer_x()
            out = om.forward_inject(int(t), pos, 1, X)
            errs += [_rel(X[l + 1], out[l]) for l in range(om.n_layers)]
            lerr.append(_rel(em.logits(), om.logits()))
    finally:
        em.set_trace(False)
    errs = np.array(errs)
    print(f"per-layer rel err: median {np.median(errs):.2e} p90 {np.percentile(errs, 90):.2e} "
          f"max {errs.max():.2e}; logits max {max(lerr):.2e}")
    assert np.median(errs) < MEDIAN_TOL
    assert np.percentile(errs, 90) < P90_TOL
    assert np.mean(errs > FLIP_TOL) < FLIP_SHARE
    assert errs.max() < MAX_TOL
    assert max(lerr) < LOGIT_TOL


def test_greedy_graph_matches_host_loop(pair):
    """generate() with the decode step replayed as one HIP graph (token and
    position advanced on the device by the argmax kernel) equals the eager
    launches and a host loop of forward() + first-index argmax over the
    read-back logits (main.c:2045-2049).  The prompt runs token by token here;
    test_gpu_prefill_engine.py covers generate() over prompt chunks."""
    _, em = pair
    em.set_prefill_chunk(0)                         # the prompt token by token, as the loop below
    prompt = [5, 77, 301, 12, 9, 400, 31]
    n_new = 24
    g_graph, _, _ = em.generate_greedy(prompt, n_new, use_graph=True)
    g_eager, _, _ = em.generate_greedy(prompt, n_new, use_graph=False)
    assert np.array_equal(g_graph, g_eager), (g_graph, g_eager)
    seq = list(prompt)
    host = []
    for pos in range(len(prompt) + n_new - 1):
        lm = 1 if pos >= len(prompt) - 1 else 0
        em.forward(seq[pos], pos, lm)
        if lm:
            nxt = int(np.argmax(em.logits()))      # numpy argmax: first index of the max
            assert em.argmax() == nxt
            if nxt == 106:                          # eos of the synthetic vocabulary
                break
            host.append(nxt)
            seq.append(nxt)
    assert np.array_equal(np.array(host, np.int32), g_eager[: len(host)]) and len(host) == len(g_eager)


def test_decode_steps_graph(pair):
    """Timed decode entry point: graph replay equals eager launches.  Each run
    starts from a fresh prefill (a sliding-window ring cannot be rewound)."""
    _, em = pair
    runs = []
    for use_graph in (True, False):
        for pos, t in enumerate([3, 1, 4, 1, 5, 9, 2, 6, 5, 3]):
            em.forward(t, pos, 0)
        toks, _ = em.decode_steps(7, 10, 12, use_graph=use_graph, record=True)
        runs.append(toks)
    assert np.array_equal(runs[0], runs[1])
