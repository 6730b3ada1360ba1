"""--dump-hidden-at fingerprints (main.c:1811-1826, 1857-2010): hidden_stats
(sum and l2 in double, max |x|) of the hidden state after the embedding,
after each layer's attention residual and at each layer's end, for one
position, from eager decode steps and from prompt chunks.

The stats kernel equals the oracle's hidden_stats (to the float rounding of
its double sums); the recorded rows equal the stats of the engine's own
traced layer inputs, and the attention-residual rows agree with the oracle's
teacher-forced forward at the bars of the layer outputs.
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

P = lambda a: a.ctypes.data  # noqa: E731


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    s = synth.tiny_shape(rope_freqs=True)
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_model_gguf(p, s, seed=4)
    return p


def _stats(orc, v):
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(3, np.float32)
    orc.L.or_hidden_stats(P(v), v.size, P(out), P(out[1:]), P(out[2:]))
    return out


def _close(a, b):
    """equal to one float ulp"""
    return bool(np.all(np.abs(a.astype(np.float64) - b) <= np.spacing(np.abs(b).astype(np.float32)).astype(np.float64)))


def _stat_err(got, want):
    """max of |d sum| / l2, |d l2| / l2, |d max| / max"""
    l2 = max(float(want[1]), 1e-30)
    return max(abs(float(got[0]) - float(want[0])) / l2, abs(float(got[1]) - float(want[1])) / l2,
               abs(float(got[2]) - float(want[2])) / max(float(want[2]), 1e-30))


def _bars(errs):
    """the layer-output bars for one position's 30 layers: a few-ulp median
    and none above 3e-2; the attention residual includes the O projection,
    which runs on Q8_K activations of the attention output, so a one-ulp
    difference there can move one activation across a rounding step
    (measured: 3 of 30 layers at 1.5-3.7e-3 at one prompt position), allowed
    in under a fifth of the layers"""
    errs = np.asarray(errs)
    assert np.median(errs) < 2e-6 and np.mean(errs > 1e-5) < 0.2 and errs.max() < 3e-2, errs


def test_hidden_stats_kernel(orc):
    import g4
    lib = g4.Lib.get()
    lib.init(0)
    rng = np.random.default_rng(2)
    for n in (2560, 7, 10001):
        v = (rng.standard_normal(n) * 3).astype(np.float32)
        v[n // 2] = -40.0
        vd, od = g4.DBuf.from_array(lib, v), g4.DBuf(lib, 12)
        lib.g4_hidden_stats(vd.ptr, n, od.ptr)
        got = od.to_array(np.float32)
        want = _stats(orc, v)
        assert got[2] == want[2] == 40.0
        assert _close(got[:2], want[:2]), (got, want)


def test_dump_decode(model_path, orc):
    import g4
    from oracle import OracleModel
    om = OracleModel(orc, model_path, max_seq=64)
    em = g4.Engine(model_path, max_seq=64)
    toks = np.random.default_rng(3).integers(0, om.vocab, 10)
    at = 7
    try:
        em.set_dump_hidden_at(at)
        em.set_trace(True)
        for pos, t in enumerate(toks):
            em.forward(int(t), pos, 0)
            X = em.layer_x()
            om.forward_inject(int(t), pos, 0, X)
            if pos == at:
                rec, Xat, astats = em.hidden_stats(), X.copy(), om.attn_stats()
        em.set_trace(False)
        L = om.n_layers
        assert _close(rec[0], _stats(orc, Xat[0]))
        for l in range(L):
            assert _close(rec[2 + 2 * l], _stats(orc, Xat[l + 1])), l
        _bars([_stat_err(rec[1 + 2 * l], astats[l]) for l in range(L)])
    finally:
        em.close()
        om.close()


def test_dump_prefill_chunk(model_path, orc):
    """the dump position inside a prompt chunk (chunks of 4 tokens, position 6)"""
    import g4
    from oracle import OracleModel
    om = OracleModel(orc, model_path, max_seq=64)
    em = g4.Engine(model_path, max_seq=64)
    toks = np.random.default_rng(4).integers(0, om.vocab, 11)
    at = 6
    try:
        em.set_prefill_chunk(4)
        em.set_dump_hidden_at(at)
        tr = em.prefill_trace(toks, 0)
        rec = em.hidden_stats()
        for i, t in enumerate(toks[:at + 1]):
            om.forward_inject(int(t), i, 0, np.ascontiguousarray(tr[:, i, :]))
        astats = om.attn_stats()
        L = om.n_layers
        assert _close(rec[0], _stats(orc, tr[0, at]))
        for l in range(L):
            assert _close(rec[2 + 2 * l], _stats(orc, tr[l + 1, at])), l
        _bars([_stat_err(rec[1 + 2 * l], astats[l]) for l in range(L)])
    finally:
        em.close()
        om.close()


def test_dump_leaves_generation_unchanged(model_path):
    """generate with a dump position runs its steps eagerly and records the
    position; the tokens equal those of the graph run without a dump."""
    import g4
    em = g4.Engine(model_path, max_seq=64)
    prompt = [5, 77, 301, 12, 9, 400, 31]
    try:
        a = em.generate_greedy(prompt, 12, use_graph=True)[0]
        em.set_dump_hidden_at(10)
        b = em.generate_greedy(prompt, 12, use_graph=True)[0]
        rec = em.hidden_stats()
        em.set_dump_hidden_at(-1)
        assert np.array_equal(a, b)
        assert np.isfinite(rec).all() and (rec[:, 1] > 0).all()
    finally:
        em.close()
