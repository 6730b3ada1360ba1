"""GPU parity of the device sampler (g4_sample) with generate's sampling
(main.c:2035-2126): apply_repetition_penalty, then sample_token -- greedy,
top-k 40 / temperature / plain or top-p draw from the xorshift64* stream.

The oracle's or_apply_repetition_penalty and or_sample_token are pinned to
the reference's own functions by the golden vectors (tests/test_golden.py).
Bars: the penalised logits, the greedy token, the top-k list order and the
rng state are bit-exact; a sampled token equals the oracle's unless the coin
lies within 1e-5 of a step of the cdf, where the device expf (which may
differ from glibc's by an ulp) can legitimately pick the neighbour -- those
draws are counted and must be rare.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P = lambda a: a.ctypes.data  # noqa: E731
F = C.c_float
N = 262144


@pytest.fixture(scope="module")
def lib():
    from g4 import Lib
    L = Lib.get()
    L.init(0)
    L.L.g4_set_stream(None)
    return L


def dbuf(lib, a):
    from g4 import DBuf
    return DBuf.from_array(lib, np.ascontiguousarray(a))


def _rng_f32(state):
    """rng_f32 (main.c:2035-2040) on a Python int: (new state, coin)"""
    m = (1 << 64) - 1
    x = state
    x ^= x >> 12
    x ^= (x << 25) & m
    x ^= x >> 27
    c = np.float32(((x * 0x2545F4914F6CDD1D) & m) >> 40) / np.float32(1 << 24)
    return x, float(c)


def _margin(lg, temp, topp, topk, state):
    """distance in float64 of the draw's coin(s) from the cdf steps (and of
    the top-p cut from topp) that decide sample_token's result"""
    order = np.lexsort((np.arange(lg.size), -lg.astype(np.float64)))[:topk]
    v = lg[order].astype(np.float64)
    p = np.exp((v - v[0]) / temp)
    p /= p.sum()
    cdf = np.cumsum(p)
    s1, c1 = _rng_f32(state)
    if topp <= 0.0 or topp >= 1.0:
        return float(np.min(np.abs(cdf - c1)))
    last = int(np.argmax(cdf > topp)) if (cdf > topp).any() else topk - 1
    _, c2 = _rng_f32(s1)
    r = c2 * cdf[last]
    return float(min(np.min(np.abs(cdf[:last + 1] - r)), np.min(np.abs(cdf - topp))))


class Sampler:
    """device buffers for g4_sample"""

    def __init__(self, lib, logits, hist=None, cap=256):
        from g4 import DBuf
        self.lib = lib
        self.n = logits.size
        self.lg = dbuf(lib, logits)
        self.part = DBuf(lib, lib.L.g4_sample_part_bytes(self.n))
        h = np.zeros(cap, np.int32)
        nh = 0
        if hist is not None:
            h[:hist.size] = hist
            nh = hist.size
        self.hist = dbuf(lib, h)
        self.hn = dbuf(lib, np.array([nh], np.int32))
        self.cap = cap
        self.rng = DBuf(lib, 8)
        self.out = DBuf(lib, 4)
        self.step = dbuf(lib, np.array([0, 10], np.int32))

    def seed(self, s):
        self.rng.write(np.array([s], np.uint64))

    def __call__(self, temp, topp, topk, penalty=1.0, last_n=64, step=False):
        self.lib.g4_sample(self.lg.ptr, self.n, F(temp), F(topp), topk, F(penalty), last_n, self.hist.ptr,
                           self.hn.ptr, self.cap, self.rng.ptr, self.part.ptr, self.out.ptr,
                           self.step.ptr if step else None, self.step.ptr + 4 if step else None)
        return int(self.out.to_array(np.int32)[0])

    def state(self):
        return int(self.rng.to_array(np.uint64)[0])


def _logits(rng, n=N):
    lg = (rng.standard_normal(n) * 3).astype(np.float32)
    return lg


@pytest.mark.parametrize("penalty,last_n", [(1.3, 64), (1.1, 0), (2.0, 500), (1.5, 5), (1.0, 64)])
def test_penalty_and_greedy(lib, orc, penalty, last_n):
    """The penalty (written back to the logits) is bit-exact, and the greedy
    token is the oracle's first index of the penalised maximum."""
    rng = np.random.default_rng(int(penalty * 100) + last_n)
    lg = _logits(rng)
    hist = rng.integers(0, N, 200).astype(np.int32)
    top = int(np.argmax(lg))
    hist[[3, 50, 120, 199]] = top               # the maximum, penalised four times
    hist[[60, 61]] = int(np.argmin(lg))          # a negative logit, twice
    s = Sampler(lib, lg, hist)
    tok = s(0.0, 1.0, 40, penalty, last_n)
    want = lg.copy()
    orc.L.or_apply_repetition_penalty(P(want), P(hist), hist.size, penalty, last_n)
    got = s.lg.to_array(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    st = np.array([1], np.uint64)
    wc = want.copy()                             # held: P() keeps no reference
    assert tok == orc.L.or_sample_token(P(wc), N, 0.0, 1.0, 40, P(st))


def test_greedy_ties_and_sizes(lib, orc):
    """First index of a tied maximum, -0.0 equal to +0.0, and sizes that are
    not multiples of the 4096-logit slices (or of 4)."""
    rng = np.random.default_rng(3)
    for n in (N, N - 101, 1000, 7):
        lg = -np.abs(_logits(rng, n))
        lg[n // 3] = -0.0
        lg[n - 1] = 0.0
        s = Sampler(lib, lg)
        assert s(0.0, 1.0, 1) == n // 3
        lg[[n // 2, n // 5]] = 5.0
        s = Sampler(lib, lg)
        assert s(0.0, 1.0, 40 if n >= 40 else n) == n // 5


def test_nan_logits(lib, orc):
    """NaN logits after the first top-k positions: the greedy token and the
    sampled tokens equal or_sample_token's (the reference's comparisons never
    admit such a NaN into its list)."""
    rng = np.random.default_rng(17)
    lg = _logits(rng)
    lg[[100, 7000, 9000, N - 1]] = np.nan
    lg[8000] = lg[~np.isnan(lg)].max() + 0.5
    lg[8001] = np.nan
    s = Sampler(lib, lg)
    st = np.array([1], np.uint64)
    lc = lg.copy()
    assert s(0.0, 1.0, 40) == orc.L.or_sample_token(P(lc), N, 0.0, 1.0, 40, P(st)) == 8000
    state = 99
    s.seed(state)
    for i in range(20):
        st = np.array([state], np.uint64)
        lc = lg.copy()
        want = orc.L.or_sample_token(P(lc), N, 0.8, 0.9, 40, P(st))
        got = s(0.8, 0.9, 40)
        if got != want:
            assert _margin(lg, 0.8, 0.9, 40, state) < 1e-5, (i, got, want)
        state = int(st[0])
        assert s.state() == state


@pytest.mark.parametrize("temp,topp,topk", [(0.6, 0.9, 40), (1.0, 1.0, 40), (0.8, 0.95, 40), (0.7, 0.5, 10),
                                            (1.5, 0.0, 64), (0.3, 0.9, 1)])
def test_draws_match_oracle(lib, orc, temp, topp, topk):
    """60 successive draws from one seed: each token equals or_sample_token's
    from the same rng state (unless the coin is within 1e-5 of a cdf step),
    and the rng state advances exactly as rng_f32's."""
    rng = np.random.default_rng(int(temp * 10 + topk))
    lg = _logits(rng)
    lg[rng.integers(0, N, 30)] = lg.max() - rng.uniform(0, 1, 30).astype(np.float32)   # a crowded top
    s = Sampler(lib, lg)
    state = 12345 + topk
    s.seed(state)
    skipped = 0
    for i in range(60):
        st = np.array([state], np.uint64)
        lc = lg.copy()                           # held: P() keeps no reference
        want = orc.L.or_sample_token(P(lc), N, temp, topp, topk, P(st))
        margin = _margin(lg, temp, topp, topk, state)
        got = s(temp, topp, topk)
        if got != want:
            assert margin < 1e-5, (i, got, want, margin)
            skipped += 1
        state = int(st[0])
        assert s.state() == state, i
    assert skipped <= 2


def test_step_and_history(lib):
    """The token becomes the next step's input (dtok), the position advances,
    and the token is appended to the history until it is full."""
    rng = np.random.default_rng(5)
    lg = _logits(rng)
    s = Sampler(lib, lg, np.array([1, 2, 3], np.int32), cap=5)
    s.seed(99)
    toks = [s(0.8, 0.9, 40, step=True) for _ in range(4)]
    step = s.step.to_array(np.int32)
    assert step[0] == toks[-1] and step[1] == 14
    h = s.hist.to_array(np.int32)
    assert s.hn.to_array(np.int32)[0] == 5
    assert list(h) == [1, 2, 3, toks[0], toks[1]]


def test_sample_errors(lib):
    from g4 import G4Error
    lg = np.zeros(N, np.float32)
    s = Sampler(lib, lg)
    for topk in (0, 65):
        with pytest.raises(G4Error):
            s(0.8, 0.9, topk)
    big = Sampler(lib, np.zeros(16, np.float32))
    with pytest.raises(G4Error):
        big(0.8, 0.9, 40)                       # top-k larger than n
    with pytest.raises(G4Error):
        lib.g4_sample(s.lg.ptr, N + 1, F(0.8), F(0.9), 40, F(1.0), 64, None, None, 0, s.rng.ptr, s.part.ptr,
                      s.out.ptr, None, None)   # more than 262144 logits
    with pytest.raises(G4Error):
        lib.g4_sample(s.lg.ptr, N, F(0.8), F(0.9), 40, F(1.3), 64, None, None, 0, s.rng.ptr, s.part.ptr,
                      s.out.ptr, None, None)   # a penalty without a history


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    import synth
    s = synth.tiny_shape(rope_freqs=True)
    p = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    synth.write_model_gguf(p, s, seed=4)
    return p


@pytest.mark.parametrize("temp,topp,topk,penalty,last_n,seed", [
    (0.6, 0.9, 40, 1.0, 64, 7),       # the reference's defaults
    (1.0, 1.0, 40, 1.3, 8, 3),        # plain draw, penalty over the last 8 tokens
    (0.8, 0.5, 10, 1.1, 0, 0),        # top-p 0.5 of top-10, penalty over all; seed 0 means 1
    (0.0, 0.9, 40, 1.5, 64, 5),       # greedy after the penalty
])
def test_generate_sampled(model_path, orc, temp, topp, topk, penalty, last_n, seed):
    """generate() with the device sampler: the graph replay equals the eager
    launches token for token, and both equal a host loop of forward() + the
    oracle's apply_repetition_penalty and sample_token on the read-back
    logits with the same xorshift64* stream (compared up to a draw that lands
    within 1e-5 of a cdf step, if any)."""
    import g4
    em = g4.Engine(model_path, max_seq=64)
    prompt = [5, 77, 301, 12, 9, 400, 31]
    n_new = 24
    try:
        g1, _, _ = em.generate(prompt, n_new, temp, topp, topk, penalty, last_n, seed, use_graph=True)
        g2, _, _ = em.generate(prompt, n_new, temp, topp, topk, penalty, last_n, seed, use_graph=False)
        assert np.array_equal(g1, g2), (g1, g2)
        em.prefill(prompt[:-1], 0)
        state = seed if seed else 1
        seq, host, n_cmp = list(prompt), [], None
        for pos in range(len(prompt) - 1, len(prompt) + n_new - 1):
            em.forward(seq[pos], pos, 1)
            lg = em.logits()
            if penalty > 1.0 and host:
                h = np.array(host, np.int32)
                orc.L.or_apply_repetition_penalty(P(lg), P(h), h.size, penalty, last_n)
            near = temp > 0 and _margin(lg, temp, topp, topk, state) < 1e-5
            st = np.array([state], np.uint64)
            nxt = orc.L.or_sample_token(P(lg), lg.size, temp, topp, topk, P(st))
            state = int(st[0])
            if near:
                n_cmp = len(host)
                break
            if nxt == 106:                       # eos of the synthetic vocabulary
                break
            host.append(nxt)
            seq.append(nxt)
        if n_cmp is None:
            assert np.array_equal(g1, np.array(host, np.int32)), (g1, host)
        else:
            assert np.array_equal(g1[:n_cmp], np.array(host[:n_cmp], np.int32))
        if temp <= 0 and penalty <= 1.0:
            assert np.array_equal(g1, em.generate_greedy(prompt, n_new, use_graph=False)[0])
    finally:
        em.close()


def test_flat_logits_draws(lib, orc):
    """Nearly flat logits (three larger values, the rest equal): the top-k
    list holds the three and then the lowest indices in order, many keys
    differing only in their index; draws and the rng state equal the
    oracle's."""
    lg = np.zeros(N, np.float32)
    lg[[100, 5000, 200000]] = 1.0
    s = Sampler(lib, lg)
    state = 777
    s.seed(state)
    skipped = 0
    for i in range(20):
        st = np.array([state], np.uint64)
        lc = lg.copy()                           # held: P() keeps no reference
        want = orc.L.or_sample_token(P(lc), N, 1.0, 1.0, 40, P(st))
        margin = _margin(lg, 1.0, 1.0, 40, state)
        got = s(1.0, 1.0, 40)
        if got != want:
            assert margin < 1e-5, (i, got, want, margin)
            skipped += 1
        assert got in (100, 5000, 200000) or got < 40, got
        state = int(st[0])
        assert s.state() == state, i
    assert skipped <= 1
