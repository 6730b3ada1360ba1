"""GPU parity of the decode-step kernels other than the GEMVs: RMSNorm family,
Neox RoPE, KV append, ISWA decode attention, embedding lookup, the PLE input,
GELU gate, argmax, and the fused residual/norm/quantize kernel -- against the
CPU oracle (pinned to the reference's own functions, tests/test_oracle.py).

Bars: bit-exact where the operation order is the reference's (embedding
lookup, argmax, Q8_K of a given fp32 vector); fp32 reductions that the GPU
sums as a tree are held to a stated relative tolerance; attention to 1e-4 of
max|o| (the north-star bar for attention outputs).
"""
import ctypes as C

import numpy as np
import pytest

import synth
from oracle import Q8K_DTYPE

pytestmark = pytest.mark.gpu

P = lambda a: a.ctypes.data  # noqa: E731


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


def empty(lib, nbytes):
    from g4 import DBuf
    return DBuf(lib, nbytes)


def rel_err(got, want):
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


# ---------------------------------------------------------------------------
# norms, softmax
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n", [256, 2560, 10240, 333])
def test_rmsnorm(lib, orc, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    xd, wd, od = dbuf(lib, x), dbuf(lib, w), empty(lib, 4 * n)
    lib.g4_rmsnorm(od.ptr, xd.ptr, wd.ptr, n, C.c_float(1e-6))
    got = od.to_array(np.float32)
    want = orc.rmsnorm(x, w)
    # only the scale s differs (tree vs sequential sum of squares): a few ulps
    assert rel_err(got, want) < 2e-6


@pytest.mark.parametrize("hd,nh", [(256, 8), (512, 8), (256, 2)])
def test_rmsnorm_heads(lib, orc, hd, nh):
    rng = np.random.default_rng(hd + nh)
    v = rng.standard_normal(nh * hd).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    a = v.copy()
    orc.L.or_rmsnorm_head_inplace(P(a), P(w), nh, hd, C.c_float(1e-6))
    b = v.copy()
    orc.L.or_rmsnorm_head_noweight_inplace(P(b), nh, hd, C.c_float(1e-6))
    vd, wd = dbuf(lib, v), dbuf(lib, w)
    lib.g4_rmsnorm_head_inplace(vd.ptr, wd.ptr, nh, hd, C.c_float(1e-6))
    assert rel_err(vd.to_array(np.float32), a) < 2e-6
    vd2 = dbuf(lib, v)
    lib.g4_rmsnorm_head_noweight_inplace(vd2.ptr, nh, hd, C.c_float(1e-6))
    assert rel_err(vd2.to_array(np.float32), b) < 2e-6


def test_softmax(lib, orc):
    rng = np.random.default_rng(9)
    for n in (1, 7, 512, 4097):
        x = (rng.standard_normal(n) * 8).astype(np.float32)
        want = x.copy()
        orc.L.or_softmax(P(want), n)
        xd = dbuf(lib, x)
        lib.g4_softmax(xd.ptr, n)
        got = xd.to_array(np.float32)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-7 * want.max())


# ---------------------------------------------------------------------------
# RoPE: the angle chain is replayed exactly; only cosf/sinf may differ by ulps
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("hd,n_rot,base,use_ff", [(256, 256, 1e4, False), (512, 512, 1e6, True), (512, 512, 1e6, False),
                                                  (256, 128, 1e4, False)])
@pytest.mark.parametrize("pos", [0, 1, 7, 511, 4095, 32767])
def test_rope(lib, orc, hd, n_rot, base, use_ff, pos):
    rng = np.random.default_rng(hd + pos)
    nh = 8
    v = rng.standard_normal(nh * hd).astype(np.float32)
    ff = rng.uniform(1.0, 4.0, n_rot // 2).astype(np.float32) if use_ff else None
    want = orc.rope(v, nh, hd, n_rot, pos, base, ff)
    vd = dbuf(lib, v)
    ffd = dbuf(lib, ff) if use_ff else None
    lib.g4_apply_rope_neox(vd.ptr, nh, hd, n_rot, pos, C.c_float(base), C.c_float(1.0), ffd.ptr if use_ff else None)
    got = vd.to_array(np.float32)
    if pos == 0:
        assert np.array_equal(got, v)     # identity at pos 0 (design.md:524-534)
    assert np.max(np.abs(got - want)) <= 4e-6 * np.max(np.abs(v))


# ---------------------------------------------------------------------------
# KV append + attention
# ---------------------------------------------------------------------------
def _attn_case(lib, orc, hd, n_heads, n_kv, T, t_start, scale, seed):
    rng = np.random.default_rng(seed)
    kv_dim = n_kv * hd
    kc = rng.standard_normal((T, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((T, kv_dim)).astype(np.float32)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    # typical post-norm magnitudes: |q|,|k| ~ sqrt(hd); scale keeps softmax non-degenerate
    want = orc.attn(q, kc, vc, kv_dim, t_start, T - t_start, n_heads, n_kv, hd, scale)
    qd, kd, vd, od = dbuf(lib, q), dbuf(lib, kc), dbuf(lib, vc), empty(lib, 4 * n_heads * hd)
    lib.g4_attn_decode(qd.ptr, kd.ptr, vd.ptr, kv_dim, t_start, T - t_start, n_heads, n_kv, hd, C.c_float(scale), od.ptr)
    return od.to_array(np.float32), want


@pytest.mark.parametrize("hd", [256, 512])
@pytest.mark.parametrize("T,t_start", [(1, 0), (2, 0), (37, 0), (512, 0), (700, 188), (4096, 0), (5000, 4488)])
@pytest.mark.parametrize("scale", [1.0, 1.0 / 16])
def test_attn_decode_flat(lib, orc, hd, T, t_start, scale):
    got, want = _attn_case(lib, orc, hd, 8, 2, T, t_start, scale, seed=T + hd)
    assert rel_err(got, want) < 1e-4


@pytest.mark.parametrize("n_heads,n_kv", [(2, 1), (8, 8), (4, 2)])
def test_attn_decode_gqa_shapes(lib, orc, n_heads, n_kv):
    got, want = _attn_case(lib, orc, 256, n_heads, n_kv, 300, 0, 1.0 / 16, seed=n_heads * 10 + n_kv)
    assert rel_err(got, want) < 1e-4


def test_attn_decode_long(lib, orc):
    # a global layer at context 32768 (many chunks, log-sum-exp merge)
    got, want = _attn_case(lib, orc, 256, 8, 2, 32768, 0, 1.0 / 16, seed=32768)
    assert rel_err(got, want) < 1e-4


@pytest.mark.parametrize("hd,window,pos", [(256, 512, 100), (256, 512, 511), (256, 512, 512), (256, 512, 1500),
                                           (512, 8, 30)])
def test_kv_append_and_ring_attention(lib, orc, hd, window, pos):
    """Ring-buffer cache (slot = t % window) against the reference's flat cache
    (main.c:1798-1809), with the append of main.c:1895-1904 at every position."""
    rng = np.random.default_rng(pos + hd)
    n_heads, n_kv, eps = 8, 2, 1e-6
    kv_dim = n_kv * hd
    base = 1e4
    k_norm = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    flat_k = np.zeros((pos + 1, kv_dim), np.float32)
    flat_v = np.zeros((pos + 1, kv_dim), np.float32)
    ring_k, ring_v = empty(lib, 4 * window * kv_dim), empty(lib, 4 * window * kv_dim)
    knd = dbuf(lib, k_norm)
    for t in range(pos + 1):
        k = rng.standard_normal(kv_dim).astype(np.float32)
        v = rng.standard_normal(kv_dim).astype(np.float32)
        kk = k.copy()
        orc.L.or_rmsnorm_head_inplace(P(kk), P(k_norm), n_kv, hd, C.c_float(eps))
        kk = orc.rope(kk, n_kv, hd, hd, t, base)
        vv = v.copy()
        orc.L.or_rmsnorm_head_noweight_inplace(P(vv), n_kv, hd, C.c_float(eps))
        flat_k[t], flat_v[t] = kk, vv
        if t >= pos + 1 - window:
            kd, vd = dbuf(lib, k), dbuf(lib, v)
            lib.g4_kv_append_rope(kd.ptr, vd.ptr, knd.ptr, ring_k.ptr, ring_v.ptr, kv_dim, window, t, n_kv, hd, hd,
                                  C.c_float(base), C.c_float(1.0), None, C.c_float(eps))
    # the appended slot holds the normalised, rotated K and the normalised V
    slot = pos % window
    rk = ring_k.to_array(np.float32).reshape(window, kv_dim)
    rv = ring_v.to_array(np.float32).reshape(window, kv_dim)
    assert np.max(np.abs(rk[slot] - flat_k[pos])) < 1e-5
    assert np.max(np.abs(rv[slot] - flat_v[pos])) < 1e-5
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    t_start = max(0, pos + 1 - window)
    want = orc.attn(q, flat_k, flat_v, kv_dim, t_start, pos + 1 - t_start, n_heads, n_kv, hd, 1.0)
    qd, od = dbuf(lib, q), empty(lib, 4 * n_heads * hd)
    lib.g4_attn_decode_ring(qd.ptr, ring_k.ptr, ring_v.ptr, kv_dim, window, pos, window, n_heads, n_kv, hd,
                            C.c_float(1.0), od.ptr)
    assert rel_err(od.to_array(np.float32), want) < 1e-4


def test_attn_dev_fused_quant(lib, orc):
    """Engine form: device position, fixed chunk count, fused Q8_K output."""
    rng = np.random.default_rng(77)
    hd, nh, nkv, T = 512, 8, 2, 900
    kv_dim = nkv * hd
    kc = rng.standard_normal((T, kv_dim)).astype(np.float32)
    vc = rng.standard_normal((T, kv_dim)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    pos = 640
    want = orc.attn(q, kc, vc, kv_dim, 0, pos + 1, nh, nkv, hd, 1.0 / 16)
    G = 8
    part = empty(lib, lib.L.g4_attn_part_bytes(nh, hd, G))
    qd, kd, vd, od = dbuf(lib, q), dbuf(lib, kc), dbuf(lib, vc), empty(lib, 4 * nh * hd)
    dpos = dbuf(lib, np.array([pos], np.int32))
    q8 = empty(lib, lib.L.g4_q8K_bytes(nh * hd))
    lib.g4_attn_decode_dev(qd.ptr, kd.ptr, vd.ptr, kv_dim, 0, dpos.ptr, 0, nh, nkv, hd, C.c_float(1.0 / 16), G, part.ptr,
                           od.ptr, q8.ptr)
    got = od.to_array(np.float32)
    assert rel_err(got, want) < 1e-4
    h = np.zeros(nh * hd // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), nh * hd)
    assert h.tobytes() == orc.quantize_q8K(got).tobytes()


@pytest.mark.parametrize("hd,window,pos,G,store", [(256, 512, 700, 16, True), (256, 512, 100, 4, True),
                                                   (256, 512, 511, 16, True), (512, 0, 300, 10, True),
                                                   (512, 0, 37, 1, True), (256, 512, 900, 16, False),
                                                   (512, 0, 640, 20, False),
                                                   # the engine's full layers at max_seq >= 4096: 128 chunks,
                                                   # the eight-wave kernel
                                                   (256, 0, 4999, 128, True), (256, 0, 4999, 128, False),
                                                   (512, 0, 4999, 128, True), (512, 0, 4999, 128, False),
                                                   (256, 0, 32767, 128, True), (256, 0, 32767, 128, False),
                                                   (512, 0, 32767, 128, True), (512, 0, 32767, 128, False),
                                                   (512, 0, 100, 128, True), (256, 0, 8191, 64, True)])
def test_attn_decode_fused(lib, orc, hd, window, pos, G, store):
    """qkv_post + attention in one pass (main.c:1886-1950): raw Q/K/V of
    position pos, per-head norms, RoPE from the position's table, K/V append
    into the (ring or flat) cache, attention over the window -- against the
    oracle's norms, RoPE and attention over a flat cache.  store=False is a
    shared-KV layer: nothing is appended and the cache already holds pos.
    With 64 or more chunks (4 q heads per kv head) the launch takes the
    eight-wave kernel, the one every full layer runs at contexts of 4096 and
    more; pos 100 at G = 128 leaves most chunks empty."""
    rng = np.random.default_rng(hd + pos + G)
    nh, nkv, eps = 8, 2, 1e-6
    kv_dim = nkv * hd
    base = 1e4 if window else 1e6
    ff = None if window else rng.uniform(1.0, 4.0, hd // 2).astype(np.float32)
    q_norm = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    k_norm = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    flat_k = rng.standard_normal((pos + 1, kv_dim)).astype(np.float32)
    flat_v = rng.standard_normal((pos + 1, kv_dim)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kv_dim).astype(np.float32)
    v = rng.standard_normal(kv_dim).astype(np.float32)
    qn = q.copy()
    orc.L.or_rmsnorm_head_inplace(P(qn), P(q_norm), nh, hd, C.c_float(eps))
    qn = orc.rope(qn, nh, hd, hd, pos, base, ff)
    if store:
        kk = k.copy()
        orc.L.or_rmsnorm_head_inplace(P(kk), P(k_norm), nkv, hd, C.c_float(eps))
        flat_k[pos] = orc.rope(kk, nkv, hd, hd, pos, base, ff)
        vv = v.copy()
        orc.L.or_rmsnorm_head_noweight_inplace(P(vv), nkv, hd, C.c_float(eps))
        flat_v[pos] = vv
    t_start = max(0, pos + 1 - window) if window else 0
    want = orc.attn(qn, flat_k, flat_v, kv_dim, t_start, pos + 1 - t_start, nh, nkv, hd, 1.0)
    # device cache: a ring of `window` slots or flat; slot pos holds garbage
    # when the kernel is to append it
    slots = window if window else pos + 1
    cache_k = np.full((slots, kv_dim), 7.0, np.float32)
    cache_v = np.full((slots, kv_dim), -7.0, np.float32)
    for t in range(t_start, pos + (0 if store else 1)):
        cache_k[t % slots], cache_v[t % slots] = flat_k[t], flat_v[t]
    kc, vc = dbuf(lib, cache_k), dbuf(lib, cache_v)
    dpos = dbuf(lib, np.array([pos], np.int32))
    tab = empty(lib, 4 * hd)
    ffd = dbuf(lib, ff) if ff is not None else None
    lib.g4_rope_table(tab.ptr, dpos.ptr, 0, hd, C.c_float(base), C.c_float(1.0), ffd.ptr if ffd else None)
    qd, kd, vd = dbuf(lib, q), dbuf(lib, k), dbuf(lib, v)
    qnd, knd = dbuf(lib, q_norm), dbuf(lib, k_norm)
    part = empty(lib, lib.L.g4_attn_part_bytes(nh, hd, G))
    od = empty(lib, 4 * nh * hd)
    q8 = empty(lib, lib.L.g4_q8K_bytes(nh * hd))
    lib.g4_attn_decode_fused(qd.ptr, qnd.ptr, kd.ptr if store else None, vd.ptr if store else None,
                             knd.ptr if store else None, kc.ptr if store else None, vc.ptr if store else None,
                             kc.ptr, vc.ptr, kv_dim, window, dpos.ptr, window, nh, nkv, hd, hd, tab.ptr,
                             C.c_float(eps), C.c_float(1.0), G, part.ptr, od.ptr, q8.ptr)
    got = od.to_array(np.float32)
    assert rel_err(got, want) < 1e-4
    assert np.array_equal(qd.to_array(np.float32), q)          # q_raw is left as it was
    ck = kc.to_array(np.float32).reshape(slots, kv_dim)
    cv = vc.to_array(np.float32).reshape(slots, kv_dim)
    s = pos % slots
    assert np.max(np.abs(ck[s] - flat_k[pos])) < 1e-5 and np.max(np.abs(cv[s] - flat_v[pos])) < 1e-5
    others = [t % slots for t in range(t_start, pos)]
    assert np.array_equal(ck[others], cache_k[others]) and np.array_equal(cv[others], cache_v[others])
    h = np.zeros(nh * hd // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), nh * hd)
    assert h.tobytes() == orc.quantize_q8K(got).tobytes()



@pytest.mark.parametrize("nh,nkv,hd,window,pos,G,store,qtype,d", [(8, 2, 256, 512, 700, 16, True, 12, 2560),
                                                                 (8, 2, 256, 512, 900, 16, False, 12, 2560),
                                                                 (8, 2, 256, 512, 100, 4, True, 13, 2560),
                                                                 (8, 2, 256, 0, 37, 1, True, 12, 200),
                                                                 (16, 2, 256, 512, 600, 16, True, 12, 2560),
                                                                 (16, 4, 256, 0, 333, 11, False, 13, 1000),
                                                                 (8, 2, 512, 0, 700, 16, True, 12, 2560),
                                                                 (8, 2, 512, 0, 1023, 16, False, 13, 2560),
                                                                 (8, 2, 512, 0, 5, 3, True, 12, 300)])
def test_attn_merge_o_prologue(lib, orc, nh, nkv, hd, window, pos, G, store, qtype, d):
    """The attention's end and the output projection in one launch
    (main.c:1909-1950 then the O mm, main.c:1955): g4_attn_decode_fused leaves
    only the chunk partials, g4_mm_attn_merge merges them per head in every
    workgroup and runs the Q4_K/Q5_K GEMV on their Q8_K (head_dim 256: one
    Q8_K block per head; 512, the global layers': two).  The merged vector is
    within 1e-4 of the oracle's attention and bit-equal to the separate merge
    kernel's, its Q8_K is quantize_row_q8_K of it, and the outputs equal the
    oracle's mm_quant_dot_rows on that Q8_K bit for bit."""
    from g4 import upload_quant
    eps = 1e-6
    rng = np.random.default_rng(nh + pos + G + qtype)
    kv_dim, n = nkv * hd, nh * hd
    base = 1e4 if window else 1e6
    q_norm = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    k_norm = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    flat_k = rng.standard_normal((pos + 1, kv_dim)).astype(np.float32)
    flat_v = rng.standard_normal((pos + 1, kv_dim)).astype(np.float32)
    q = rng.standard_normal(n).astype(np.float32)
    k = rng.standard_normal(kv_dim).astype(np.float32)
    v = rng.standard_normal(kv_dim).astype(np.float32)
    qn = q.copy()
    orc.L.or_rmsnorm_head_inplace(P(qn), P(q_norm), nh, hd, C.c_float(eps))
    qn = orc.rope(qn, nh, hd, hd, pos, base, None)
    if store:
        kk = k.copy()
        orc.L.or_rmsnorm_head_inplace(P(kk), P(k_norm), nkv, hd, C.c_float(eps))
        flat_k[pos] = orc.rope(kk, nkv, hd, hd, pos, base, None)
        vv = v.copy()
        orc.L.or_rmsnorm_head_noweight_inplace(P(vv), nkv, hd, C.c_float(eps))
        flat_v[pos] = vv
    t_start = max(0, pos + 1 - window) if window else 0
    want = orc.attn(qn, flat_k, flat_v, kv_dim, t_start, pos + 1 - t_start, nh, nkv, hd, 1.0)
    slots = window if window else pos + 1
    cache_k = np.full((slots, kv_dim), 7.0, np.float32)
    cache_v = np.full((slots, kv_dim), -7.0, np.float32)
    for t in range(t_start, pos + (0 if store else 1)):
        cache_k[t % slots], cache_v[t % slots] = flat_k[t], flat_v[t]
    kc, vc = dbuf(lib, cache_k), dbuf(lib, cache_v)
    dpos = dbuf(lib, np.array([pos], np.int32))
    tab = empty(lib, 4 * hd)
    lib.g4_rope_table(tab.ptr, dpos.ptr, 0, hd, C.c_float(base), C.c_float(1.0), None)
    qd, kd, vd = dbuf(lib, q), dbuf(lib, k), dbuf(lib, v)
    qnd, knd = dbuf(lib, q_norm), dbuf(lib, k_norm)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    part = empty(lib, lib.L.g4_attn_part_bytes(nh, hd, G))

    def attn(out, q8):
        lib.g4_attn_decode_fused(qd.ptr, qnd.ptr, kd.ptr if store else None, vd.ptr if store else None,
                                 knd.ptr if store else None, kc.ptr if store else None, vc.ptr if store else None,
                                 kc.ptr, vc.ptr, kv_dim, window, dpos.ptr, window, nh, nkv, hd, hd, tab.ptr,
                                 C.c_float(eps), C.c_float(1.0), G, part.ptr, out, q8)

    # the separate merge kernel, then the plain GEMV on its Q8_K
    o_sep, q8_sep, y_sep = empty(lib, 4 * n), empty(lib, lib.L.g4_q8K_bytes(n)), empty(lib, 4 * d)
    attn(o_sep.ptr, q8_sep.ptr)
    lib.g4_mm_quant_dot_rows(y_sep.ptr, w.ptr, n, d, qtype, q8_sep.ptr)
    # partials only (the append is repeated with the same row), merged in the GEMV
    o_m, q8_m, y_m = empty(lib, 4 * n), empty(lib, lib.L.g4_q8K_bytes(n)), empty(lib, 4 * d)
    attn(None, None)
    lib.g4_mm_attn_merge(y_m.ptr, w.ptr, n, d, qtype, part.ptr, G, nh, hd, o_m.ptr, q8_m.ptr)
    got = o_m.to_array(np.float32)
    assert rel_err(got, want) < 1e-4
    assert np.array_equal(got.view(np.uint32), o_sep.to_array(np.float32).view(np.uint32))
    h = np.zeros(n // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8_m.ptr, P(h), n)
    assert h.tobytes() == orc.quantize_q8K(got).tobytes()
    y = y_m.to_array(np.float32)
    assert np.array_equal(y.view(np.uint32), orc.mm_quant_dot_rows(raw, n, d, qtype, h).view(np.uint32))
    assert np.array_equal(y.view(np.uint32), y_sep.to_array(np.float32).view(np.uint32))
    # without the optional stores the outputs are the same
    y2 = empty(lib, 4 * d)
    lib.g4_mm_attn_merge(y2.ptr, w.ptr, n, d, qtype, part.ptr, G, nh, hd, None, None)
    assert np.array_equal(y2.to_array(np.float32).view(np.uint32), y.view(np.uint32))


def test_attn_merge_o_prologue_rejects(lib):
    from g4 import DBuf, G4Error
    b = DBuf(lib, 1 << 20)
    for args in [(b.ptr, b.ptr, 2048, 2560, 12, b.ptr, 17, 8, 256, None, None),    # too many chunks
                 (b.ptr, b.ptr, 2048, 2560, 12, b.ptr, 8, 16, 128, None, None),    # head_dim 128
                 (b.ptr, b.ptr, 6144, 2560, 12, b.ptr, 8, 12, 512, None, None),    # 12 heads of 512
                 (b.ptr, b.ptr, 3072, 2560, 12, b.ptr, 8, 12, 256, None, None),    # 12 heads
                 (b.ptr, b.ptr, 2048, 2560, 14, b.ptr, 8, 8, 256, None, None)]:    # Q6_K
        with pytest.raises(G4Error):
            lib.g4_mm_attn_merge(*args)


# ---------------------------------------------------------------------------
# embedding lookup, PLE, GELU gate, argmax
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_emb_lookup_bitexact(lib, orc, qtype):
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(qtype)
    rows, dim = 300, 2560
    raw = synth.rand_kquant(rng, qtype, rows, dim)
    w = upload_quant(lib, raw, qtype, dim, rows)
    out = DBuf(lib, 4 * dim)
    for tok in (0, 17, 299):
        lib.g4_emb_lookup(out.ptr, w.ptr, qtype, rows, tok, dim)
        want = np.empty(dim, np.float32)
        assert orc.L.or_emb_lookup(P(want), P(raw), qtype, tok, dim) == 0
        assert np.array_equal(out.to_array(np.float32).view(np.uint32), want.view(np.uint32))
    assert lib.L.g4_emb_lookup(out.ptr, w.ptr, qtype, rows, rows, dim) == 1   # G4_ERR_ARG, id out of range



@pytest.mark.parametrize("qtype,pos", [(14, 0), (12, 519), (14, 32767)])
def test_emb_lookup_rope(lib, orc, qtype, pos):
    """The decode step's inputs in one launch: the embedding row times its
    scale, bit-exact against the oracle's emb_lookup, and both RoPE tables
    (sliding: n_rot 256, base 1e4; full: n_rot 512, base 1e6 with freq
    factors) equal, bit for bit, to g4_rope_table's at the same position."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(qtype + pos)
    rows, dim, tok, scale = 300, 2560, 123, np.float32(np.sqrt(2560.0))
    raw = synth.rand_kquant(rng, qtype, rows, dim)
    w = upload_quant(lib, raw, qtype, dim, rows)
    ff = rng.uniform(1.0, 4.0, 256).astype(np.float32)
    ffd = dbuf(lib, ff)
    dtok, dpos = dbuf(lib, np.array([tok], np.int32)), dbuf(lib, np.array([pos], np.int32))
    out, ta, tb = DBuf(lib, 4 * dim), DBuf(lib, 4 * 256), DBuf(lib, 4 * 512)
    lib.g4_emb_lookup_rope(out.ptr, w.ptr, qtype, rows, dtok.ptr, dim, C.c_float(scale), dpos.ptr, ta.ptr, 256,
                           C.c_float(1e4), None, tb.ptr, 512, C.c_float(1e6), ffd.ptr, C.c_float(1.0))
    want = np.empty(dim, np.float32)
    assert orc.L.or_emb_lookup(P(want), P(raw), qtype, tok, dim) == 0
    assert np.array_equal(out.to_array(np.float32).view(np.uint32), (want * scale).view(np.uint32))
    ra, rb = DBuf(lib, 4 * 256), DBuf(lib, 4 * 512)
    lib.g4_rope_table(ra.ptr, dpos.ptr, 0, 256, C.c_float(1e4), C.c_float(1.0), None)
    lib.g4_rope_table(rb.ptr, dpos.ptr, 0, 512, C.c_float(1e6), C.c_float(1.0), ffd.ptr)
    assert np.array_equal(ta.to_array(np.float32).view(np.uint32), ra.to_array(np.float32).view(np.uint32))
    assert np.array_equal(tb.to_array(np.float32).view(np.uint32), rb.to_array(np.float32).view(np.uint32))
    if pos == 0:   # angle 0: (1, 0) pairs
        assert np.array_equal(ta.to_array(np.float32).reshape(-1, 2), np.tile([1.0, 0.0], (128, 1)).astype(np.float32))

@pytest.mark.parametrize("qtype,pos,d_ctx", [(14, 519, 10752), (12, 0, 1000), (14, 32767, 8)])
def test_emb_lookup_rope_ple(lib, orc, qtype, pos, d_ctx):
    """The step's inputs with the bf16 PLE context projection in the same
    launch: x, both RoPE tables and ctx equal, bit for bit, to
    g4_emb_lookup_rope followed by g4_mm_bf16 on its x; x against the
    oracle's emb_lookup and ctx within 1e-5 of the oracle's mm_bf16
    (normalised by sum |w x|).  d_ctx 10752 is E4B's 42 x 256."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(qtype + pos + d_ctx)
    rows, dim, tok, scale = 300, 2560, 123, np.float32(np.sqrt(2560.0))
    raw = synth.rand_kquant(rng, qtype, rows, dim)
    w = upload_quant(lib, raw, qtype, dim, rows)
    wc_raw = synth.rand_bf16(rng, d_ctx, dim)
    wc = dbuf(lib, wc_raw)
    ff = rng.uniform(1.0, 4.0, 256).astype(np.float32)
    ffd = dbuf(lib, ff)
    dtok, dpos = dbuf(lib, np.array([tok], np.int32)), dbuf(lib, np.array([pos], np.int32))
    out, ta, tb, ctx = DBuf(lib, 4 * dim), DBuf(lib, 4 * 256), DBuf(lib, 4 * 512), DBuf(lib, 4 * d_ctx)
    seq = dbuf(lib, np.array([41], np.uint32))
    lib.g4_emb_lookup_rope_ple(out.ptr, w.ptr, qtype, rows, dtok.ptr, dim, C.c_float(scale), dpos.ptr, ta.ptr, 256,
                               C.c_float(1e4), None, tb.ptr, 512, C.c_float(1e6), ffd.ptr, C.c_float(1.0), ctx.ptr,
                               wc.ptr, d_ctx, seq.ptr)
    out2, ta2, tb2, ctx2 = DBuf(lib, 4 * dim), DBuf(lib, 4 * 256), DBuf(lib, 4 * 512), DBuf(lib, 4 * d_ctx)
    lib.g4_emb_lookup_rope(out2.ptr, w.ptr, qtype, rows, dtok.ptr, dim, C.c_float(scale), dpos.ptr, ta2.ptr, 256,
                           C.c_float(1e4), None, tb2.ptr, 512, C.c_float(1e6), ffd.ptr, C.c_float(1.0))
    lib.g4_mm_bf16(ctx2.ptr, out2.ptr, wc.ptr, dim, d_ctx)
    for a, b in ((out, out2), (ta, ta2), (tb, tb2), (ctx, ctx2)):
        assert np.array_equal(a.to_array(np.uint32), b.to_array(np.uint32))
    assert seq.to_array(np.uint32)[0] == 42   # advanced once
    want = np.empty(dim, np.float32)
    assert orc.L.or_emb_lookup(P(want), P(raw), qtype, tok, dim) == 0
    x = want * scale
    assert np.array_equal(out.to_array(np.float32).view(np.uint32), x.view(np.uint32))
    Wf = (wc_raw.astype(np.uint32) << 16).view(np.float32).reshape(d_ctx, dim).astype(np.float64)
    want_c = Wf @ x.astype(np.float64)
    mag = np.abs(Wf) @ np.abs(x.astype(np.float64))
    assert np.max(np.abs(ctx.to_array(np.float32) - want_c) / mag) < 1e-5


def test_ple_finish(lib, orc):
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(5)
    L, pd, vocab, dim = 42, 256, 64, 2560
    raw = synth.rand_q6K(rng, vocab, pd * L)
    ctx = (rng.standard_normal(pd * L) * 20).astype(np.float32)
    norm = rng.uniform(0.8, 1.2, pd).astype(np.float32)
    tok = 37
    w = upload_quant(lib, raw, 14, pd * L, vocab)
    ctxd, nd = dbuf(lib, ctx), dbuf(lib, norm)
    out = DBuf(lib, 4 * pd * L)
    st, sc, mix = np.float32(np.sqrt(np.float32(pd))), np.float32(1) / np.sqrt(np.float32(dim)), np.float32(1) / np.sqrt(np.float32(2))
    lib.g4_ple_finish(out.ptr, ctxd.ptr, w.ptr, 14, vocab, nd.ptr, None, tok, pd, L, C.c_float(st), C.c_float(sc),
                      C.c_float(mix), C.c_float(1e-6))
    # oracle composition of build_ple (main.c:1751-1777)
    row = np.empty(pd * L, np.float32)
    orc.L.or_emb_lookup(P(row), P(raw), 14, tok, pd * L)
    row = row * st
    c = ctx * sc
    want = np.empty_like(c)
    for l in range(L):
        want[l * pd:(l + 1) * pd] = orc.rmsnorm(c[l * pd:(l + 1) * pd], norm)
    want = (row + want) * mix
    assert rel_err(out.to_array(np.float32), want) < 2e-6


def test_gelu_mul_quant(lib, orc):
    rng = np.random.default_rng(8)
    g = (rng.standard_normal(256) * 3).astype(np.float32)
    ple = rng.standard_normal(256).astype(np.float32)
    want = np.array([orc.L.or_gelu(float(v)) for v in g], np.float32) * ple
    gd, pd_, q8 = dbuf(lib, g), dbuf(lib, ple), empty(lib, 292)
    lib.g4_gelu_mul_quant(gd.ptr, pd_.ptr, 256, q8.ptr)
    got = gd.to_array(np.float32)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-7)   # tanhf: device libm vs glibc
    h = np.zeros(1, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), 256)
    assert h.tobytes() == orc.quantize_q8K(got).tobytes()


def test_argmax_first_index(lib):
    rng = np.random.default_rng(12)
    n = 262144
    part = empty(lib, lib.L.g4_argmax_part_bytes(n))
    out = empty(lib, 4)
    for case in range(4):
        v = rng.standard_normal(n).astype(np.float32)
        if case == 1:
            v[[100, 5000, 260000]] = 9.0            # tie: first index wins
        if case == 2:
            v[:] = -1.0
            v[77777] = -0.0
            v[99999] = 0.0                           # -0 == +0: first wins
        if case == 3:
            v[:] = -np.inf
            v[n - 1] = -1e30
        vd = dbuf(lib, v)
        lib.g4_argmax(vd.ptr, n, out.ptr, part.ptr, None, None)
        got = int(out.to_array(np.int32)[0])
        best = 0
        m = v[0]
        for i in np.flatnonzero(v == v.max()):
            best = int(i)
            break
        assert got == best, (case, got, best, m)


def test_argmax_nan(lib, orc):
    """NaN logits, against the reference's scan (main.c:2046-2048) as the
    oracle's first-index argmax: a NaN after index 0 never wins; a NaN at
    index 0 is never left (every comparison with it is false)."""
    rng = np.random.default_rng(13)
    n = 262144
    part = empty(lib, lib.L.g4_argmax_part_bytes(n))
    out = empty(lib, 4)
    for case in range(3):
        v = rng.standard_normal(n).astype(np.float32)
        if case == 0:
            v[[5, 4096, 200000]] = np.nan
        if case == 1:
            v[int(np.argmax(v)) + 1:int(np.argmax(v)) + 3] = np.nan
        if case == 2:
            v[0] = np.nan
        vd = dbuf(lib, v)
        lib.g4_argmax(vd.ptr, n, out.ptr, part.ptr, None, None)
        vc = v.copy()
        want = orc.L.or_argmax_first(vc.ctypes.data, n)
        assert int(out.to_array(np.int32)[0]) == want, case


def test_residual_norm(lib, orc):
    rng = np.random.default_rng(13)
    n = 2560
    x = rng.standard_normal(n).astype(np.float32)
    y = (rng.standard_normal(n) * 4).astype(np.float32)
    wp = rng.uniform(0.5, 1.5, n).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, n).astype(np.float32)
    osc = np.array([0.9], np.float32)
    xd, yd, wpd, wnd, od = dbuf(lib, x), dbuf(lib, y), dbuf(lib, wp), dbuf(lib, wn), dbuf(lib, osc)
    xb2 = empty(lib, 4 * n)
    q8 = empty(lib, lib.L.g4_q8K_bytes(n))
    lib.g4_residual_norm(xd.ptr, yd.ptr, wpd.ptr, od.ptr, wnd.ptr, xb2.ptr, q8.ptr, 0, n, C.c_float(1e-6))
    want_x = (x + orc.rmsnorm(y, wp)) * osc[0]
    want_xb2 = orc.rmsnorm(want_x, wn)
    gx, gxb2 = xd.to_array(np.float32), xb2.to_array(np.float32)
    assert rel_err(gx, want_x) < 2e-6
    assert rel_err(gxb2, want_xb2) < 4e-6
    h = np.zeros(n // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), n)
    assert h.tobytes() == orc.quantize_q8K(gxb2).tobytes()
    # qsrc = 1: Q8_K of x itself, no y
    xd2 = dbuf(lib, x)
    lib.g4_residual_norm(xd2.ptr, None, None, None, None, None, q8.ptr, 1, n, C.c_float(1e-6))
    lib.g4_download_q8K(q8.ptr, P(h), n)
    assert h.tobytes() == orc.quantize_q8K(x).tobytes()
