"""GPU parity of the batched prefill GEMMs: g4_mm_batch_q8 (Q4_K / Q5_K on
Q8_K rows), g4_split_rows_f16 + g4_mm_batch_split (Q6_K) and g4_mm_batch.

The reference has no batched path; its prefill is forward() per token
(main.c:2366-2384), i.e. quantize_row_q8_K + mm_quant_dot_rows per token for
Q4_K / Q5_K, mm_quant_rows / mm_bf16 on the fp32 activations for Q6_K / bf16.
The batched kernels compute the same sums from the same integer codes and
scales on the matrix cores; the fp32 rounding of the partial sums is the only
difference, so the bar is the GEMVs' one: 1e-5 of sum |terms| against the
oracle, for every token of the small shapes and sampled tokens of the large
ones (the 511-token E4B shapes included).  A token's outputs must not depend
on the other tokens of the batch or its place in it (bit for bit), which is
what makes a prompt's result independent of its chunking.
"""
import numpy as np
import pytest

import kquant_np as kq
import synth
from oracle import Q8K_DTYPE

pytestmark = pytest.mark.gpu

P = lambda a: a.ctypes.data  # noqa: E731
TOL = 1e-5


@pytest.fixture(scope="module")
def lib():
    from g4 import Lib
    L = Lib.get()
    L.init(0)
    return L


def _acts(rng, m, n):
    x = rng.standard_normal((m, n)).astype(np.float32)
    x[m // 2] = 0.0                      # an all-zero token: Q8_K d = 0, split scale 1
    if m > 3:
        x[1] *= 1e3
        x[2, :256] = 0.0                 # one all-zero block inside a token
    if m > 4:
        x[3] *= 1e-6                     # small activations (the split scales them up)
    return x


def _q8rows(lib, xd, n, m):
    from g4 import DBuf
    qb = lib.L.g4_q8K_row_stride(n)
    q8 = DBuf(lib, qb * m)
    lib.g4_quantize_rows_q8_K(xd.ptr, q8.ptr, n, m)
    return q8, qb


def _mm_q8(lib, w, q8ptr, n, d, m, qtype):
    from g4 import DBuf
    out = DBuf(lib, 4 * m * d)
    lib.g4_mm_batch_q8(out.ptr, w.ptr, q8ptr, n, d, m, qtype)
    return out.to_array(np.float32).reshape(m, d)


def test_quantize_rows_equals_per_row(lib, orc):
    from g4 import DBuf
    rng = np.random.default_rng(5)
    m, n = 7, 2560
    x = _acts(rng, m, n)
    xd = DBuf.from_array(lib, x)
    q8, qb = _q8rows(lib, xd, n, m)
    for t in range(m):
        got = np.zeros(n // 256, Q8K_DTYPE)
        lib.g4_download_q8K(q8.ptr + t * qb, P(got), n)
        assert got.tobytes() == orc.quantize_q8K(x[t]).tobytes(), t


SHAPES = [(256, 80, 37), (2560, 70, 17), (2560, 2048, 64), (2048, 2560, 100), (10240, 192, 65), (2560, 10240, 130)]


def _check_q8(orc, raw, qtype, n, d, x, got, toks):
    q8s = np.stack([orc.quantize_q8K(x[t]) for t in toks])
    mag = kq.abs_terms_q8(raw, qtype, n, q8s)           # [d, len(toks)]
    for z, t in enumerate(toks):
        want = orc.mm_quant_dot_rows(raw, n, d, qtype, q8s[z])
        err = np.abs(got[t].astype(np.float64) - want)
        bad = np.flatnonzero(err > TOL * mag[:, z] + 1e-30)
        assert bad.size == 0, f"token {t}: {bad.size} rows, first {bad[:4]}: {got[t][bad[:4]]} vs {want[bad[:4]]}"


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n,d,m", SHAPES)
def test_mm_batch_q8_vs_oracle(lib, orc, qtype, n, d, m):
    """Every token (every 8th on the two largest shapes) against the
    oracle's mm_quant_dot_rows on its Q8_K row; the same token rows in a
    batch shifted by 5 tokens give the same bits."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(100 * qtype + n + d + m)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = _acts(rng, m + 5, n)
    xd = DBuf.from_array(lib, x)
    q8, qb = _q8rows(lib, xd, n, m + 5)
    got = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    got2 = _mm_q8(lib, w, q8.ptr + 5 * qb, n, d, m, qtype)
    assert np.array_equal(got[5:].view(np.uint32), got2[:m - 5].view(np.uint32))
    toks = range(m) if d * m <= 200_000 else sorted(set(range(0, m, 8)) | {1, 2, 3, m - 1})
    _check_q8(orc, raw, qtype, n, d, x, got, list(toks))


@pytest.mark.parametrize("qtype", [12, 13])
def test_mm_batch_q8_prefill_shape(lib, orc, qtype):
    """The benchmarked shape: gate/up 10240 x 2560 over a 511-token chunk,
    sampled tokens against the oracle."""
    from g4 import DBuf, upload_quant
    n, d, m = 2560, 10240, 511
    rng = np.random.default_rng(31 + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = _acts(rng, m, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    got = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    _check_q8(orc, raw, qtype, n, d, x, got, [0, 1, 2, 3, 63, 64, 255, 256, 509, 510])


@pytest.mark.parametrize("qtype", [12, 13])
def test_mm_batch_q8_every_token(lib, orc, qtype):
    """Every token of the benchmarked gate/up shape (10240 x 2560, 511 tokens)
    within 1e-5 of sum |terms| of the exact float64 product of the dequantized
    weights with each token's Q8_K row (the sampled-token checks above would
    miss an error confined to a few tokens of a tile)."""
    from g4 import DBuf, upload_quant
    n, d, m = 2560, 10240, 511
    rng = np.random.default_rng(61 + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = _acts(rng, m, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    got = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    q8s = np.stack([orc.quantize_q8K(x[t]) for t in range(m)])
    W = kq.dequant_f64(raw.reshape(-1, {12: 144, 13: 176}[qtype]), qtype).reshape(d, n)
    X = (q8s["qs"].astype(np.float64) * q8s["d"].astype(np.float64)[..., None]).reshape(m, n)
    want = X @ W.T
    mag = kq.abs_terms_q8(raw, qtype, n, q8s).T
    bad = np.argwhere(np.abs(got - want) > TOL * mag + 1e-30)
    assert bad.size == 0, f"{len(bad)} outputs, first (token, row) {bad[:6].tolist()}"


@pytest.mark.parametrize("qtype", [12, 13])
def test_mm_batch_q8_wave_shapes(lib, orc, qtype):
    """A 2560-row matrix at 511 tokens takes 160-row (five-wave) workgroups,
    at 37 tokens 128-row ones: a token's outputs are the same bits either way,
    and sampled tokens of the five-wave launch are within the bar of the
    oracle."""
    from g4 import DBuf, upload_quant
    n, d = 2048, 2560
    rng = np.random.default_rng(71 + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = _acts(rng, 511, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, 511)
    full = _mm_q8(lib, w, q8.ptr, n, d, 511, qtype)
    part = _mm_q8(lib, w, q8.ptr, n, d, 37, qtype)
    assert np.array_equal(full[:37].view(np.uint32), part.view(np.uint32))
    _check_q8(orc, raw, qtype, n, d, x, full, [0, 1, 2, 3, 159, 160, 255, 256, 479, 510])


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("d,m", [(256, 511), (256, 37), (512, 5)])
def test_mm_batch_q8_blocks_fold(lib, qtype, d, m):
    """The PLE gate split by K block (main.c:1988-1993): folding the per-block
    terms in block order gives g4_mm_batch_q8's output bit for bit; with the
    PLE rows, gelu * ple equals g4_gelu_mul_rows on that output and the Q8_K
    rows equal g4_quantize_rows_q8_K's, bit for bit."""
    from g4 import DBuf, G4Error, upload_quant
    n = 2560
    rng = np.random.default_rng(81 + qtype + d + m)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = _acts(rng, m, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    want = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    u = DBuf(lib, 4 * (n // 256) * m * d)
    lib.g4_mm_batch_q8_blocks(u.ptr, w.ptr, q8.ptr, n, d, m, qtype)
    out = DBuf(lib, 4 * m * d)
    lib.g4_fold_gelu_mul_q8(u.ptr, q8.ptr, n, None, 0, out.ptr, None, d, m)
    assert np.array_equal(out.to_array(np.float32).reshape(m, d).view(np.uint32), want.view(np.uint32))
    pstride = d + 64
    ple = DBuf.from_array(lib, rng.standard_normal((m, pstride)).astype(np.float32))
    rs = lib.L.g4_q8K_row_stride(d)
    q8o = DBuf(lib, rs * m)
    lib.g4_fold_gelu_mul_q8(u.ptr, q8.ptr, n, ple.ptr, pstride, out.ptr, q8o.ptr, d, m)
    wd = DBuf.from_array(lib, want)
    ref = DBuf(lib, 4 * m * d)
    lib.g4_gelu_mul_rows(ref.ptr, wd.ptr, ple.ptr, d, m, pstride)
    assert np.array_equal(out.to_array(np.uint32), ref.to_array(np.uint32))
    q8r = DBuf(lib, rs * m)
    lib.g4_quantize_rows_q8_K(ref.ptr, q8r.ptr, d, m)
    used = 292 * (d // 256)   # a Q8_K row's bytes before its padding (qs, bsums, d)
    assert np.array_equal(q8o.to_array(np.uint8).reshape(m, rs)[:, :used], q8r.to_array(np.uint8).reshape(m, rs)[:, :used])
    with pytest.raises(G4Error):
        lib.g4_fold_gelu_mul_q8(u.ptr, q8.ptr, n, None, 0, out.ptr, None, 2048, m)


@pytest.mark.parametrize("qtype", [12, 13])
def test_mm_batch_q8_multi(lib, orc, qtype):
    """Three matrices of one type over the same Q8_K rows in one launch (the
    engine's Q|K and gate|up): each output equals the single-matrix launch
    bit for bit, and sampled tokens are within the bar of the oracle."""
    import ctypes as C
    from g4 import DBuf, G4Error, upload_quant
    n, m = 2560, 77
    ds = (2048, 512, 200)
    rng = np.random.default_rng(41 + qtype)
    raws = [synth.rand_kquant(rng, qtype, d, n) for d in ds]
    ws = [upload_quant(lib, r, qtype, n, d) for r, d in zip(raws, ds)]
    x = _acts(rng, m, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    outs = [DBuf(lib, 4 * m * d) for d in ds]
    O = (C.c_void_p * 3)(*[o.ptr for o in outs])
    W = (C.c_void_p * 3)(*[w.ptr for w in ws])
    D = (C.c_int * 3)(*ds)
    lib.g4_mm_batch_q8_multi(O, W, D, 3, q8.ptr, n, m, qtype)
    for k, d in enumerate(ds):
        got = outs[k].to_array(np.float32).reshape(m, d)
        one = _mm_q8(lib, ws[k], q8.ptr, n, d, m, qtype)
        assert np.array_equal(got.view(np.uint32), one.view(np.uint32)), k
        _check_q8(orc, raws[k], qtype, n, d, x, got, [0, 3, m - 1])
    with pytest.raises(G4Error):
        lib.g4_mm_batch_q8_multi(O, W, D, 5, q8.ptr, n, m, qtype)
    with pytest.raises(G4Error):
        lib.g4_mm_batch_q8_multi(O, W, D, 0, q8.ptr, n, m, qtype)


# ---- Q6_K over split activations ----------------------------------------

def _split_pos(e):
    """element (0..255) of a block -> its half index in the split layout"""
    h, k, s, half = e >> 7, (e >> 5) & 3, (e >> 4) & 1, (e >> 3) & 1
    return (((2 * k + half) * 4 + 2 * h + s) << 3) | (e & 7)


def _unsplit(raw, n, m):
    """split bytes -> (hi, lo) as float64 [m, n] in element order, scales [m]"""
    rows = np.frombuffer(raw[:m * n * 4].tobytes(), np.float16).reshape(m, n // 256, 2, 256)
    perm = np.array([_split_pos(e) for e in range(256)])
    hi = rows[:, :, 0, perm].reshape(m, n).astype(np.float64)
    lo = rows[:, :, 1, perm].reshape(m, n).astype(np.float64)
    sc = np.frombuffer(raw[m * n * 4:m * n * 4 + 4 * m].tobytes(), np.float32)
    return hi, lo, sc


def test_split_rows(lib):
    """hi + lo reproduce x * 2^-s to 2^-22 of each |x 2^-s| (2^-25 absolute in
    fp16's subnormal range); 2^s is a power of two that brings the row's
    largest |x| into [2^14, 2^15); an all-zero row has factor 1."""
    from g4 import DBuf
    rng = np.random.default_rng(11)
    m, n = 9, 2560
    x = _acts(rng, m, n)
    x[5] *= 3e4                         # above fp16's range before scaling
    x[6, ::7] = 1e-9                    # tiny elements beside normal ones
    x[7] *= 1e-6
    x[7, 7] = 50.0                      # one large element among small ones
    xd = DBuf.from_array(lib, x)
    nbytes = lib.L.g4_split_rows_bytes(n, m)
    assert nbytes == m * n * 4 + 4 * m
    xs = DBuf(lib, nbytes)
    lib.g4_split_rows_f16(xd.ptr, xs.ptr, n, m)
    hi, lo, sc = _unsplit(xs.to_array(np.uint8), n, m)
    for t in range(m):
        mx = np.abs(x[t]).max()
        if mx == 0:
            assert sc[t] == 1.0 and not hi[t].any() and not lo[t].any()
            continue
        e = np.frexp(sc[t])
        assert e[0] == 0.5, sc[t]                           # a power of two
        xsd = x[t].astype(np.float64) / float(sc[t])
        assert 2.0 ** 14 <= np.abs(xsd).max() < 2.0 ** 15, (t, np.abs(xsd).max())
        err = np.abs(xsd - hi[t] - lo[t])
        assert (err <= 2.0 ** -22 * np.abs(xsd) + 2.0 ** -25).all(), (t, err.max())
        assert (np.abs(hi[t]) <= 2.0 ** 15).all()


@pytest.mark.parametrize("n,m,ustride", [(10240, 37, 10240), (2048, 5, 2100), (4096, 1, 4096), (10240, 511, 10240)])
def test_gelu_mul_split_rows(lib, n, m, ustride):
    """gelu(g) * u split in one launch: byte for byte g4_gelu_mul_rows followed
    by g4_split_rows_f16, with an all-zero row, a row far above fp16's range,
    tiny rows and u rows wider than g's; unsupported widths are refused."""
    from g4 import DBuf, G4Error
    rng = np.random.default_rng(n + m)
    g = (rng.standard_normal((m, n)) * 2).astype(np.float32)
    u = rng.standard_normal((m, ustride)).astype(np.float32)
    if m > 3:
        g[1] = 0.0
        u[2] *= 1e5
        g[3] *= 1e-4
    gd, ud = DBuf.from_array(lib, g), DBuf.from_array(lib, u)
    nbytes = lib.L.g4_split_rows_bytes(n, m)
    got, h, want = DBuf(lib, nbytes), DBuf(lib, 4 * m * n), DBuf(lib, nbytes)
    lib.g4_gelu_mul_split_rows(gd.ptr, ud.ptr, ustride, got.ptr, n, m)
    lib.g4_gelu_mul_rows(h.ptr, gd.ptr, ud.ptr, n, m, ustride)
    lib.g4_split_rows_f16(h.ptr, want.ptr, n, m)
    assert np.array_equal(got.to_array(np.uint8), want.to_array(np.uint8))
    with pytest.raises(G4Error):
        lib.g4_gelu_mul_split_rows(gd.ptr, ud.ptr, ustride, got.ptr, 2560, m)


def _mag_f32(raw, qtype, n, d, x):
    """sum_j |w_ij x_j| per row, the scale of an fp32 dot's rounding"""
    if qtype == 30:
        W = (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(d, n)
        return np.abs(W) @ np.abs(x.astype(np.float64))
    return kq.abs_dot_rows(raw, 14, n, x)


F32W_SHAPES = [(2560, 512, 511), (2560, 1024, 130), (10240, 2560, 37), (2560, 10752, 33), (256, 40, 5),
               (512, 256, 24), (2560, 96, 1), (10240, 2560, 511)]


def _split_mm(lib, w, xptr, n, d, m):
    from g4 import DBuf
    xs = DBuf(lib, lib.L.g4_split_rows_bytes(n, m))
    lib.g4_split_rows_f16(xptr, xs.ptr, n, m)
    out = DBuf(lib, 4 * m * d)
    lib.g4_mm_batch_split(out.ptr, w.ptr, xs.ptr, n, d, m, 14)
    return out.to_array(np.float32).reshape(m, d)


@pytest.mark.parametrize("n,d,m", F32W_SHAPES)
def test_mm_batch_split_q6k(lib, orc, n, d, m):
    """Q6_K (V, FFN down) over m tokens: sampled tokens within 1e-5 of
    sum |w x| of the oracle's mm_quant_rows (main.c:1539-1556); the same token
    rows in a batch shifted by 5 tokens give the same bits."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(7 * n + d + m)
    raw = synth.rand_q6K(rng, d, n)
    w = upload_quant(lib, raw, 14, n, d)
    x = _acts(rng, m + 5, n)
    xd = DBuf.from_array(lib, x)
    got = _split_mm(lib, w, xd.ptr, n, d, m)
    got2 = _split_mm(lib, w, xd.ptr + 4 * 5 * n, n, d, m)
    assert np.array_equal(got[5:].view(np.uint32), got2[:m - 5].view(np.uint32))
    for t in sorted({0, min(1, m - 1), min(3, m - 1), m // 2, m - 1}):
        want = orc.mm_quant_rows(x[t], raw, n, d, 14)
        mag = _mag_f32(raw, 14, n, d, x[t])
        err = np.abs(got[t].astype(np.float64) - want)
        assert (err <= TOL * mag + 1e-30).all(), (t, float((err / (mag + 1e-30)).max()))


@pytest.mark.parametrize("n,d", [(2560, 512), (10240, 2560)])
def test_mm_batch_split_every_token(lib, n, d):
    """Every token of a 511-token batch (V and FFN down at the E4B shape)
    within 1e-5 of sum |w x| of the exact float64 product.  Each wave of the
    kernel copies its tokens' activation rows straight into LDS one block
    ahead; a wait that let a wave's last copy still be in flight at the
    barrier corrupted the rows of one token in sixteen now and then (offsets
    12-15 of a tile), which sampled tokens did not catch."""
    from g4 import DBuf, upload_quant
    m = 511
    rng = np.random.default_rng(n + d + 9)
    raw = synth.rand_q6K(rng, d, n)
    w = upload_quant(lib, raw, 14, n, d)
    x = _acts(rng, m, n)
    got = _split_mm(lib, w, DBuf.from_array(lib, x).ptr, n, d, m)
    W = kq.dequant_f64(raw.reshape(-1, 210), 14).reshape(d, n)
    want = x.astype(np.float64) @ W.T
    mag = np.abs(x).astype(np.float64) @ np.abs(W).T
    err = np.abs(got - want)
    bad = np.argwhere(err > TOL * mag + 1e-30)
    assert bad.size == 0, f"{len(bad)} outputs, first (token, row) {bad[:6].tolist()}"


@pytest.mark.parametrize("d", [2560, 512])
def test_mm_batch_split_token_tiles(lib, d):
    """The launch takes 16- or 32-token workgroups by the grid's size (FFN
    down at 511 tokens 32, at 37 tokens 16; V 16 at both); a token's outputs
    are the same bits either way, so a prompt's result does not depend on its
    chunking."""
    from g4 import DBuf, upload_quant
    n = 10240 if d == 2560 else 2560
    rng = np.random.default_rng(d + 5)
    raw = synth.rand_q6K(rng, d, n)
    w = upload_quant(lib, raw, 14, n, d)
    xd = DBuf.from_array(lib, _acts(rng, 511, n))
    full = _split_mm(lib, w, xd.ptr, n, d, 511)
    part = _split_mm(lib, w, xd.ptr, n, d, 37)
    assert np.array_equal(full[:37].view(np.uint32), part.view(np.uint32))


@pytest.mark.parametrize("qtype", [14, 30])
@pytest.mark.parametrize("n,d,m", [(2560, 512, 130), (256, 40, 5), (2560, 96, 1), (512, 10752, 33)])
def test_mm_batch_f32_weights(lib, orc, qtype, n, d, m):
    """The workspace-free g4_mm_batch for Q6_K and bf16 (the PLE projection):
    fp32 matrix-core sums of the reference's dequantized weights, sampled
    tokens within 1e-5 of sum |w x| of mm_quant_rows / mm_bf16
    (main.c:1539-1556, 1529-1537), shift-invariant bit for bit."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(7 * n + d + m + qtype)
    raw = synth.rand_bf16(rng, d, n) if qtype == 30 else synth.rand_q6K(rng, d, n)
    w = DBuf.from_array(lib, raw) if qtype == 30 else upload_quant(lib, raw, 14, n, d)
    x = _acts(rng, m + 5, n)
    xd = DBuf.from_array(lib, x)
    out, out2 = DBuf(lib, 4 * m * d), DBuf(lib, 4 * m * d)
    lib.g4_mm_batch(out.ptr, xd.ptr, w.ptr, n, d, m, qtype, None)
    got = out.to_array(np.float32).reshape(m, d)
    lib.g4_mm_batch(out2.ptr, xd.ptr + 4 * 5 * n, w.ptr, n, d, m, qtype, None)
    got2 = out2.to_array(np.float32).reshape(m, d)
    assert np.array_equal(got[5:].view(np.uint32), got2[:m - 5].view(np.uint32))
    for t in sorted({0, min(1, m - 1), m // 2, m - 1}):
        want = orc.mm_bf16(x[t], raw, n, d) if qtype == 30 else orc.mm_quant_rows(x[t], raw, n, d, 14)
        mag = _mag_f32(raw, qtype, n, d, x[t])
        assert (np.abs(got[t].astype(np.float64) - want) <= TOL * mag + 1e-30).all(), t


def test_mm_batch_wrapper(lib, orc):
    """g4_mm_batch for every type against the oracle per token: Q4_K / Q5_K
    through Q8_K rows (1e-5 of sum |terms| of the Q8_K dot), Q6_K and bf16
    (1e-5 of sum |w x|)."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(9)
    n, d, m = 2560, 96, 9
    x = _acts(rng, m, n)
    xd = DBuf.from_array(lib, x)
    q8 = DBuf(lib, lib.L.g4_q8K_row_stride(n) * m)
    for qtype in (12, 13, 14, 30):
        raw = synth.rand_bf16(rng, d, n) if qtype == 30 else synth.rand_kquant(rng, qtype, d, n)
        w = upload_quant(lib, raw, qtype, n, d) if qtype != 30 else DBuf.from_array(lib, raw)
        out = DBuf(lib, 4 * m * d)
        lib.g4_mm_batch(out.ptr, xd.ptr, w.ptr, n, d, m, qtype, q8.ptr)
        got = out.to_array(np.float32).reshape(m, d)
        if qtype in (12, 13):
            _check_q8(orc, raw, qtype, n, d, x, got, list(range(m)))
            continue
        for t in range(m):
            want = orc.mm_bf16(x[t], raw, n, d) if qtype == 30 else orc.mm_quant_rows(x[t], raw, n, d, 14)
            mag = _mag_f32(raw, qtype, n, d, x[t])
            assert (np.abs(got[t].astype(np.float64) - want) <= TOL * mag + 1e-30).all(), (qtype, t)


def test_mm_batch_errors(lib):
    from g4 import DBuf, G4Error
    w = DBuf(lib, 4096)
    q8 = DBuf(lib, 4096)
    o = DBuf(lib, 4096)
    with pytest.raises(G4Error):
        lib.g4_mm_batch_q8(o.ptr, w.ptr, q8.ptr, 256, 4, 2, 14)    # Q6_K has no Q8_K batched path
    with pytest.raises(G4Error):
        lib.g4_mm_batch_q8(o.ptr, w.ptr, q8.ptr, 300, 4, 2, 12)    # n not a multiple of 256
    with pytest.raises(G4Error):
        lib.g4_mm_batch_q8(o.ptr + 4, w.ptr, q8.ptr, 256, 4, 2, 12)   # unaligned output
    with pytest.raises(G4Error):
        lib.g4_quantize_rows_q8_K(o.ptr, q8.ptr, 256, 0)
    with pytest.raises(G4Error):
        lib.g4_mm_batch_split(o.ptr, w.ptr, q8.ptr, 256, 4, 2, 12)   # Q4_K has no split path
    with pytest.raises(G4Error):
        lib.g4_split_rows_f16(o.ptr, q8.ptr, 300, 2)                # n not a multiple of 256
    assert lib.L.g4_split_rows_bytes(300, 2) == 0


def _image(lib, w, qtype, n, d):
    from g4 import DBuf
    img = DBuf(lib, lib.L.g4_kq_image_bytes(n, d))
    lib.g4_kq_image(img.ptr, w.ptr, n, d, qtype)
    return img


IMG_SHAPES = [(256, 80, 37), (2560, 70, 17), (2560, 2048, 64), (2048, 2560, 100), (10240, 192, 65), (2560, 10240, 130)]


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n,d,m", IMG_SHAPES)
def test_mm_batch_img_vs_q8(lib, orc, qtype, n, d, m):
    """The fp16-image GEMM gives g4_mm_batch_q8's outputs bit for bit (the
    block sums are exact integers at these sizes), in every tile shape,
    and each token against the oracle's mm_quant_dot_rows at the 1e-5 bar."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(300 * qtype + n + d + m)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    img = _image(lib, w, qtype, n, d)
    x = _acts(rng, m, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    ref = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    for nt, nwv in [(0, 0), (1, 2), (1, 4), (1, 8), (2, 4), (2, 8)]:
        out = DBuf(lib, 4 * m * d)
        lib.g4_mm_batch_img_tile(out.ptr, img.ptr, q8.ptr, n, d, m, qtype, nt, nwv)
        got = out.to_array(np.float32).reshape(m, d)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (nt, nwv)
    toks = range(m) if d * m <= 200_000 else sorted(set(range(0, m, 8)) | {1, 2, 3, m - 1})
    _check_q8(orc, raw, qtype, n, d, x, got, list(toks))


@pytest.mark.parametrize("qtype", [12, 13])
def test_mm_batch_img_multi_prefill_shape(lib, orc, qtype):
    """gate and up (10240 x 2560) over a 511-token chunk in one launch on
    their images: both equal g4_mm_batch_q8_multi's outputs bit for bit, and
    sampled tokens meet the oracle bar."""
    from g4 import DBuf, upload_quant
    import ctypes as C
    n, d, m = 2560, 10240, 511
    rng = np.random.default_rng(71 + qtype)
    raws = [synth.rand_kquant(rng, qtype, d, n) for _ in range(2)]
    ws = [upload_quant(lib, r, qtype, n, d) for r in raws]
    imgs = [_image(lib, w, qtype, n, d) for w in ws]
    x = _acts(rng, m, n)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    outs = [DBuf(lib, 4 * m * d) for _ in range(4)]
    VPA = C.c_void_p * 2
    dd = (C.c_int * 2)(d, d)
    lib.g4_mm_batch_q8_multi(VPA(outs[0].ptr, outs[1].ptr), VPA(ws[0].ptr, ws[1].ptr), dd, 2, q8.ptr, n, m, qtype)
    lib.g4_mm_batch_img_multi(VPA(outs[2].ptr, outs[3].ptr), VPA(imgs[0].ptr, imgs[1].ptr), dd, 2, q8.ptr, n, m, qtype)
    for k in range(2):
        ref = outs[k].to_array(np.float32).reshape(m, d)
        got = outs[2 + k].to_array(np.float32).reshape(m, d)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), k
        _check_q8(orc, raws[k], qtype, n, d, x, got, [0, 1, 2, 3, 64, 255, 256, 510])


def test_kq_image_args(lib):
    """Sizes and argument checks of the image entry points."""
    from g4 import DBuf
    assert lib.L.g4_kq_image_bytes(2560, 100) == 4 * 10 * (16384 + 1024)
    assert lib.L.g4_kq_image_bytes(100, 100) == 0
    buf = DBuf(lib, 4096)
    assert lib.L.g4_kq_image(buf.ptr, buf.ptr, 256, 1, 14) != 0       # Q6_K has no image
    assert lib.L.g4_mm_batch_img_tile(buf.ptr, buf.ptr, buf.ptr, 256, 1, 1, 12, 3, 4) != 0
    assert lib.L.g4_mm_batch_img_tile(buf.ptr, buf.ptr, buf.ptr, 256, 1, 1, 14, 1, 4) != 0   # no Q6_K image
    S = DBuf(lib, 64)
    assert lib.L.g4_debug_batch_block_sums(buf.ptr, 0, 256, 1, 1, 14, buf.ptr, S.ptr, S.ptr) != 0
    assert lib.L.g4_debug_batch_block_sums(buf.ptr, 0, 300, 1, 1, 12, buf.ptr, S.ptr, S.ptr) != 0


def _saturated(rng, qtype, d, n):
    """Q4_K / Q5_K rows whose blocks reach the largest integer sums: every
    6-bit scale and min 63 (all scale bytes 0xff), every code 15 (Q4_K) or 31
    (Q5_K); rows 0 .. d/2 - 1 saturated everywhere, the rest random with every
    third block saturated."""
    raw = synth.rand_kquant(rng, qtype, d, n)
    bs = synth.BLOCK_BYTES[qtype]
    blk = raw.reshape(d, n // 256, bs)
    sat = np.zeros((d, n // 256), bool)
    sat[: d // 2] = True
    sat[d // 2:, ::3] = True
    code_end = bs                                    # scales 4..16, then (Q5_K: qh 16..48) and qs
    blk[sat, 4:code_end] = 0xFF
    return raw, sat


@pytest.mark.parametrize("qtype", [12, 13])
def test_batch_block_sums_exact_saturated(lib, orc, qtype):
    """The batched GEMM's own per-block integer sums S_b and M_b (from the
    quantized tensor and from its fp16 image) equal the exact integers of
    vec_dot_q4_K_q8_K / q5_K (main.c:500-523, 556-590) for every (token,
    row, block), on blocks that reach |S_b| = 256 * 63 * 15 * 127 (Q4_K,
    3.1e7) or 256 * 63 * 31 * 127 (Q5_K, 6.3e7), past fp32's 2^24 exact
    range: constant-sign tokens (Q8_K codes all -127, or +127) against
    saturated scales and codes.  They also equal the per-token GEMV's
    g4_debug_block_sums, and the outputs meet the 1e-5 bar against the
    oracle; the image GEMM's outputs equal the quantized GEMM's bit for bit."""
    from g4 import DBuf, upload_quant
    n, d, m = 2560, 256, 40
    nb = n // 256
    rng = np.random.default_rng(91 + qtype)
    raw, sat = _saturated(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = rng.standard_normal((m, n)).astype(np.float32)
    x[0] = 1.0                                       # Q8_K codes all -127 (iscale = -127 / max)
    x[1] = 1.0
    x[1, ::256] = -1.0                               # the block maximum negative: the rest +127
    x[2] = np.abs(x[2])                              # one sign, varied codes
    x[3] = -np.abs(x[3]) * 7.0
    x[4, :1280] = 2.0                                # half constant, half random
    x[5] = 0.0                                       # d = 0 token
    q8, qb = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    q8s = np.stack([orc.quantize_q8K(x[t]) for t in range(m)])
    assert (q8s[0]["qs"] == -127).all() and (q8s[1]["qs"][:, 1:] == 127).all()
    bsz = synth.BLOCK_BYTES[qtype]
    eS = np.zeros((m, d, nb), np.int64)
    eM = np.zeros((m, d, nb), np.int64)
    for t in range(m):
        for r in range(d):
            eS[t, r], eM[t, r] = kq.kquant_block_sums(raw[r].reshape(-1, bsz), qtype, q8s[t])
    big = np.abs(eS) > (1 << 24)
    assert big.sum() > 1000 and np.abs(eS).max() >= (30_000_000 if qtype == 12 else 60_000_000)
    for image in (0, 1):   # 0: the int8 matrix-core kernel on w; 1: the fp16 image kernel
        src = _image(lib, w, qtype, n, d) if image else w
        S, M = DBuf(lib, 4 * m * d * nb), DBuf(lib, 4 * m * d * nb)
        lib.g4_debug_batch_block_sums(src.ptr, image, n, d, m, qtype, q8.ptr, S.ptr, M.ptr)
        gS = S.to_array(np.int32).reshape(m, d, nb)
        gM = M.to_array(np.int32).reshape(m, d, nb)
        bad = np.argwhere(gS != eS)
        assert bad.size == 0, f"image={image}: S_b differs at {len(bad)} (token, row, block), first {bad[:4].tolist()}"
        assert np.array_equal(gM, eM), f"image={image}: M_b differs"
    # the per-token decode GEMV's own sums are the same integers
    for t in (0, 1, 3, 9):
        S1, M1 = DBuf(lib, 4 * d * nb), DBuf(lib, 4 * d * nb)
        lib.g4_debug_block_sums(w.ptr, n, d, qtype, q8.ptr + t * qb, S1.ptr, M1.ptr)
        assert np.array_equal(S1.to_array(np.int32).reshape(d, nb), eS[t])
        assert np.array_equal(M1.to_array(np.int32).reshape(d, nb), eM[t])
    got = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    _check_q8(orc, raw, qtype, n, d, x, got, list(range(m)))
    img = _image(lib, w, qtype, n, d)
    for nt, nwv in [(0, 0), (1, 2), (1, 4), (2, 4)]:
        out = DBuf(lib, 4 * m * d)
        lib.g4_mm_batch_img_tile(out.ptr, img.ptr, q8.ptr, n, d, m, qtype, nt, nwv)
        assert np.array_equal(out.to_array(np.float32).reshape(m, d).view(np.uint32), got.view(np.uint32)), (nt, nwv)


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n,d,m", [(2560, 2048, 511), (2560, 10240, 511), (2560, 256, 511), (2048, 2560, 511),
                                   (2560, 2560, 1), (512, 100, 33), (256, 40, 5), (4096, 520, 64)])
def test_mm_batch_q8_int8_equals_fp16_image(lib, orc, qtype, n, d, m):
    """The quantized-tensor GEMM (int8 matrix cores: one v_mfma_i32_32x32x32_i8
    per sub-block, scales applied in int32) and the fp16 image GEMM (sc * q
    folded into fp16 operands, chained in exact pieces) form the same integer
    block sums and the same fold: the same bits at the E4B prompt shapes and
    ragged ones, and sampled tokens meet the 1e-5 bar against the oracle's
    per-token mm_quant_dot_rows."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(n + d + m + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = rng.standard_normal((m, n)).astype(np.float32)
    q8, _ = _q8rows(lib, DBuf.from_array(lib, x), n, m)
    got = _mm_q8(lib, w, q8.ptr, n, d, m, qtype)
    img = _image(lib, w, qtype, n, d)
    oi = DBuf(lib, 4 * m * d)
    lib.g4_mm_batch_img(oi.ptr, img.ptr, q8.ptr, n, d, m, qtype)
    gi = oi.to_array(np.float32).reshape(m, d)
    assert np.array_equal(gi.view(np.uint32), got.view(np.uint32)), np.argwhere(gi != got)[:8]
    _check_q8(orc, raw, qtype, n, d, x, got, sorted({0, m // 2, m - 1}))
