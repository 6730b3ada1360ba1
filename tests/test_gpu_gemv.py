"""GPU parity: Q8_K quantization, HBM layout, K-quant / BF16 GEMVs against the
CPU oracle (which is pinned bit-exact to the reference's own functions).

Bars: Q8_K bytes, per-block int32 sums, and the Q4_K/Q5_K fp32 outputs are
bit-exact; fp32-activation GEMVs are within 1e-5 of the result, normalised by
sum |w * x| (the reference sums sequentially, the GPU in a tree).
"""
import ctypes as C

import numpy as np
import pytest

import kquant_np as kq
import synth
from oracle import Q8K_DTYPE

pytestmark = pytest.mark.gpu

P = lambda a: a.ctypes.data  # noqa: E731


@pytest.fixture(scope="module")
def lib():
    from g4 import Lib
    L = Lib.get()
    L.init(0)
    return L


def dbuf(lib, a):
    from g4 import DBuf
    return DBuf.from_array(lib, a)


def gpu_q8(lib, x):
    from g4 import DBuf
    xd = dbuf(lib, np.ascontiguousarray(x, np.float32))
    q8 = DBuf(lib, lib.L.g4_q8K_bytes(x.size))
    lib.g4_quantize_row_q8_K(xd.ptr, q8.ptr, x.size)
    return xd, q8


def download_q8(lib, q8, k):
    out = np.zeros(k // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(out), k)
    return out


def q8_cases():
    rng = np.random.default_rng(3)
    cases = [rng.standard_normal(2560).astype(np.float32), rng.standard_normal(10240).astype(np.float32) * 50]
    z = np.zeros(512, np.float32)
    z[256 + 7] = 1.0
    cases.append(z)
    t = rng.standard_normal(256).astype(np.float32)
    t[10], t[20] = 3.0, -3.0
    cases.append(t)
    t = rng.standard_normal(256).astype(np.float32)
    t[5], t[6] = -3.0, 3.0
    cases.append(t)
    h = np.zeros(256, np.float32)
    h[0] = 127.0
    h[1:40] = np.arange(39, dtype=np.float32) - 19.5
    cases.append(h)
    cases.append((rng.standard_normal(256) * 1e-30).astype(np.float32))
    cases.append(np.full(256, -2.0, np.float32))
    return cases


def test_quantize_q8K_bitexact(lib, orc):
    for x in q8_cases():
        _, q8 = gpu_q8(lib, x)
        got = download_q8(lib, q8, x.size)
        assert got.tobytes() == orc.quantize_q8K(x).tobytes()


def test_q8K_upload_download_roundtrip(lib, orc):
    x = np.random.default_rng(4).standard_normal(2560).astype(np.float32)
    ref = orc.quantize_q8K(x)
    from g4 import DBuf
    q8 = DBuf(lib, lib.L.g4_q8K_bytes(2560))
    lib.g4_upload_q8K(q8.ptr, P(ref), 2560)
    assert download_q8(lib, q8, 2560).tobytes() == ref.tobytes()


@pytest.mark.parametrize("qtype", [12, 13, 14])
@pytest.mark.parametrize("n,d", [(256, 5), (2560, 37), (10240, 3)])
def test_layout_roundtrip(lib, qtype, n, d):
    from g4 import download_quant, upload_quant
    raw = synth.rand_kquant(np.random.default_rng(n + d + qtype), qtype, d, n)
    buf = upload_quant(lib, raw, qtype, n, d)
    back = download_quant(lib, buf, qtype, n, d)
    assert back.tobytes() == raw.tobytes()
    assert lib.L.g4_tensor_bytes(qtype, n, d) == raw.nbytes


GEMV_SHAPES = [(256, 300), (2560, 10240), (2560, 2048), (2560, 512), (2048, 2560), (4096, 2560), (10240, 64),
               (2560, 256), (2560, 1)]


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n,d", GEMV_SHAPES)
def test_q45_gemv_bitexact(lib, orc, qtype, n, d):
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(1000 * qtype + n + d)
    raw = synth.rand_kquant(rng, qtype, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, qtype, n, d)
    _, q8 = gpu_q8(lib, x)
    out = DBuf(lib, 4 * d)
    lib.g4_mm_quant_dot_rows(out.ptr, w.ptr, n, d, qtype, q8.ptr)
    got = out.to_array(np.float32)
    want = orc.mm_quant_dot_rows(raw, n, d, qtype, orc.quantize_q8K(x))
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {got[bad[:5]]} vs {want[bad[:5]]}"


@pytest.mark.parametrize("qtype", [12, 13])
def test_block_sums_exact(lib, orc, qtype):
    from g4 import DBuf, upload_quant
    n, d = 2560, 96
    rng = np.random.default_rng(7 + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, qtype, n, d)
    _, q8 = gpu_q8(lib, x)
    S, M = DBuf(lib, 4 * d * 10), DBuf(lib, 4 * d * 10)
    lib.g4_debug_block_sums(w.ptr, n, d, qtype, q8.ptr, S.ptr, M.ptr)
    gS, gM = S.to_array(np.int32).reshape(d, 10), M.to_array(np.int32).reshape(d, 10)
    q8h = orc.quantize_q8K(x)
    bs = synth.BLOCK_BYTES[qtype]
    for r in range(d):
        eS, eM = kq.kquant_block_sums(raw[r].reshape(-1, bs), qtype, q8h)
        assert np.array_equal(gS[r], eS) and np.array_equal(gM[r], eM)


def test_vec_dot_single_row(lib, orc):
    from g4 import DBuf, upload_quant
    n = 2560
    rng = np.random.default_rng(11)
    for qtype, fn in ((12, "g4_vec_dot_q4_K_q8_K"), (13, "g4_vec_dot_q5_K_q8_K"), (14, "g4_vec_dot_q6_K_q8_K")):
        raw = synth.rand_kquant(rng, qtype, 1, n)
        x = rng.standard_normal(n).astype(np.float32)
        w = upload_quant(lib, raw, qtype, n, 1)
        _, q8 = gpu_q8(lib, x)
        out = DBuf(lib, 4)
        getattr(lib, fn)(n, w.ptr, q8.ptr, out.ptr)
        q8h = orc.quantize_q8K(x)
        f = {12: orc.L.or_vec_dot_q4K_q8K, 13: orc.L.or_vec_dot_q5K_q8K, 14: orc.L.or_vec_dot_q6K_q8K}[qtype]
        want = np.float32(f(n, P(raw), P(q8h)))
        assert out.to_array(np.float32)[0].tobytes() == want.tobytes()


@pytest.mark.parametrize("n,d", [(2560, 512), (10240, 2560), (2560, 8192), (256, 40)])
def test_q6K_f32_gemv(lib, orc, n, d):
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(n * 3 + d)
    raw = synth.rand_q6K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, 14, n, d)
    xd = dbuf(lib, x)
    out = DBuf(lib, 4 * d)
    lib.g4_mm_quant_rows(out.ptr, xd.ptr, w.ptr, n, d, 14)
    got = out.to_array(np.float32)
    want = orc.mm_quant_rows(x, raw, n, d, 14)
    W = np.abs(kq.dequant_f64(raw.reshape(-1, 210), 14).reshape(d, n))
    mag = W @ np.abs(x.astype(np.float64))
    err = np.abs(got.astype(np.float64) - want) / mag
    assert err.max() <= 1e-5, err.max()


@pytest.mark.parametrize("d", [4096, 16384, 262144])
def test_q6K_softcap(lib, orc, d):
    """logits_tied's GEMV + soft-cap.  262144 and 16384 rows (at n = 2560)
    take the kernel with x held in registers, batches of 64 rows dealt to the
    workgroups (262144 rows is the LM head itself, the instantiation the
    decode step runs); 4096 rows takes the K-sliced LDS form."""
    from g4 import DBuf, upload_quant
    n = 2560
    rng = np.random.default_rng(2 + d)
    raw = synth.rand_q6K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, 14, n, d)
    xd = dbuf(lib, x)
    out = DBuf(lib, 4 * d)
    lib.g4_mm_quant_rows_softcap(out.ptr, xd.ptr, w.ptr, n, d, 14, 30.0)
    got = out.to_array(np.float32)
    raw_l = orc.mm_quant_rows(x, raw, n, d, 14)
    want = (np.float32(30.0) * np.tanh(raw_l * np.float32(1.0 / 30.0))).astype(np.float32)
    # the cap's derivative is <= 1, so the GEMV bar (1e-5 of sum |w*x|) carries
    # over; a few ulps of 30 cover tanhf itself
    mag = kq.abs_dot_rows(raw, 14, n, x)
    err = np.abs(got.astype(np.float64) - want) - 1e-5
    assert (err <= 1e-5 * mag).all(), float(np.max(err / mag))


@pytest.mark.parametrize("d", [16384, 262144])
def test_q6K_f32_gemv_lm_head_rows(lib, orc, d):
    """mm_quant_rows (no cap) at LM-head row counts."""
    from g4 import DBuf, upload_quant
    n = 2560
    rng = np.random.default_rng(7 + d)
    raw = synth.rand_q6K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, 14, n, d)
    xd = dbuf(lib, x)
    out = DBuf(lib, 4 * d)
    lib.g4_mm_quant_rows(out.ptr, xd.ptr, w.ptr, n, d, 14)
    got = out.to_array(np.float32)
    want = orc.mm_quant_rows(x, raw, n, d, 14)
    err = np.abs(got.astype(np.float64) - want) / kq.abs_dot_rows(raw, 14, n, x)
    assert err.max() <= 1e-5, err.max()


@pytest.mark.parametrize("d", [3000, 262144])
def test_q6K_q8K_gemv_bitexact(lib, orc, d):
    """Q6_K x Q8_K rows (the form the north star names for the LM head): bit
    for bit with the oracle, at a small row count and at 262144 rows (where
    the launch picks another rows-per-group tiling)."""
    from g4 import DBuf, upload_quant
    n = 2560
    rng = np.random.default_rng(21 + d)
    raw = synth.rand_q6K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, 14, n, d)
    _, q8 = gpu_q8(lib, x)
    out = DBuf(lib, 4 * d)
    lib.g4_mm_quant_dot_rows(out.ptr, w.ptr, n, d, 14, q8.ptr)
    want = orc.mm_quant_dot_rows(raw, n, d, 14, orc.quantize_q8K(x))
    assert np.array_equal(out.to_array(np.float32).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n,d", [(2560, 10752), (256, 100), (4096, 33)])
def test_bf16_gemv(lib, orc, n, d):
    from g4 import DBuf
    rng = np.random.default_rng(n + d)
    wh = synth.rand_bf16(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w, xd, out = dbuf(lib, wh), dbuf(lib, x), DBuf(lib, 4 * d)
    lib.g4_mm_bf16(out.ptr, xd.ptr, w.ptr, n, d)
    got = out.to_array(np.float32)
    want = orc.mm_bf16(x, wh, n, d)
    W = (wh.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    assert (np.abs(got - want) <= 1e-5 * mag).all()


@pytest.mark.parametrize("qtype", [12, 13])
def test_gate_up_gelu(lib, orc, qtype):
    from g4 import DBuf, upload_quant
    n, d = 2560, 10240
    rng = np.random.default_rng(31 + qtype)
    g_raw = synth.rand_kquant(rng, qtype, d, n)
    u_raw = synth.rand_kquant(rng, qtype, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    gw, uw = upload_quant(lib, g_raw, qtype, n, d), upload_quant(lib, u_raw, qtype, n, d)
    _, q8 = gpu_q8(lib, x)
    out = DBuf(lib, 4 * d)
    lib.g4_mm_gate_up_gelu(out.ptr, gw.ptr, uw.ptr, n, d, qtype, q8.ptr)
    q8h = orc.quantize_q8K(x)
    g = orc.mm_quant_dot_rows(g_raw, n, d, qtype, q8h)
    u = orc.mm_quant_dot_rows(u_raw, n, d, qtype, q8h)
    want = np.array([orc.L.or_gelu(float(v)) for v in g], np.float32) * u
    got = out.to_array(np.float32)
    # gate and up are bit-exact; only tanhf (device libm vs glibc) may differ by ulps
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


def test_mm_dispatch(lib, orc):
    from g4 import DBuf, upload_quant
    n, d = 2560, 512
    rng = np.random.default_rng(41)
    raw = synth.rand_q4K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = upload_quant(lib, raw, 12, n, d)
    xd = dbuf(lib, x)
    q8 = DBuf(lib, lib.L.g4_q8K_bytes(n))
    out = DBuf(lib, 4 * d)
    lib.g4_mm(out.ptr, xd.ptr, w.ptr, n, d, 12, q8.ptr, 0)
    want = orc.mm_quant_dot_rows(raw, n, d, 12, orc.quantize_q8K(x))
    assert np.array_equal(out.to_array(np.float32).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", [12, 13])
def test_gelu_mul_epilogue(lib, orc, qtype):
    """PLE gate: gelu(W.q8) * mul (main.c:1988-1993) in the GEMV epilogue."""
    from g4 import DBuf, upload_quant
    n, d = 2560, 256
    rng = np.random.default_rng(51 + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    mul = rng.standard_normal(d).astype(np.float32)
    w = upload_quant(lib, raw, qtype, n, d)
    _, q8 = gpu_q8(lib, x)
    md, out = dbuf(lib, mul), DBuf(lib, 4 * d)
    lib.g4_mm_quant_dot_rows_gelu_mul(out.ptr, w.ptr, n, d, qtype, q8.ptr, md.ptr)
    g = orc.mm_quant_dot_rows(raw, n, d, qtype, orc.quantize_q8K(x))
    want = np.array([orc.L.or_gelu(float(v)) for v in g], np.float32) * mul
    # the GEMV is bit-exact; tanhf (device libm vs glibc) may differ by ulps
    assert np.allclose(out.to_array(np.float32), want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


@pytest.mark.parametrize("qtype", [12, 13])
def test_mm_single_block_quantizes_inside(lib, orc, qtype):
    """mm() on a 256-wide input quantizes inside the GEMV; the output and the
    q8 side effect equal the reference's quantize_row_q8_K + dot."""
    from g4 import DBuf, upload_quant
    n, d = 256, 2560
    rng = np.random.default_rng(61 + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = upload_quant(lib, raw, qtype, n, d)
    xd, q8, out = dbuf(lib, x), DBuf(lib, lib.L.g4_q8K_bytes(n)), DBuf(lib, 4 * d)
    lib.g4_mm(out.ptr, xd.ptr, w.ptr, n, d, qtype, q8.ptr, 0)
    q8h = orc.quantize_q8K(x)
    want = orc.mm_quant_dot_rows(raw, n, d, qtype, q8h)
    assert np.array_equal(out.to_array(np.float32).view(np.uint32), want.view(np.uint32))
    assert download_q8(lib, q8, n).tobytes() == q8h.tobytes()


def rel_err(got, want):
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


@pytest.mark.parametrize("qtype,n,d,mode", [(12, 2560, 2048, "attn"), (12, 2560, 256, "ple"), (13, 2560, 200, "attn"),
                                            (12, 2048, 96, "first"), (12, 4096, 520, "attn"), (13, 2560, 256, "ple"),
                                            (12, 2560, 10240, "ffn"), (13, 2560, 1000, "ffn")])
def test_mm_residual_q8(lib, orc, qtype, n, d, mode):
    """Residual step + norm + Q8_K as the GEMV's prologue (g4_mm_residual_q8):
    x_out and xb2 to the residual_norm bars against the oracle's rmsnorm; the
    stored Q8_K equal to quantize_row_q8_K of the stored vector; every output
    row equal, bit for bit, to mm_quant_dot_rows on that stored Q8_K (each
    workgroup quantizes for itself, so this also checks that they agree)."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(n + d + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    w = upload_quant(lib, raw, qtype, n, d)
    x = rng.standard_normal(n).astype(np.float32)
    y = (rng.standard_normal(n) * 4).astype(np.float32)
    wp = rng.uniform(0.5, 1.5, n).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, n).astype(np.float32)
    osc = np.array([0.9], np.float32)
    mul = rng.standard_normal(d).astype(np.float32)
    xd, yd, wpd, wnd, od = (DBuf.from_array(lib, a) for a in (x, y, wp, wn, osc))
    xo, xb2, out = DBuf(lib, 4 * n), DBuf(lib, 4 * n), DBuf(lib, 4 * d)
    q8 = DBuf(lib, lib.L.g4_q8K_bytes(n))
    muld = DBuf.from_array(lib, mul)
    eps = C.c_float(1e-6)
    up_raw = synth.rand_kquant(rng, qtype, d, n) if mode == "ffn" else None
    up = upload_quant(lib, up_raw, qtype, n, d) if mode == "ffn" else None
    if mode == "ffn":        # post_attention_norm + residual, ffn_norm, Q8_K; gelu(gate) * up
        lib.g4_mm_residual_q8(out.ptr, w.ptr, up.ptr, n, d, qtype, None, xd.ptr, xo.ptr, yd.ptr, wpd.ptr, None, wnd.ptr,
                              xb2.ptr, q8.ptr, 0, eps)
        want_x = x + orc.rmsnorm(y, wp)
        want_v = orc.rmsnorm(want_x, wn)
        got_v = xb2.to_array(np.float32)
        assert rel_err(got_v, want_v) < 4e-6
    elif mode == "attn":     # post_norm + residual + out_scale, next attn_norm, Q8_K of xb2
        lib.g4_mm_residual_q8(out.ptr, w.ptr, None, n, d, qtype, None, xd.ptr, xo.ptr, yd.ptr, wpd.ptr, od.ptr, wnd.ptr,
                              xb2.ptr, q8.ptr, 0, eps)
        want_x = (x + orc.rmsnorm(y, wp)) * osc[0]
        want_v = orc.rmsnorm(want_x, wn)
        got_v = xb2.to_array(np.float32)
        assert rel_err(got_v, want_v) < 4e-6
    elif mode == "ple":      # post_ffw_norm + residual, Q8_K of x, gelu * mul epilogue
        lib.g4_mm_residual_q8(out.ptr, w.ptr, None, n, d, qtype, muld.ptr, xd.ptr, xo.ptr, yd.ptr, wpd.ptr, None, None, None,
                              q8.ptr, 1, eps)
        want_x = x + orc.rmsnorm(y, wp)
        got_v = xo.to_array(np.float32)
    else:                    # layer 0: attn_norm only, the stream is not rewritten
        lib.g4_mm_residual_q8(out.ptr, w.ptr, None, n, d, qtype, None, xd.ptr, xd.ptr, None, None, None, wnd.ptr, xb2.ptr,
                              q8.ptr, 0, eps)
        want_x = x
        got_v = xb2.to_array(np.float32)
        assert rel_err(got_v, orc.rmsnorm(x, wn)) < 4e-6
    gx = xo.to_array(np.float32) if mode != "first" else xd.to_array(np.float32)
    assert rel_err(gx, want_x) < 2e-6
    if mode == "first":
        assert np.array_equal(gx, x)
    h = np.zeros(n // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), n)
    assert h.tobytes() == orc.quantize_q8K(got_v).tobytes()
    ref = DBuf(lib, 4 * d)
    if mode == "ffn":
        lib.g4_mm_gate_up_gelu(ref.ptr, w.ptr, up.ptr, n, d, qtype, q8.ptr)
    elif mode == "ple":
        lib.g4_mm_quant_dot_rows_gelu_mul(ref.ptr, w.ptr, n, d, qtype, q8.ptr, muld.ptr)
    else:
        lib.g4_mm_quant_dot_rows(ref.ptr, w.ptr, n, d, qtype, q8.ptr)
    g, r = out.to_array(np.float32), ref.to_array(np.float32)
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), np.flatnonzero(g != r)[:8]
    # and against the oracle: mm_quant_dot_rows on the stored Q8_K bit for bit,
    # the GELU epilogues within 1e-6 of the oracle's gelu (device tanhf)
    dot = orc.mm_quant_dot_rows(raw, n, d, qtype, h)
    if mode in ("ffn", "ple"):
        other = orc.mm_quant_dot_rows(up_raw, n, d, qtype, h) if mode == "ffn" else mul
        want = np.array([orc.L.or_gelu(C.c_float(v)) for v in dot], np.float32) * other
        assert rel_err(g, want) < 1e-6
    else:
        assert np.array_equal(g.view(np.uint32), dot.view(np.uint32))


@pytest.mark.parametrize("cancel", [0.0, 0.9, 0.999])
def test_residual_step_norms_when_the_step_cancels(lib, orc, cancel):
    """The two norms of a residual step (post_norm + residual + out_scale,
    then the next attn_norm, main.c:1995-2003, 1878) when the step cancels
    most of x: inputs with x = -cancel * (y s_y) w + noise drive x' toward
    zero, and the normed vector must stay within 4e-6 of the float64 RMSNorm
    of the x' the kernel itself stored (its second sum of squares is that of
    x', not of x and the step), in the single-workgroup step and in the GEMV
    prologue, which give the same bits."""
    from g4 import DBuf, upload_quant
    n, d = 2560, 256
    rng = np.random.default_rng(int(cancel * 1000) + 5)
    y = (rng.standard_normal(n) * 4).astype(np.float32)
    wp = rng.uniform(0.5, 1.5, n).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, n).astype(np.float32)
    sy = 1.0 / np.sqrt(np.mean(y.astype(np.float64) ** 2) + 1e-6)
    x = (-cancel * (y * sy) * wp + 0.01 * rng.standard_normal(n)).astype(np.float32)
    osc = np.array([0.9], np.float32)
    xd, yd, wpd, wnd, od = (DBuf.from_array(lib, a) for a in (x, y, wp, wn, osc))
    eps = C.c_float(1e-6)
    raw = synth.rand_kquant(rng, 12, d, n)
    w = upload_quant(lib, raw, 12, n, d)
    outs = []
    for form in ("step", "prologue"):
        xo, xb2, q8 = DBuf(lib, 4 * n), DBuf(lib, 4 * n), DBuf(lib, lib.L.g4_q8K_bytes(n))
        if form == "step":
            x2 = DBuf.from_array(lib, x)
            lib.g4_residual_norm(x2.ptr, yd.ptr, wpd.ptr, od.ptr, wnd.ptr, xb2.ptr, q8.ptr, 0, n, eps)
            gx = x2.to_array(np.float32)
        else:
            out = DBuf(lib, 4 * d)
            lib.g4_mm_residual_q8(out.ptr, w.ptr, None, n, d, 12, None, xd.ptr, xo.ptr, yd.ptr, wpd.ptr, od.ptr,
                                  wnd.ptr, xb2.ptr, q8.ptr, 0, eps)
            gx = xo.to_array(np.float32)
        gv = xb2.to_array(np.float32)
        x64 = gx.astype(np.float64)
        want = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-6) * wn
        assert rel_err(gv, want) < 4e-6, form
        h = np.zeros(n // 256, Q8K_DTYPE)
        lib.g4_download_q8K(q8.ptr, P(h), n)
        assert h.tobytes() == orc.quantize_q8K(gv).tobytes()
        outs.append((gx, gv))
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))


def test_mm_residual_q8_rejects_alias(lib):
    from g4 import DBuf, G4Error
    b = DBuf(lib, 4 * 4096)
    with pytest.raises(G4Error):
        lib.g4_mm_residual_q8(b.ptr, b.ptr, None, 2560, 8, 12, None, b.ptr, b.ptr, b.ptr, b.ptr, None, None, None, None, 1,
                              C.c_float(1e-6))


@pytest.mark.parametrize("qtype,d1,d2", [(12, 2048, 512), (13, 200, 70), (12, 4096, 1024)])
def test_mm_residual_q8_pair(lib, orc, qtype, d1, d2):
    """Two GEMVs stacked in one prologue launch (Q and K): the stored Q8_K is
    quantize_row_q8_K of the stored normed vector, and each output equals,
    bit for bit, the GPU's and the oracle's mm_quant_dot_rows on it."""
    from g4 import DBuf, upload_quant
    n = 2560
    rng = np.random.default_rng(d1 + d2 + qtype)
    r1, r2 = synth.rand_kquant(rng, qtype, d1, n), synth.rand_kquant(rng, qtype, d2, n)
    w1, w2 = upload_quant(lib, r1, qtype, n, d1), upload_quant(lib, r2, qtype, n, d2)
    x = rng.standard_normal(n).astype(np.float32)
    y = (rng.standard_normal(n) * 4).astype(np.float32)
    wp = rng.uniform(0.5, 1.5, n).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, n).astype(np.float32)
    xd, yd, wpd, wnd = (DBuf.from_array(lib, a) for a in (x, y, wp, wn))
    xo, xb2, o1, o2 = DBuf(lib, 4 * n), DBuf(lib, 4 * n), DBuf(lib, 4 * d1), DBuf(lib, 4 * d2)
    q8 = DBuf(lib, lib.L.g4_q8K_bytes(n))
    lib.g4_mm_residual_q8_pair(o1.ptr, w1.ptr, d1, o2.ptr, w2.ptr, d2, n, qtype, xd.ptr, xo.ptr, yd.ptr, wpd.ptr, None,
                               wnd.ptr, xb2.ptr, q8.ptr, 0, C.c_float(1e-6))
    assert rel_err(xo.to_array(np.float32), x + orc.rmsnorm(y, wp)) < 2e-6
    h = np.zeros(n // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), n)
    assert h.tobytes() == orc.quantize_q8K(xb2.to_array(np.float32)).tobytes()
    for o, w, d, raw in ((o1, w1, d1, r1), (o2, w2, d2, r2)):
        ref = DBuf(lib, 4 * d)
        lib.g4_mm_quant_dot_rows(ref.ptr, w.ptr, n, d, qtype, q8.ptr)
        g, r = o.to_array(np.float32), ref.to_array(np.float32)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (d, np.flatnonzero(g != r)[:8])
        want = orc.mm_quant_dot_rows(raw, n, d, qtype, h)
        assert np.array_equal(g.view(np.uint32), want.view(np.uint32)), (d, np.flatnonzero(g != want)[:8])


@pytest.mark.parametrize("qtype,d1,d2,d3", [(12, 2048, 512, 512), (13, 200, 70, 90), (12, 4096, 1024, 1024)])
def test_mm_residual_q8_qkv(lib, orc, qtype, d1, d2, d3):
    """Q, K (K-quant, stacked) and V (Q6_K on the fp32 normed vector) in one
    prologue launch: Q and K bit-exact against the GPU's and the oracle's
    mm_quant_dot_rows on the stored Q8_K (itself quantize_row_q8_K of the
    stored normed vector); V against the oracle's mm_quant_rows on the stored
    normed vector to 1e-5 of sum |w*x|."""
    from g4 import DBuf, upload_quant
    n = 2560
    rng = np.random.default_rng(d1 + d2 + d3 + qtype)
    r1, r2 = synth.rand_kquant(rng, qtype, d1, n), synth.rand_kquant(rng, qtype, d2, n)
    r3 = synth.rand_q6K(rng, d3, n)
    w1, w2, w3 = upload_quant(lib, r1, qtype, n, d1), upload_quant(lib, r2, qtype, n, d2), upload_quant(lib, r3, 14, n, d3)
    x = rng.standard_normal(n).astype(np.float32)
    y = (rng.standard_normal(n) * 4).astype(np.float32)
    wp = rng.uniform(0.5, 1.5, n).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, n).astype(np.float32)
    osc = np.array([0.9], np.float32)
    xd, yd, wpd, wnd, od = (DBuf.from_array(lib, a) for a in (x, y, wp, wn, osc))
    xo, xb2 = DBuf(lib, 4 * n), DBuf(lib, 4 * n)
    o1, o2, o3 = DBuf(lib, 4 * d1), DBuf(lib, 4 * d2), DBuf(lib, 4 * d3)
    q8 = DBuf(lib, lib.L.g4_q8K_bytes(n))
    lib.g4_mm_residual_q8_qkv(o1.ptr, w1.ptr, d1, o2.ptr, w2.ptr, d2, o3.ptr, w3.ptr, d3, 14, n, qtype, xd.ptr, xo.ptr,
                              yd.ptr, wpd.ptr, od.ptr, wnd.ptr, xb2.ptr, q8.ptr, C.c_float(1e-6))
    want_x = (x + orc.rmsnorm(y, wp)) * osc[0]
    assert rel_err(xo.to_array(np.float32), want_x) < 2e-6
    xb = xb2.to_array(np.float32)
    assert rel_err(xb, orc.rmsnorm(want_x, wn)) < 4e-6
    h = np.zeros(n // 256, Q8K_DTYPE)
    lib.g4_download_q8K(q8.ptr, P(h), n)
    assert h.tobytes() == orc.quantize_q8K(xb2.to_array(np.float32)).tobytes()
    for o, w, d, raw in ((o1, w1, d1, r1), (o2, w2, d2, r2)):
        ref = DBuf(lib, 4 * d)
        lib.g4_mm_quant_dot_rows(ref.ptr, w.ptr, n, d, qtype, q8.ptr)
        g, r = o.to_array(np.float32), ref.to_array(np.float32)
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (d, np.flatnonzero(g != r)[:8])
        want = orc.mm_quant_dot_rows(raw, n, d, qtype, h)
        assert np.array_equal(g.view(np.uint32), want.view(np.uint32)), (d, np.flatnonzero(g != want)[:8])
    want = orc.mm_quant_rows(xb, r3, n, d3, 14)
    W = np.abs(kq.dequant_f64(r3.reshape(-1, 210), 14).reshape(d3, n))
    mag = W @ np.abs(xb.astype(np.float64))
    err = np.abs(o3.to_array(np.float32).astype(np.float64) - want) / mag
    assert err.max() <= 1e-5, err.max()


def _dense(rng, qtype, d, n):
    """(device bytes, oracle function) of a random dense matrix"""
    if qtype == 30:
        return synth.rand_bf16(rng, d, n), "or_mm_bf16"
    a = (rng.standard_normal((d, n), dtype=np.float32) * 0.05)
    if qtype == 1:
        return a.astype(np.float16).view(np.uint16), "or_mm_f16"
    return a.astype(np.float32), "or_mm_f32"


@pytest.mark.parametrize("qtype,n,d", [(1, 2560, 300), (1, 10240, 64), (0, 2560, 77), (0, 10240, 33), (0, 4100, 9),
                                       (30, 10240, 40), (30, 2560, 96), (1, 256, 16), (1, 16384, 8)])
def test_dense_gemv(lib, orc, qtype, n, d):
    """mm_f16 / mm_f32 / mm_bf16 (main.c:1494-1537) through g4_mm, rows up to
    16384 long: 1e-5 of sum |w x| against the oracle's sequential sums."""
    from g4 import DBuf
    rng = np.random.default_rng(n + d + qtype)
    w, fn = _dense(rng, qtype, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    wd, xd, out = dbuf(lib, w), dbuf(lib, x), DBuf(lib, 4 * d)
    lib.g4_mm(out.ptr, xd.ptr, wd.ptr, n, d, qtype, None, 0)
    got = out.to_array(np.float32)
    want = np.empty(d, np.float32)
    getattr(orc.L, fn)(P(want), P(x), P(w), n, d)
    W = {30: (w.astype(np.uint32) << 16).view(np.float32), 1: w.view(np.float16).astype(np.float32),
         0: w}[qtype].astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    assert (np.abs(got.astype(np.float64) - want) <= 1e-5 * mag).all()


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n,d", [(2560, 96), (10240, 40), (256, 8)])
def test_quant_rows_f32_q45(lib, orc, qtype, n, d):
    """mm_quant_rows for Q4_K / Q5_K (the reference's --f32-matmul path,
    main.c:1680-1683): dequantized weights times fp32 x, 1e-5 of sum |w x|."""
    from g4 import DBuf, upload_quant
    rng = np.random.default_rng(n * 7 + d + qtype)
    raw = synth.rand_kquant(rng, qtype, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w, xd, out = upload_quant(lib, raw, qtype, n, d), dbuf(lib, x), DBuf(lib, 4 * d)
    lib.g4_mm_quant_rows(out.ptr, xd.ptr, w.ptr, n, d, qtype)
    got = out.to_array(np.float32)
    want = orc.mm_quant_rows(x, raw, n, d, qtype)
    W = np.abs(kq.dequant_f64(raw.reshape(-1, synth.BLOCK_BYTES[qtype]), qtype).reshape(d, n))
    mag = W @ np.abs(x.astype(np.float64))
    assert (np.abs(got.astype(np.float64) - want) / mag).max() <= 1e-5


def test_softcap(lib):
    """logits_tied's soft-cap (main.c:1789-1795) within a few ulp of
    cap * tanh(v / cap) (device tanhf against the exact value)."""
    rng = np.random.default_rng(17)
    v = (rng.standard_normal(100003) * 40).astype(np.float32)
    vd = dbuf(lib, v)
    lib.g4_softcap(vd.ptr, v.size, C.c_float(30.0))
    got = vd.to_array(np.float32).astype(np.float64)
    inv = np.float32(1.0) / np.float32(30.0)
    want = 30.0 * np.tanh((v * inv).astype(np.float64))
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) < 2e-6


@pytest.mark.parametrize("qg,qp", [(12, 12), (13, 12), (12, 13)])
def test_mm_ple_gate_proj(lib, orc, qg, qp):
    """The PLE gate and projection in one launch (g4_mm_ple_gate_proj):
    y and x_out equal, bit for bit, to g4_mm_residual_q8 (qsrc 1, gelu * mul)
    followed by g4_mm on the 256 gate values, over three calls on one pairs
    buffer with the sequence word advanced between them (new inputs each
    time, so values left from an earlier call would show); y also against
    the oracle: mm_quant_dot_rows of the projection on quantize_row_q8_K of
    the gate values."""
    from g4 import DBuf, upload_quant
    n, pd, dp = 2560, 256, 2560
    rng = np.random.default_rng(70 + qg + 3 * qp)
    g_raw = synth.rand_kquant(rng, qg, pd, n)
    p_raw = synth.rand_kquant(rng, qp, dp, pd)
    wg, wp = upload_quant(lib, g_raw, qg, n, pd), upload_quant(lib, p_raw, qp, pd, dp)
    pairs = DBuf(lib, lib.L.g4_ple_pairs_bytes(pd))
    lib.g4_memset(pairs.ptr, 0, lib.L.g4_ple_pairs_bytes(pd))
    seq = dbuf(lib, np.array([0], np.uint32))
    eps = C.c_float(1e-6)
    for call in range(3):
        lib.g4_memcpy_h2d(seq.ptr, P(np.array([call + 1], np.uint32)), 4)
        x = rng.standard_normal(n).astype(np.float32)
        y_in = (rng.standard_normal(n) * 4).astype(np.float32)
        wpost = rng.uniform(0.5, 1.5, n).astype(np.float32)
        mul = rng.standard_normal(pd).astype(np.float32)
        xd, yd, wpd, muld = dbuf(lib, x), dbuf(lib, y_in), dbuf(lib, wpost), dbuf(lib, mul)
        xo, y = DBuf(lib, 4 * n), DBuf(lib, 4 * dp)
        lib.g4_mm_ple_gate_proj(y.ptr, wp.ptr, qp, dp, wg.ptr, qg, n, pd, muld.ptr, xd.ptr, xo.ptr, yd.ptr, wpd.ptr,
                                eps, pairs.ptr, seq.ptr)
        xo2, g2, y2 = DBuf(lib, 4 * n), DBuf(lib, 4 * pd), DBuf(lib, 4 * dp)
        q8a, q8b = DBuf(lib, lib.L.g4_q8K_bytes(n)), DBuf(lib, lib.L.g4_q8K_bytes(pd))
        lib.g4_mm_residual_q8(g2.ptr, wg.ptr, None, n, pd, qg, muld.ptr, xd.ptr, xo2.ptr, yd.ptr, wpd.ptr, None, None,
                              None, q8a.ptr, 1, eps)
        lib.g4_mm(y2.ptr, g2.ptr, wp.ptr, pd, dp, qp, q8b.ptr, 0)
        lib.g4_sync()
        assert np.array_equal(y.to_array(np.uint32), y2.to_array(np.uint32)), f"call {call}: y"
        assert np.array_equal(xo.to_array(np.uint32), xo2.to_array(np.uint32)), f"call {call}: x_out"
        words = pairs.to_array(np.uint32)
        assert np.all(words[1:2 * pd:2] == call + 1) and words[2 * pd] == 0
        assert np.array_equal(words[0:2 * pd:2], g2.to_array(np.uint32))
    g = g2.to_array(np.float32)
    want = orc.mm_quant_dot_rows(p_raw, pd, dp, qp, orc.quantize_q8K(g))
    assert np.array_equal(y.to_array(np.float32).view(np.uint32), want.view(np.uint32))
