"""GPU parity of the batched prefill GEMMs (g4_mm_batch_q8 / g4_mm_batch):
m tokens through one matrix on the matrix cores.

The reference has no batched path; its prefill is forward() per token
(main.c:2366-2384), i.e. quantize_row_q8_K + mm_quant_dot_rows per token for
Q4_K / Q5_K, mm_quant_rows / mm_bf16 on the fp32 activations for Q6_K / bf16.
Q4_K / Q5_K: bit-equality with the per-token path -- every output of the
batched kernel has the same fp32 bits as the per-token GEMV (itself bit-exact
to the oracle's AVX2 dot), and, for sampled tokens, as the oracle.  Q6_K /
bf16: the weights are dequantized to the reference's fp32 values and only the
order of the fp32 sums differs, so the bar is that of the GEMVs, 1e-5 of
sum |w x| against the oracle; and a token's outputs do not depend on the
other tokens of the batch or its place in it (bit for bit).
"""
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
    return L


def _acts(rng, m, n):
    x = rng.standard_normal((m, n)).astype(np.float32)
    x[m // 2] = 0.0                      # an all-zero token: Q8_K d = 0
    if m > 3:
        x[1] *= 1e3
        x[2, :256] = 0.0                 # one all-zero block inside a token
    return x


def _batch(lib, raw, qtype, n, d, x):
    from g4 import DBuf, upload_quant
    m = x.shape[0]
    w = upload_quant(lib, raw, qtype, n, d)
    xd = DBuf.from_array(lib, x)
    qb = lib.L.g4_q8K_row_stride(n)
    q8 = DBuf(lib, qb * m)
    lib.g4_quantize_rows_q8_K(xd.ptr, q8.ptr, n, m)
    out = DBuf(lib, 4 * m * d)
    lib.g4_mm_batch_q8(out.ptr, w.ptr, q8.ptr, n, d, m, qtype)
    return w, q8, qb, out.to_array(np.float32).reshape(m, d)


def test_quantize_rows_equals_per_row(lib, orc):
    from g4 import DBuf
    rng = np.random.default_rng(5)
    m, n = 7, 2560
    x = _acts(rng, m, n)
    xd = DBuf.from_array(lib, x)
    qb = lib.L.g4_q8K_row_stride(n)
    q8 = DBuf(lib, qb * m)
    lib.g4_quantize_rows_q8_K(xd.ptr, q8.ptr, n, m)
    for t in range(m):
        got = np.zeros(n // 256, Q8K_DTYPE)
        lib.g4_download_q8K(q8.ptr + t * qb, P(got), n)
        assert got.tobytes() == orc.quantize_q8K(x[t]).tobytes(), t


SHAPES = [(256, 80, 37), (2560, 70, 17), (2560, 2048, 64), (2048, 2560, 100), (10240, 192, 65), (2560, 10240, 130)]


@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n,d,m", SHAPES)
def test_mm_batch_bitexact_vs_per_token(lib, orc, qtype, n, d, m):
    from g4 import DBuf
    rng = np.random.default_rng(100 * qtype + n + d + m)
    raw = synth.rand_kquant(rng, qtype, d, n)
    x = _acts(rng, m, n)
    w, q8, qb, got = _batch(lib, raw, qtype, n, d, x)
    one = DBuf(lib, 4 * d)
    for t in range(m):
        lib.g4_mm_quant_dot_rows(one.ptr, w.ptr, n, d, qtype, q8.ptr + t * qb)
        want = one.to_array(np.float32)
        bad = np.flatnonzero(got[t].view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"token {t}: {bad.size} rows differ, first {bad[:4]}: {got[t][bad[:4]]} vs {want[bad[:4]]}"
    for t in sorted({0, 1, m // 2, m - 1}):
        want = orc.mm_quant_dot_rows(raw, n, d, qtype, orc.quantize_q8K(x[t]))
        assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), t


def test_mm_batch_wrapper(lib, orc):
    """g4_mm_batch against mm() per token for every type: Q4_K/Q5_K equal it
    bit for bit; Q6_K and bf16 (fp32 matrix-core sums) to 1e-5 of sum |w x|."""
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
        one = DBuf(lib, 4 * d)
        q1 = DBuf(lib, lib.L.g4_q8K_bytes(n))
        for t in range(m):
            xt = DBuf.from_array(lib, x[t])
            lib.g4_mm(one.ptr, xt.ptr, w.ptr, n, d, qtype, q1.ptr, 0)
            if qtype in (12, 13):
                assert np.array_equal(got[t].view(np.uint32), one.to_array(np.float32).view(np.uint32)), (qtype, t)
            else:
                mag = _mag(raw, qtype, n, d, x[t])
                assert (np.abs(got[t] - one.to_array(np.float32)) <= 1e-5 * mag).all(), (qtype, t)


def _mag(raw, qtype, n, d, x):
    """sum_j |w_ij x_j| per row, the scale of an fp32 dot's rounding"""
    import kquant_np as kq
    if qtype == 30:
        W = (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(d, n)
    else:
        W = kq.dequant_f64(raw.reshape(-1, 210), 14).reshape(d, n)
    return np.abs(W) @ np.abs(x.astype(np.float64))


F32W_SHAPES = [(2560, 512, 511), (2560, 1024, 130), (10240, 2560, 37), (2560, 10752, 33), (256, 40, 5),
               (512, 256, 24), (2560, 96, 1)]


@pytest.mark.parametrize("qtype", [14, 30])
@pytest.mark.parametrize("n,d,m", F32W_SHAPES)
def test_mm_batch_f32_weights(lib, orc, qtype, n, d, m):
    """Q6_K (V, FFN down) and bf16 (PLE projection) over m tokens: each
    sampled token within 1e-5 of sum |w x| of the oracle's mm_quant_rows /
    mm_bf16 (main.c:1539-1556, 1529-1537); the same token rows in a batch
    shifted by 5 tokens (other tile positions, other neighbours) give the
    same bits."""
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
        mag = _mag(raw, qtype, n, d, x[t])
        assert (np.abs(got[t].astype(np.float64) - want) <= 1e-5 * mag + 1e-30).all(), t


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
