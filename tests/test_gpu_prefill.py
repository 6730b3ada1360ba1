"""GPU parity of the batched prefill GEMM (g4_mm_batch_q8 / g4_mm_batch):
m tokens through one Q4_K / Q5_K matrix on the matrix cores.

The reference has no batched path; its prefill is forward() per token
(main.c:2366-2384), i.e. quantize_row_q8_K + mm_quant_dot_rows per token.
The bar is therefore bit-equality with the per-token path: every output of
the batched kernel must have the same fp32 bits as the per-token GEMV (itself
bit-exact to the oracle's AVX2 dot), and, for sampled tokens, as the oracle.
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
    """g4_mm_batch = mm() per token for every type: Q4_K/Q5_K through the
    batched kernel, Q6_K and BF16 through the per-token GEMV."""
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
            assert np.array_equal(got[t].view(np.uint32), one.to_array(np.float32).view(np.uint32)), (qtype, t)


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
