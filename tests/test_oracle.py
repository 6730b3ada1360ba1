"""Pins the CPU oracle: bit-exact against the reference's own functions
(oracle/_ref, compiled from gemma4-4b/cpu-blas/main.c) and against closed
forms / brute force that a plausible mistake would break."""
import ctypes as C
import math

import numpy as np
import pytest

import kquant_np as kq
import synth
from oracle import Q8K_DTYPE

P = lambda a: a.ctypes.data  # noqa: E731


def _blocks(qtype, rows, n, seed):
    return synth.rand_kquant(np.random.default_rng(seed), qtype, rows, n)


def _subnormal_d(blk, qtype):
    """Force some fp16 subnormal d/dmin values (main.c:133-140 path)."""
    b = blk.reshape(-1, synth.BLOCK_BYTES[qtype])
    sub = np.array([1, 3, 0x3FF, 0x200, 0x8001], np.uint16).view(np.uint8)
    for i in range(min(5, b.shape[0])):
        off = 208 if qtype == 14 else 0
        b[i, off:off + 2] = sub[2 * i:2 * i + 2]
    return blk


# --------------------------------------------------------------------------
# fp16 / bf16 / scale unpack
# --------------------------------------------------------------------------
def test_f16_all_values(orc, ref):
    h = np.arange(65536, dtype=np.uint16)
    ours = np.array([orc.L.or_f16_to_f32(int(v)) for v in h], np.float32)
    theirs = np.array([ref.L.ref_host_f16f32(int(v)) for v in h], np.float32)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    # closed form: IEEE binary16 widening (numpy), NaN payloads aside
    npv = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(npv)
    assert np.array_equal(ours[fin].view(np.uint32), npv[fin].view(np.uint32))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(5000) * 1e-3, rng.standard_normal(5000) * 1e-6,
                        rng.standard_normal(2000) * 3e4, [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.1e-5]]).astype(np.float32)
    ours = np.array([orc.L.or_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(ours, x.astype(np.float16).view(np.uint16))


def test_bf16(orc, ref):
    h = np.random.default_rng(1).integers(0, 65536, 4096).astype(np.uint16)
    for v in h:
        a, b = orc.L.or_bf16_to_f32(int(v)), ref.L.ref_host_bf16f32(int(v))
        assert np.float32(a).tobytes() == np.float32(b).tobytes() or (math.isnan(a) and math.isnan(b))


def test_scale_unpack_forms(orc, ref):
    rng = np.random.default_rng(2)
    for _ in range(300):
        s = rng.integers(0, 256, 12).astype(np.uint8)
        sc_w, mn_w = np.zeros(8, np.uint8), np.zeros(8, np.uint8)
        orc.L.or_unpack_scales_words(P(s), P(sc_w), P(mn_w))
        sc_np, mn_np = kq.unpack_scales(s)
        assert np.array_equal(sc_w, sc_np) and np.array_equal(mn_w, mn_np)
        for j in range(8):
            a, b = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
            c_, d_ = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
            orc.L.or_scale_min_k4(j, P(s), P(a), P(b))
            ref.L.ref_get_scale_min_k4(j, P(s), P(c_), P(d_))
            assert a[0] == c_[0] == sc_w[j] and b[0] == d_[0] == mn_w[j]


# --------------------------------------------------------------------------
# dequantizers
# --------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", [12, 13, 14])
def test_dequant_bitexact_and_exact(orc, ref, qtype):
    blk = _subnormal_d(_blocks(qtype, 64, 256, 10 + qtype), qtype)
    bs = synth.BLOCK_BYTES[qtype]
    flat = blk.reshape(-1, bs)
    ours = orc.dequant(blk, qtype, 256)
    theirs = np.empty_like(ours)
    for b in range(flat.shape[0]):
        ref.L.ref_dequant_block(P(flat) + b * bs, qtype, P(theirs) + b * 1024)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    # float64 decoding of the format: products are exact, only the fp32
    # roundings of d*sc (and -m) differ, so agreement is to a few ulp
    ex = kq.dequant_f64(flat, qtype)
    assert np.allclose(ours, ex, rtol=5e-7, atol=1e-12)


# --------------------------------------------------------------------------
# Q8_K quantization
# --------------------------------------------------------------------------
def _q8_edge_inputs():
    rng = np.random.default_rng(3)
    cases = [rng.standard_normal(2560).astype(np.float32)]
    z = np.zeros(512, np.float32)
    z[256 + 7] = 1.0                              # zero block then a one-hot
    cases.append(z)
    t = rng.standard_normal(256).astype(np.float32)
    t[10], t[20] = 3.0, -3.0                     # equal |x|, opposite signs: first wins
    cases.append(t)
    t = rng.standard_normal(256).astype(np.float32)
    t[5], t[6] = -3.0, 3.0
    cases.append(t)
    h = np.zeros(256, np.float32)                # exact .5 after scaling: -127/127*(k+0.5)
    h[0] = 127.0
    h[1:40] = np.arange(39, dtype=np.float32) - 19.5
    cases.append(h)
    c = (rng.standard_normal(256) * 1e-30).astype(np.float32)   # tiny values
    cases.append(c)
    big = rng.standard_normal(256).astype(np.float32)
    big[0] = -big[np.argmax(np.abs(big))] * 1.0000001 if big[0] == 0 else big[0]
    cases.append(big)
    return cases


def test_quantize_q8K_matches_reference_variants(orc, ref):
    for x in _q8_edge_inputs():
        a = orc.quantize_q8K(x)
        b = np.zeros_like(a)
        c = np.zeros_like(a)
        ref.L.ref_quantize_row_q8_K(P(x), P(b), x.size)
        ref.L.ref_quantize_row_q8_K_ref(P(x), P(c), x.size)
        assert a.tobytes() == b.tobytes() == c.tobytes()


def test_quantize_q8K_closed_form(orc):
    for x in _q8_edge_inputs():
        a = orc.quantize_q8K(x)
        d, qs, bsums = kq.q8_quantize_np(x)
        assert np.array_equal(a["qs"], qs)
        assert np.array_equal(a["bsums"], bsums)
        assert np.array_equal(a["d"].view(np.uint32), d.view(np.uint32))
    # d is negative for a positive maximum (d = 1/(-127/maxv))
    a = orc.quantize_q8K(np.full(256, 2.0, np.float32))
    assert a["d"][0] < 0 and (a["qs"] == -127).all()


# --------------------------------------------------------------------------
# Q4_K / Q5_K x Q8_K dots
# --------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", [12, 13])
@pytest.mark.parametrize("n", [256, 2560, 4096])
def test_kquant_dot_bitexact(orc, ref, qtype, n):
    rows = 48
    blk = _subnormal_d(_blocks(qtype, rows, n, 100 + n + qtype), qtype)
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    q8 = orc.quantize_q8K(x)
    bs = synth.BLOCK_BYTES[qtype]
    f_or = orc.L.or_vec_dot_q4K_q8K if qtype == 12 else orc.L.or_vec_dot_q5K_q8K
    f_ref = ref.L.ref_vec_dot_q4_K_q8_K if qtype == 12 else ref.L.ref_vec_dot_q5_K_q8_K
    g_or = orc.L.or_vec_dot_q4K_q8K_generic if qtype == 12 else orc.L.or_vec_dot_q5K_q8K_generic
    g_ref = ref.L.ref_vec_dot_q4_K_q8_K_generic if qtype == 12 else ref.L.ref_vec_dot_q5_K_q8_K_generic
    for r in range(rows):
        rp = P(blk) + r * (n // 256) * bs
        a, b = f_or(n, rp, P(q8)), f_ref(n, rp, P(q8))
        assert np.float32(a).tobytes() == np.float32(b).tobytes(), (r, a, b)
        a, b = g_or(n, rp, P(q8)), g_ref(n, rp, P(q8))
        assert np.float32(a).tobytes() == np.float32(b).tobytes(), (r, a, b)


@pytest.mark.parametrize("qtype", [12, 13])
def test_kquant_block_sums_exact(orc, qtype):
    n = 2560
    blk = _blocks(qtype, 16, n, 7 + qtype)
    x = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    q8 = orc.quantize_q8K(x)
    bs = synth.BLOCK_BYTES[qtype]
    f = orc.L.or_q4K_block_SM if qtype == 12 else orc.L.or_q5K_block_SM
    for r in range(16):
        rb = blk[r].reshape(-1, bs)
        S_np, M_np = kq.kquant_block_sums(rb, qtype, q8)
        for b in range(n // 256):
            S, M = np.zeros(1, np.int32), np.zeros(1, np.int32)
            f(P(rb) + b * bs, P(q8) + b * 292, P(S), P(M))
            assert S[0] == S_np[b] and M[0] == M_np[b]
        # fp32 dot within 1e-5 of the float64 value, normalised by sum |terms|
        v, mag = kq.kquant_dot_f64(rb, qtype, q8)
        got = (orc.L.or_vec_dot_q4K_q8K if qtype == 12 else orc.L.or_vec_dot_q5K_q8K)(n, P(rb), P(q8))
        assert abs(got - v) <= 1e-5 * mag


def test_q6K_q8K_block_sum_exact(orc):
    n = 2560
    blk = _blocks(14, 8, n, 77)
    x = np.random.default_rng(78).standard_normal(n).astype(np.float32)
    q8 = orc.quantize_q8K(x)
    for r in range(8):
        rb = blk[r].reshape(-1, 210)
        S_np, _ = kq.kquant_block_sums(rb, 14, q8)
        for b in range(n // 256):
            assert orc.L.or_q6K_block_S(P(rb) + b * 210, P(q8) + b * 292) == S_np[b]
        v, mag = kq.kquant_dot_f64(rb, 14, q8)
        assert abs(orc.L.or_vec_dot_q6K_q8K(n, P(rb), P(q8)) - v) <= 1e-5 * mag


# --------------------------------------------------------------------------
# GEMV row drivers
# --------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", [12, 14])
def test_mm_quant_rows_bitexact(orc, ref, qtype):
    n, d = 2560, 96
    w = _blocks(qtype, d, n, 31 + qtype)
    x = np.random.default_rng(32).standard_normal(n).astype(np.float32)
    ours = orc.mm_quant_rows(x, w, n, d, qtype)
    theirs = np.empty(d, np.float32)
    ref.L.ref_mm_quant_rows(P(theirs), P(x), P(w), n, d, qtype)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    W = kq.dequant_f64(w.reshape(-1, synth.BLOCK_BYTES[qtype]), qtype).reshape(d, n)
    ex = W @ x.astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    assert (np.abs(ours - ex) <= 1e-5 * mag).all()


def test_mm_quant_dot_rows_bitexact(orc, ref):
    n, d = 2560, 64
    w = _blocks(12, d, n, 41)
    x = np.random.default_rng(42).standard_normal(n).astype(np.float32)
    q8 = orc.quantize_q8K(x)
    ours = orc.mm_quant_dot_rows(w, n, d, 12, q8)
    theirs = np.empty(d, np.float32)
    ref.L.ref_mm_quant_dot_rows(P(theirs), P(w), n, d, 12, P(q8))
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_mm_bf16_bitexact(orc, ref):
    n, d = 2560, 64
    rng = np.random.default_rng(51)
    w = synth.rand_bf16(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    ours = orc.mm_bf16(x, w, n, d)
    theirs = np.empty(d, np.float32)
    ref.L.ref_mm_bf16(P(theirs), P(x), P(w), n, d)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    W = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ex = W @ x
    assert (np.abs(ours - ex) <= 1e-5 * (np.abs(W) @ np.abs(x))).all()


# --------------------------------------------------------------------------
# norms, softmax, gelu, RoPE, embeddings
# --------------------------------------------------------------------------
def test_norms_bitexact(orc, ref):
    rng = np.random.default_rng(61)
    for n in (256, 2560, 10240):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        w = rng.uniform(0.5, 1.5, n).astype(np.float32)
        a, b = np.empty_like(x), np.empty_like(x)
        orc.L.or_rmsnorm(P(a), P(x), P(w), n, 1e-6)
        ref.L.ref_rmsnorm(P(b), P(x), P(w), n, 1e-6)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        ex = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * w
        assert np.allclose(a, ex, rtol=2e-6)
    for hd, nh in ((256, 8), (512, 2)):
        v = rng.standard_normal(nh * hd).astype(np.float32)
        w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        a, b = v.copy(), v.copy()
        orc.L.or_rmsnorm_head_inplace(P(a), P(w), nh, hd, 1e-6)
        ref.L.ref_rmsnorm_head_inplace(P(b), P(w), nh, hd, 1e-6)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        a, b = v.copy(), v.copy()
        orc.L.or_rmsnorm_head_noweight_inplace(P(a), nh, hd, 1e-6)
        ref.L.ref_rmsnorm_head_noweight_inplace(P(b), nh, hd, 1e-6)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        vv = v.reshape(nh, hd).astype(np.float64)
        ex = vv / np.sqrt((vv ** 2).mean(-1, keepdims=True) + 1e-6)
        assert np.allclose(a.reshape(nh, hd), ex, rtol=2e-6)


def test_softmax_gelu_bitexact(orc, ref):
    rng = np.random.default_rng(71)
    for n in (1, 7, 512, 4096):
        x = (rng.standard_normal(n) * 8).astype(np.float32)
        a, b = x.copy(), x.copy()
        orc.L.or_softmax(P(a), n)
        ref.L.ref_softmax(P(b), n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        e = np.exp(x.astype(np.float64) - x.max())
        assert np.allclose(a, e / e.sum(), rtol=1e-5, atol=1e-12)
    xs = np.concatenate([rng.standard_normal(20000) * 4, np.linspace(-20, 20, 4001)]).astype(np.float32)
    for v in xs:
        a, b = orc.L.or_gelu(float(v)), ref.L.ref_gelu(float(v))
        assert np.float32(a).tobytes() == np.float32(b).tobytes()
    xd = xs.astype(np.float64)
    ex = 0.5 * xd * (1 + np.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    got = np.array([orc.L.or_gelu(float(v)) for v in xs[:2000]])
    assert np.allclose(got, ex[:2000], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("hd,n_rot,base,use_ff", [(256, 256, 1e4, False), (512, 512, 1e6, True), (512, 512, 1e6, False)])
def test_rope_bitexact(orc, ref, hd, n_rot, base, use_ff):
    rng = np.random.default_rng(81)
    nh = 8
    ff = rng.uniform(1.0, 8.0, n_rot // 2).astype(np.float32) if use_ff else None
    for pos in (0, 1, 2, 511, 4095, 32767):
        v = rng.standard_normal(nh * hd).astype(np.float32)
        a = orc.rope(v, nh, hd, n_rot, pos, base, ff)
        b = v.copy()
        ref.L.ref_apply_rope_neox(P(b), nh, hd, n_rot, pos, base, 1.0, None if ff is None else P(ff))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), pos
        # rotation preserves each pair's norm
        va, vb = v.reshape(nh, hd), a.reshape(nh, hd)
        half = hd // 2
        n0 = va[:, :half] ** 2 + va[:, half:] ** 2
        n1 = vb[:, :half].astype(np.float64) ** 2 + vb[:, half:].astype(np.float64) ** 2
        assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
        if pos == 0:
            assert np.array_equal(a, v)


def test_rope_toy_example(orc):
    """design.md:969-986: hd=4, n_rot=4, base 1e4, pos=1; pairs (0,2),(1,3);
    pair 0 rotates by pos, pair 1 by pos*base^(-2/n_rot)."""
    a, b, c, d = 0.3, -1.2, 0.7, 2.0
    out = orc.rope(np.array([a, b, c, d], np.float32), 1, 4, 4, 1, 1e4)
    t0, t1 = 1.0, 1.0 * 1e4 ** (-0.5)
    ex = [a * math.cos(t0) - c * math.sin(t0), b * math.cos(t1) - d * math.sin(t1),
          a * math.sin(t0) + c * math.cos(t0), b * math.sin(t1) + d * math.cos(t1)]
    assert np.allclose(out, ex, rtol=1e-6, atol=1e-7)
    # the adjacent-pair (wrong) convention gives a different answer
    wrong = [a * math.cos(t0) - b * math.sin(t0), a * math.sin(t0) + b * math.cos(t0)]
    assert not np.allclose(out[:2], wrong, atol=1e-3)


def test_emb_lookup_bitexact(orc, ref):
    dim, vocab = 2560, 32
    w = _blocks(14, vocab, dim, 91)
    for tok in (0, 5, 31):
        a = np.empty(dim, np.float32)
        b = np.empty(dim, np.float32)
        assert orc.L.or_emb_lookup(P(a), P(w), 14, tok, dim) == 0
        ref.L.ref_emb_lookup(P(b), P(w), 14, tok, dim)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_sampler_matches_reference(orc, ref):
    rng = np.random.default_rng(101)
    for trial in range(40):
        n = 1000
        logits = (rng.standard_normal(n) * 3).astype(np.float32)
        if trial % 5 == 0:
            logits[17] = logits[400] = logits.max() + 1   # tie: first index wins
        temp = [0.0, 0.6, 1.0, 1.3][trial % 4]
        topp = [0.9, 1.0, 0.5, 0.0][trial % 4]
        s1 = np.array([trial + 1], np.uint64)
        s2 = s1.copy()
        la, lb = logits.copy(), logits.copy()
        a = orc.L.or_sample_token(P(la), n, temp, topp, 40, P(s1))
        b = ref.L.ref_sample_token(P(lb), n, temp, topp, 40, P(s2))
        assert a == b and s1[0] == s2[0]
        if temp == 0.0 and trial % 5 == 0:
            assert a == 17


def test_layer_routing_table(ref):
    """ISWA map of design.md:841-860 as a known-answer table."""
    full = {5, 11, 17, 23, 29, 35, 41}
    for l in range(42):
        swa = l not in full
        assert ref.L.ref_is_swa_layer(42, 6, l) == int(swa)
        src = l if l < 24 else (22 if swa else 23)
        assert ref.L.ref_kv_source_for_layer(42, 6, l) == src
        assert ref.L.ref_layer_head_dim(42, 6, 256, 512, l) == (256 if swa else 512)
    assert synth.E4B.is_swa(5) is False and synth.E4B.is_swa(4) is True


# --------------------------------------------------------------------------
# attention block (OpenBLAS absent: brute force in float64 pins it)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("hd,t_start,nwin,scale", [(256, 0, 1, 1.0), (256, 0, 37, 1.0), (256, 100, 512, 1 / 16),
                                                    (512, 0, 300, 1.0)])
def test_attention_block_bruteforce(orc, hd, t_start, nwin, scale):
    rng = np.random.default_rng(hd + nwin)
    nh, nkv, stride = 8, 2, 1024
    T = t_start + nwin
    kc = rng.standard_normal((T, stride)).astype(np.float32)
    vc = rng.standard_normal((T, stride)).astype(np.float32)
    q = (rng.standard_normal(nh * hd) * 0.1).astype(np.float32)
    out = orc.attn(q, kc, vc, stride, t_start, nwin, nh, nkv, hd, scale)
    for h in range(nh):
        kvh = h // (nh // nkv)
        K = kc[t_start:T, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        V = vc[t_start:T, kvh * hd:(kvh + 1) * hd].astype(np.float64)
        s = scale * (K @ q[h * hd:(h + 1) * hd].astype(np.float64))
        p = np.exp(s - s.max())
        p /= p.sum()
        ex = p @ V
        assert np.allclose(out[h * hd:(h + 1) * hd], ex, rtol=1e-4, atol=1e-5 * np.abs(ex).max())
        if nwin == 1:   # single token: output is that token's V row
            assert np.allclose(out[h * hd:(h + 1) * hd], V[0], rtol=1e-6)
