"""Independent numpy decoding of the K-quant block formats, for brute-force checks.

Formats as stored by GGUF (gemma4-4b/cpu-blas/main.c:94-122): Q4_K 144 B
(d, dmin, scales[12], qs[128]), Q5_K 176 B (+ qh[32] before qs), Q6_K 210 B
(ql[128], qh[64], int8 scales[16], d).  Everything here is exact integer
arithmetic or float64, so it pins sums and orderings without sharing code
with the C oracle.
"""
import numpy as np


def f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float64)


def unpack_scales(s12: np.ndarray):
    s = s12.astype(np.int64)
    sc = np.empty(s.shape[:-1] + (8,), np.int64)
    mn = np.empty_like(sc)
    for j in range(4):
        sc[..., j] = s[..., j] & 63
        mn[..., j] = s[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
        mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    return sc, mn


def q4_values(blk: np.ndarray) -> np.ndarray:
    """[..., 144] -> [..., 256] nibble values 0..15 in weight order."""
    qs = blk[..., 16:144].astype(np.int64)
    out = np.empty(blk.shape[:-1] + (256,), np.int64)
    for c in range(4):
        out[..., 64 * c:64 * c + 32] = qs[..., 32 * c:32 * c + 32] & 15
        out[..., 64 * c + 32:64 * c + 64] = qs[..., 32 * c:32 * c + 32] >> 4
    return out


def q5_values(blk: np.ndarray) -> np.ndarray:
    qh = blk[..., 16:48].astype(np.int64)
    qs = blk[..., 48:176].astype(np.int64)
    out = np.empty(blk.shape[:-1] + (256,), np.int64)
    for c in range(4):
        out[..., 64 * c:64 * c + 32] = (qs[..., 32 * c:32 * c + 32] & 15) + 16 * ((qh >> (2 * c)) & 1)
        out[..., 64 * c + 32:64 * c + 64] = (qs[..., 32 * c:32 * c + 32] >> 4) + 16 * ((qh >> (2 * c + 1)) & 1)
    return out


def q6_values_scales(blk: np.ndarray):
    """[..., 210] -> (q6-32 values [...,256], per-weight int8 scale [...,256])."""
    ql = blk[..., 0:128].astype(np.int64)
    qh = blk[..., 128:192].astype(np.int64)
    sc = blk[..., 192:208].view(np.int8).astype(np.int64)
    q = np.empty(blk.shape[:-1] + (256,), np.int64)
    s = np.empty_like(q)
    for h in range(2):
        for l in range(32):
            hb = qh[..., 32 * h + l]
            base = 128 * h + l
            q[..., base + 0] = (ql[..., 64 * h + l] & 15) | (((hb >> 0) & 3) << 4)
            q[..., base + 32] = (ql[..., 64 * h + 32 + l] & 15) | (((hb >> 2) & 3) << 4)
            q[..., base + 64] = (ql[..., 64 * h + l] >> 4) | (((hb >> 4) & 3) << 4)
            q[..., base + 96] = (ql[..., 64 * h + 32 + l] >> 4) | (((hb >> 6) & 3) << 4)
            for k in range(4):
                s[..., base + 32 * k] = sc[..., 8 * h + l // 16 + 2 * k]
    return q - 32, s


def q8_quantize_np(x: np.ndarray):
    """Closed form of absmax-symmetric Q8_K over 256-blocks (float32 math)."""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    qs = np.zeros(x.shape, np.int8)
    d = np.zeros(x.shape[0], np.float32)
    for b in range(x.shape[0]):
        ax = np.abs(x[b])
        j = int(np.argmax(ax))          # first index of the maximum
        if ax[j] == 0:
            continue
        iscale = np.float32(-127.0) / x[b, j]
        v = np.rint(iscale * x[b]).astype(np.int64)   # rint: round half to even
        qs[b] = np.minimum(v, 127).astype(np.int8)
        d[b] = np.float32(1.0) / iscale
    bsums = qs.astype(np.int64).reshape(-1, 16, 16).sum(-1).astype(np.int16)
    return d, qs, bsums


def kquant_block_sums(blk: np.ndarray, qtype: int, q8) -> tuple:
    """Exact S_b and M_b for blocks [nb, bytes] against Q8_K blocks (structured array)."""
    qs8 = q8["qs"].astype(np.int64)
    if qtype == 14:
        q, s = q6_values_scales(blk)
        return (s * q * qs8).sum(-1), np.zeros(blk.shape[0], np.int64)
    vals = q4_values(blk) if qtype == 12 else q5_values(blk)
    sc, mn = unpack_scales(blk[..., 4:16])
    prod = (vals * qs8).reshape(-1, 8, 32).sum(-1)
    S = (sc * prod).sum(-1)
    M = (q8["bsums"].astype(np.int64) * np.repeat(mn, 2, axis=-1)).sum(-1)
    return S, M


def kquant_dot_f64(blk_row: np.ndarray, qtype: int, q8):
    """Float64 value of the Q8_K dot and sum of |terms| (for normalised errors)."""
    S, M = kquant_block_sums(blk_row, qtype, q8)
    yd = q8["d"].astype(np.float64)
    if qtype == 14:
        d = f16(blk_row[:, 208:210].copy().view(np.uint16)[:, 0])
        t = d * yd * S
        return t.sum(), np.abs(t).sum()
    d = f16(blk_row[:, 0:2].copy().view(np.uint16)[:, 0])
    dm = f16(blk_row[:, 2:4].copy().view(np.uint16)[:, 0])
    t1 = d * yd * S
    t2 = dm * yd * M
    return (t1 - t2).sum(), (np.abs(t1) + np.abs(t2)).sum()


def dequant_f64(blk: np.ndarray, qtype: int) -> np.ndarray:
    """[nb, bytes] -> float64 weights [nb*256] (exact products in float64)."""
    if qtype == 14:
        q, s = q6_values_scales(blk)
        d = f16(blk[:, 208:210].copy().view(np.uint16)[:, 0])[:, None]
        return (d * s * q).reshape(-1)
    vals = q4_values(blk) if qtype == 12 else q5_values(blk)
    sc, mn = unpack_scales(blk[..., 4:16])
    d = f16(blk[:, 0:2].copy().view(np.uint16)[:, 0])[:, None]
    dm = f16(blk[:, 2:4].copy().view(np.uint16)[:, 0])[:, None]
    w = d * np.repeat(sc, 32, -1) * vals - dm * np.repeat(mn, 32, -1)
    return w.reshape(-1)


def _q6_abs_values(blk: np.ndarray) -> np.ndarray:
    """[nb, 210] -> |q6 - 32| as float32 [nb, 256] in weight order (vectorised
    form of q6_values_scales' layout)"""
    ql = blk[:, 0:128]
    qh = blk[:, 128:192]
    q = np.empty((blk.shape[0], 256), np.int16)
    for h in range(2):
        lo, hi, b = ql[:, 64 * h:64 * h + 32], ql[:, 64 * h + 32:64 * h + 64], qh[:, 32 * h:32 * h + 32]
        base = 128 * h
        q[:, base + 0:base + 32] = (lo & 15) | ((b & 3) << 4)
        q[:, base + 32:base + 64] = (hi & 15) | (((b >> 2) & 3) << 4)
        q[:, base + 64:base + 96] = (lo >> 4) | (((b >> 4) & 3) << 4)
        q[:, base + 96:base + 128] = (hi >> 4) | (((b >> 6) & 3) << 4)
    return np.abs(q - 32).astype(np.float32)


def abs_dot_rows(raw: np.ndarray, qtype: int, n: int, x: np.ndarray, chunk: int = 4096) -> np.ndarray:
    """sum_i |w_ri| * |x_i| per row of a d x n K-quant matrix (raw bytes), in
    row chunks so that large matrices (the 262144-row LM head) stay within
    memory; the normaliser of the fp32 GEMV bars.  Q6_K: the 16-weight
    sub-block s of a block uses scale s in weight order, so per block
    |d| * sum_s |sc_s| * sum_{i in s} |q_i - 32| |x_i|."""
    bpb = {12: 144, 13: 176, 14: 210}[qtype]
    nb = n // 256
    rows = raw.reshape(-1, nb * bpb)
    ax = np.abs(np.asarray(x, np.float64))
    out = np.empty(rows.shape[0], np.float64)
    for r0 in range(0, rows.shape[0], chunk):
        blk = rows[r0:r0 + chunk].reshape(-1, bpb)
        if qtype == 14:
            A = _q6_abs_values(blk).reshape(-1, nb, 16, 16)
            T = np.einsum("rbst,bst->rbs", A, ax.astype(np.float32).reshape(nb, 16, 16), dtype=np.float64)
            sc = np.abs(blk[:, 192:208].view(np.int8).astype(np.float64)).reshape(-1, nb, 16)
            d = np.abs(f16(blk[:, 208:210].copy().view(np.uint16)[:, 0])).reshape(-1, nb)
            out[r0:r0 + chunk] = (d * (sc * T).sum(-1)).sum(-1)
        else:
            w = np.abs(dequant_f64(blk, qtype)).reshape(-1, n)
            out[r0:r0 + chunk] = w @ ax
    return out


def abs_terms_q8(raw: np.ndarray, qtype: int, n: int, q8rows) -> np.ndarray:
    """[d, m] sum of |terms| of the Q4_K / Q5_K x Q8_K dot of every row with
    every Q8_K row (q8rows: BlockQ8_K [m, n/256]): per block
    |y.d| * (|d| * sum_e sc_j(e) * q_e * |q8_e| + |dmin| * sum_j m_j * |bs_j|),
    the scale of the fp32 rounding in any order of the partial sums."""
    bpb = {12: 144, 13: 176}[qtype]
    nb = n // 256
    blk = raw.reshape(-1, bpb)
    vals = (q4_values(blk) if qtype == 12 else q5_values(blk)).astype(np.float64)
    sc, mn = unpack_scales(blk[..., 4:16])
    d = np.abs(f16(blk[:, 0:2].copy().view(np.uint16)[:, 0]))[:, None]
    dm = np.abs(f16(blk[:, 2:4].copy().view(np.uint16)[:, 0]))[:, None]
    A = (d * np.repeat(sc, 32, -1) * vals).reshape(-1, n)                 # [d, n]
    C = (dm * np.repeat(mn, 2, -1)).reshape(-1, nb * 16)                  # [d, nb*16]
    yd = np.abs(q8rows["d"].astype(np.float64))                           # [m, nb]
    B = (np.abs(q8rows["qs"].astype(np.float64)) * yd[..., None]).reshape(-1, n)
    D = (np.abs(q8rows["bsums"].astype(np.float64)) * yd[..., None]).reshape(-1, nb * 16)
    return A @ B.T + C @ D.T
