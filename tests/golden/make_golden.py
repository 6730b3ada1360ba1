"""Write tests/golden/ref_vectors.npz: inputs and outputs of the reference's
own hot-path functions (gemma4-4b/cpu-blas/main.c, compiled unchanged into
oracle/_ref/libg4ref.so by oracle/Makefile) on small seeded inputs.

The fixtures let tests/test_golden.py pin the CPU oracle bit for bit on any
machine, with or without the reference tree.  Run from the repository root
after `make -C oracle`:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "gemma4.c_amd")]

import oracle  # noqa: E402
import synth  # noqa: E402

P = lambda a: a.ctypes.data  # noqa: E731


def q8_inputs(rng):
    xs = [rng.standard_normal(2560).astype(np.float32)]
    z = np.zeros(512, np.float32)
    z[256 + 7] = 1.0
    xs.append(z)
    t = rng.standard_normal(256).astype(np.float32)
    t[10], t[20] = 3.0, -3.0
    xs.append(t)
    h = np.zeros(256, np.float32)
    h[0] = 127.0
    h[1:40] = np.arange(39, dtype=np.float32) - 19.5
    xs.append(h)
    xs.append((rng.standard_normal(256) * 1e-30).astype(np.float32))
    xs.append((rng.standard_normal(768) * 40).astype(np.float32))
    return np.concatenate(xs), np.cumsum([0] + [x.size for x in xs]).astype(np.int64)


def main() -> None:
    if not oracle.Ref.available():
        sys.exit("oracle/_ref/libg4ref.so is not built (make -C oracle with the reference tree present)")
    ref = oracle.Ref()
    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # quantize_row_q8_K (AVX2, main.c:282) and quantize_row_q8_K_ref (main.c:247)
    x, offs = q8_inputs(rng)
    y_avx = np.zeros(x.size // 256, oracle.Q8K_DTYPE)
    y_ref = np.zeros_like(y_avx)
    ref.L.ref_quantize_row_q8_K(P(x), P(y_avx), x.size)
    ref.L.ref_quantize_row_q8_K_ref(P(x), P(y_ref), x.size)
    out.update(q8_x=x, q8_offs=offs, q8_avx=y_avx.view(np.uint8), q8_ref=y_ref.view(np.uint8))

    # K-quant dots, both fp32 orders (main.c:347-593), on 12 rows of 2560
    xa = rng.standard_normal(2560).astype(np.float32)
    q8 = np.zeros(10, oracle.Q8K_DTYPE)
    ref.L.ref_quantize_row_q8_K(P(xa), P(q8), 2560)
    out["dot_q8"] = q8.view(np.uint8)
    for qt, name in ((12, "q4K"), (13, "q5K")):
        raw = synth.rand_kquant(rng, qt, 12, 2560)
        raw[0, 0:2] = np.array([3, 0], np.uint8)          # an fp16 subnormal d (main.c:133-140)
        bs = synth.BLOCK_BYTES[qt]
        avx = np.array([ref.L.ref_vec_dot_q4_K_q8_K(2560, P(raw) + r * 10 * bs, P(q8)) if qt == 12 else
                        ref.L.ref_vec_dot_q5_K_q8_K(2560, P(raw) + r * 10 * bs, P(q8)) for r in range(12)], np.float32)
        gen = np.array([ref.L.ref_vec_dot_q4_K_q8_K_generic(2560, P(raw) + r * 10 * bs, P(q8)) if qt == 12 else
                        ref.L.ref_vec_dot_q5_K_q8_K_generic(2560, P(raw) + r * 10 * bs, P(q8)) for r in range(12)],
                       np.float32)
        mmd = np.empty(12, np.float32)
        ref.L.ref_mm_quant_dot_rows(P(mmd), P(raw), 2560, 12, qt, P(q8))
        out.update({f"dot_{name}_w": raw, f"dot_{name}_avx": avx, f"dot_{name}_generic": gen, f"mmdot_{name}": mmd})

    # mm_quant_rows (Q6_K, fp32 activation, main.c:1539-1556)
    raw6 = synth.rand_q6K(rng, 8, 2560)
    x6 = rng.standard_normal(2560).astype(np.float32)
    o6 = np.empty(8, np.float32)
    ref.L.ref_mm_quant_rows(P(o6), P(x6), P(raw6), 2560, 8, 14)
    out.update(mmq6_w=raw6, mmq6_x=x6, mmq6_o=o6)

    # mm_bf16 (main.c:1529-1537)
    wb = synth.rand_bf16(rng, 8, 512)
    xb = rng.standard_normal(512).astype(np.float32)
    ob = np.empty(8, np.float32)
    ref.L.ref_mm_bf16(P(ob), P(xb), P(wb), 512, 8)
    out.update(bf16_w=wb, bf16_x=xb, bf16_o=ob)

    # dequantizers (main.c:172-237, 767-776), incl. subnormal d
    for qt, name in ((12, "q4K"), (13, "q5K"), (14, "q6K")):
        raw = synth.rand_kquant(rng, qt, 1, 1024).reshape(-1)
        bs = synth.BLOCK_BYTES[qt]
        off = 208 if qt == 14 else 0
        raw[off:off + 2] = np.array([0xff, 0x03], np.uint8)
        deq = np.empty(1024, np.float32)
        for b in range(4):
            ref.L.ref_dequant_block(P(raw) + b * bs, qt, P(deq) + b * 1024)
        out.update({f"deq_{name}_w": raw, f"deq_{name}_o": deq})

    # norms, softmax, gelu (main.c:1451-1492)
    xn = (rng.standard_normal(2560) * 3).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, 2560).astype(np.float32)
    on = np.empty(2560, np.float32)
    ref.L.ref_rmsnorm(P(on), P(xn), P(wn), 2560, 1e-6)
    vh = rng.standard_normal(8 * 256).astype(np.float32)
    wh = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    oh = vh.copy()
    ref.L.ref_rmsnorm_head_inplace(P(oh), P(wh), 8, 256, 1e-6)
    ohn = vh.copy()
    ref.L.ref_rmsnorm_head_noweight_inplace(P(ohn), 8, 256, 1e-6)
    xs = (rng.standard_normal(777) * 5).astype(np.float32)
    os_ = xs.copy()
    ref.L.ref_softmax(P(os_), 777)
    xg = np.concatenate([(rng.standard_normal(1000) * 4), [0.0, -0.0, 1e-20, -30.0, 30.0]]).astype(np.float32)
    og = np.array([ref.L.ref_gelu(float(v)) for v in xg], np.float32)
    out.update(norm_x=xn, norm_w=wn, norm_o=on, head_v=vh, head_w=wh, head_o=oh, headnw_o=ohn,
               softmax_x=xs, softmax_o=os_, gelu_x=xg, gelu_o=og)

    # apply_rope_neox (main.c:1725-1745)
    for tag, hd, base, use_ff in (("swa", 256, 1e4, False), ("full", 512, 1e6, True)):
        ff = rng.uniform(1.0, 8.0, hd // 2).astype(np.float32) if use_ff else np.zeros(0, np.float32)
        for pos in (0, 1, 511, 4095, 32767):
            v = rng.standard_normal(8 * hd).astype(np.float32)
            o = v.copy()
            ref.L.ref_apply_rope_neox(P(o), 8, hd, hd, pos, base, 1.0, P(ff) if use_ff else None)
            out[f"rope_{tag}_{pos}_x"] = v
            out[f"rope_{tag}_{pos}_o"] = o
        out[f"rope_{tag}_ff"] = ff

    # emb_lookup (main.c:1696-1723) of a Q6_K table
    te = synth.rand_q6K(rng, 4, 2560)
    oe = np.empty((4, 2560), np.float32)
    for t in range(4):
        ref.L.ref_emb_lookup(P(oe) + t * 2560 * 4, P(te), 14, t, 2560)
    out.update(emb_w=te, emb_o=oe)

    # sample_token (main.c:2035-2112): greedy and top-k/temperature/top-p draws
    lg = (rng.standard_normal(512) * 3).astype(np.float32)
    lg[[7, 300]] = lg.max() + 1.0          # a tie at the maximum: the first index wins
    draws = []
    for temp, topp, topk, seed in ((0.0, 1.0, 40, 1), (0.8, 0.95, 40, 42), (1.0, 1.0, 40, 7), (0.7, 0.5, 10, 99)):
        st = np.array([seed], np.uint64)
        toks = []
        for _ in range(8):
            work = lg.copy()          # sample_token may reorder its input; keep the copy alive
            toks.append(ref.L.ref_sample_token(P(work), 512, temp, topp, topk, P(st)))
        draws.append([temp, topp, topk, seed] + toks)
    out.update(sample_logits=lg, sample_draws=np.array(draws, np.float64))

    # apply_repetition_penalty (main.c:2114-2126): a 100-token history with
    # repeats (a token penalised twice or more), ids at either sign of the
    # logit, windows 64 / all / longer than the history, penalty 1.0 (no-op)
    hist = rng.integers(0, 512, 100).astype(np.int32)
    hist[[10, 50, 90, 95]] = 7
    hist[[60, 61]] = 300
    pen_out = []
    pen_cases = ((1.3, 64), (1.1, 0), (2.0, 200), (1.0, 64), (1.5, 5))
    for penalty, last_n in pen_cases:
        work = lg.copy()
        ref.L.ref_apply_repetition_penalty(P(work), P(hist), hist.size, penalty, last_n)
        pen_out.append(work)
    out.update(penalty_hist=hist, penalty_cases=np.array(pen_cases, np.float64), penalty_out=np.array(pen_out))

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
