#!/usr/bin/env python3
"""Benchmark of the Gemma 4 E4B decode-step hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads (synthetic inputs, generated from fixed seeds on the host):
  decode  full E4B-shape forward: 42 layers, hidden 2560, FFN 10240, vocab
          262144, Q4_K_M weight mix, random init; a step is one decode token
          (the default; the metric's workload)
  gemv    one Q4_K x Q8_K GEMV 10240x2560 (seed 0)
  layer   one E4B sliding-window layer's decode projections (Q|K|V, O,
          gate|up, down) as the engine launches them, and the Q5_K gate|up
          variant (seed 1)
  gateup  the fused gate|up GELU GEMV at its decode shape, Q4_K 2 x 10240x2560
          (seed 1): the decode's dominant kernel alone
  lmhead  tied LM head, Q6_K 262144x2560 times an fp32 hidden vector, with the
          30*tanh(l/30) soft-cap (seed 2)
  copy    a 64 MiB device copy: the practical HBM ceiling
  prefill batched prefill GEMM: 512 tokens through one E4B layer's Q4_K
          matrices on the matrix cores (seed 1)
  prefill_e2e  batched prompt prefill through the engine at the E4B shape:
          511 tokens in one chunk (seed 4); roofline on the Q6_K GEMM (V, FFN down)
  floors  probe kernels: a dependent launch with no work, streaming reads at
          14.8 / 29.5 / 551.6 MB, a last-workgroup hand-off inside a kernel
  attn    ISWA decode attention step (norms, RoPE, K/V append, attention):
          sliding ring 512 and global T = 4096 / 32768 at head_dim 256 and 512
          (seed 3); value: the global T=32768 hd 256 case

Prints ONE JSON line.  `value` is whole-job throughput with inputs resident
in HBM; `roofline` is the dominant kernel's algorithmic bytes over its average
launch time (HIP events on the library stream); `cpu_baseline` times the
reference CPU path on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "gemma4.c_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 512 << 20        # rotate through this many distinct bytes to defeat the 256 MB Infinity Cache
METRIC = "decode tok/s at E4B shape (1 GPU); K-quant GEMV GB/s as % of HBM peak"


def cpu_threads() -> int:
    """OpenMP threads of the CPU leg: OMP_NUM_THREADS (16 on the GPU boxes,
    the host-core share of one GPU there), else the usable cores."""
    v = os.environ.get("OMP_NUM_THREADS")
    if v and v.isdigit():
        return int(v)
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)


def cpu_host() -> dict:
    """lscpu's model, sockets and physical cores of the host, and the cores
    this process may use"""
    info = {"usable_cores": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(ln.split(":", 1) for ln in out.splitlines() if ":" in ln)
        g = lambda k: kv.get(k, "").strip()
        info["model"] = g("Model name")
        sockets, cps = int(g("Socket(s)") or 0), int(g("Core(s) per socket") or 0)
        info.update(sockets=sockets, physical_cores=sockets * cps, threads_per_core=int(g("Thread(s) per core") or 0))
    except Exception as e:                     # lscpu absent: the usable cores alone
        info["lscpu"] = f"unavailable ({e.__class__.__name__})"
    return info


def omp_threads(n: int) -> None:
    """set the OpenMP team size of the CPU leg's later parallel regions"""
    import ctypes
    try:
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
    except OSError:
        pass


class Timer:
    """HIP events on the library stream around a region."""

    def __init__(self, lib):
        self.lib = lib
        self.a, self.b = C.c_void_p(), C.c_void_p()
        lib.check(lib.L.g4_event_create(C.byref(self.a)))
        lib.check(lib.L.g4_event_create(C.byref(self.b)))

    def start(self):
        self.lib.check(self.lib.L.g4_event_record(self.a))

    def stop_ms(self) -> float:
        self.lib.check(self.lib.L.g4_event_record(self.b))
        ms = C.c_float()
        self.lib.check(self.lib.L.g4_event_elapsed_ms(self.a, self.b, C.byref(ms)))
        return ms.value


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE KiB per dispatch, each
    scaled by what the counter reads for a plain copy of known size)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        t = json.load(open(path))[kernel]
    except (OSError, KeyError, ValueError):
        return None
    return round(1024 * (t["fetch_kib"] * t["fetch_scale"] + t["write_kib"] * t["write_scale"]))


def roofline(bytes_per_launch: float, sec_per_launch: float, kernel: str = "") -> dict:
    gbs = bytes_per_launch / sec_per_launch / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel)}


# ---------------------------------------------------------------------------
# GEMV workloads
# ---------------------------------------------------------------------------
def _copies(nbytes: int) -> int:
    return max(2, -(-MALL_BYTES // nbytes))


GEMV_KERNEL = "gemv_q45_stream_kernel<Q4_K> 10240x2560"


def bench_gemv(lib, g4, synth, args):
    """Q4_K x Q8_K GEMV 10240x2560; rotates weight copies so every launch reads HBM."""
    n, d = 2560, 10240
    rng = np.random.default_rng(0)
    raw = synth.rand_q4K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    ncp = _copies(raw.nbytes)
    ws = [g4.upload_quant(lib, raw, g4.Q4_K, n, d) for _ in range(ncp)]
    xd = g4.DBuf.from_array(lib, x)
    q8 = g4.DBuf(lib, lib.L.g4_q8K_bytes(n))
    out = g4.DBuf(lib, 4 * d)
    lib.g4_quantize_row_q8_K(xd.ptr, q8.ptr, n)
    L = lib.L

    def step(i):
        L.g4_mm_quant_dot_rows(out.ptr, ws[i % ncp].ptr, n, d, g4.Q4_K, q8.ptr)

    launches = 1
    algo = raw.nbytes + lib.L.g4_q8K_bytes(n) + 4 * d
    ms = _time_steps(lib, step, args)
    per_launch = ms / 1e3 / args.steps / launches
    res = {
        "value": round(algo / per_launch / 1e9, 1), "unit": "GB/s", "higher_is_better": True,
        "ms_per_step": ms / args.steps, "dtype": "int8xu4->int32, fp32 combine",
        "config": {"workload": "Q4_K x Q8_K GEMV 10240x2560 (seed 0), batch 1", "rows": d, "n": n,
                   "weight_copies_rotated": ncp},
        "roofline": dict(roofline(algo, per_launch, GEMV_KERNEL), kernel=GEMV_KERNEL,
                         bytes_per_launch=algo),
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_gemv_baseline(raw, x, n, d, algo)
    return res


def cpu_gemv_baseline(raw, x, n, d, algo):
    import oracle as orc_mod
    thr = cpu_threads()
    if orc_mod.Ref.available():
        ref = orc_mod.Ref()
        kind = "reference"
        q8 = np.zeros(n // 256, orc_mod.Q8K_DTYPE)
        o = np.empty(d, np.float32)

        def run():
            ref.L.ref_quantize_row_q8_K(x.ctypes.data, q8.ctypes.data, n)
            ref.L.ref_mm_quant_dot_rows(o.ctypes.data, raw.ctypes.data, n, d, 12, q8.ctypes.data)
    else:
        orc = orc_mod.Oracle()
        kind = "port"

        def run():
            q8 = orc.quantize_q8K(x)
            orc.mm_quant_dot_rows(raw, n, d, 12, q8)
    for _ in range(3):
        run()
    ts = []
    t_end = time.perf_counter() + 10.0
    while time.perf_counter() < t_end or len(ts) < 20:
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    med = float(np.median(ts))
    return {"value": round(algo / med / 1e9, 2), "unit": "GB/s", "cores": thr, "kind": kind,
            "sample": f"quantize_row_q8_K + mm_quant_dot_rows (Q4_K 10240x2560), median of {len(ts)} runs "
                      f"after 3 warm-ups, OpenMP {thr} threads"}


def bench_layer(lib, g4, synth, args):
    """One E4B sliding-window layer's decode projections at batch 1 (seed 1),
    launched as the engine launches them: Q|K (Q4_K) and V (Q6_K) in one
    launch with the residual/norm/Q8_K prologue, O (Q4_K, Q8_K of the
    attention output ready), the fused gate|up GELU (Q4_K) and down (Q6_K on
    the fp32 hidden vector).  Weight copies rotated through >= 512 MB.  value:
    weight bytes over the four launches' time; config: each projection alone
    and the Q5_K gate|up variant."""
    n, hid, nq, nkv = 2560, 10240, 2048, 512
    rng = np.random.default_rng(1)
    raws = {"q": synth.rand_q4K(rng, nq, n), "k": synth.rand_q4K(rng, nkv, n),
            "v": synth.rand_kquant(rng, g4.Q6_K, nkv, n), "o": synth.rand_q4K(rng, n, nq),
            "gate": synth.rand_q4K(rng, hid, n), "up": synth.rand_q4K(rng, hid, n),
            "down": synth.rand_kquant(rng, g4.Q6_K, n, hid),
            "gate5": synth.rand_kquant(rng, g4.Q5_K, hid, n), "up5": synth.rand_kquant(rng, g4.Q5_K, hid, n)}
    shapes = {"q": (g4.Q4_K, n, nq), "k": (g4.Q4_K, n, nkv), "v": (g4.Q6_K, n, nkv), "o": (g4.Q4_K, nq, n),
              "gate": (g4.Q4_K, n, hid), "up": (g4.Q4_K, n, hid), "down": (g4.Q6_K, hid, n),
              "gate5": (g4.Q5_K, n, hid), "up5": (g4.Q5_K, n, hid)}
    layer_bytes = sum(raws[k].nbytes for k in ("q", "k", "v", "o", "gate", "up", "down"))
    ncp = _copies(layer_bytes + raws["gate5"].nbytes + raws["up5"].nbytes)
    W = [{k: g4.upload_quant(lib, raws[k], *shapes[k]) for k in raws} for _ in range(ncp)]
    vec = lambda m, s=1.0: g4.DBuf.from_array(lib, (rng.standard_normal(m) * s).astype(np.float32))
    x, y = vec(n), vec(n, 4.0)
    wpost = g4.DBuf.from_array(lib, rng.uniform(0.5, 1.5, n).astype(np.float32))
    wnext = g4.DBuf.from_array(lib, rng.uniform(0.5, 1.5, n).astype(np.float32))
    osc = g4.DBuf.from_array(lib, np.array([0.9], np.float32))
    attn, hb = vec(nq), vec(hid)
    xo, xb2 = g4.DBuf(lib, 4 * n), g4.DBuf(lib, 4 * n)
    q, k, v, o, hbo, down = (g4.DBuf(lib, 4 * m) for m in (nq, nkv, nkv, n, hid, n))
    q8 = g4.DBuf(lib, lib.L.g4_q8K_bytes(n))
    q8o = g4.DBuf(lib, lib.L.g4_q8K_bytes(nq))
    lib.g4_quantize_row_q8_K(attn.ptr, q8o.ptr, nq)
    lib.g4_quantize_row_q8_K(x.ptr, q8.ptr, n)
    eps = C.c_float(1e-6)
    L = lib.L

    def qkv(i):
        w = W[i % ncp]
        L.g4_mm_residual_q8_qkv(q.ptr, w["q"].ptr, nq, k.ptr, w["k"].ptr, nkv, v.ptr, w["v"].ptr, nkv, g4.Q6_K, n,
                                g4.Q4_K, x.ptr, xo.ptr, y.ptr, wpost.ptr, osc.ptr, wnext.ptr, xb2.ptr, None, eps)

    def oproj(i):
        L.g4_mm_quant_dot_rows(o.ptr, W[i % ncp]["o"].ptr, nq, n, g4.Q4_K, q8o.ptr)

    def gateup(i, sfx=""):
        w = W[i % ncp]
        L.g4_mm_gate_up_gelu(hbo.ptr, w["gate" + sfx].ptr, w["up" + sfx].ptr, n, hid,
                             g4.Q5_K if sfx else g4.Q4_K, q8.ptr)

    def dproj(i):
        L.g4_mm_quant_rows(down.ptr, hb.ptr, W[i % ncp]["down"].ptr, hid, n, g4.Q6_K)

    def layer(i):
        qkv(i)
        oproj(i)
        gateup(i)
        dproj(i)

    class A:
        warmup, steps = args.warmup, args.steps
    ms = _time_steps(lib, layer, A)
    per = ms / 1e3 / args.steps
    parts = {}
    for name, f, b in (("q|k|v", qkv, raws["q"].nbytes + raws["k"].nbytes + raws["v"].nbytes),
                       ("o", oproj, raws["o"].nbytes), ("gate|up", gateup, raws["gate"].nbytes + raws["up"].nbytes),
                       ("down", dproj, raws["down"].nbytes),
                       ("gate|up Q5_K", lambda i: gateup(i, "5"), raws["gate5"].nbytes + raws["up5"].nbytes)):
        t = _time_steps(lib, f, A) / 1e3 / args.steps
        parts[name] = {"us": round(t * 1e6, 2), "weight_bytes": b, "GBps": round(b / t / 1e9, 1)}
    q5_bytes = layer_bytes - raws["gate"].nbytes - raws["up"].nbytes + raws["gate5"].nbytes + raws["up5"].nbytes
    q5_per = per - parts["gate|up"]["us"] / 1e6 + parts["gate|up Q5_K"]["us"] / 1e6
    res = {"value": round(layer_bytes / per / 1e9, 1), "unit": "GB/s", "higher_is_better": True,
           "ms_per_step": ms / args.steps, "dtype": "int8xu4->int32 (Q4_K/Q5_K), fp32 (Q6_K)",
           "config": {"workload": "one E4B sliding-window layer's decode projections, batch 1 (seed 1): Q|K Q4_K + V "
                                  "Q6_K (residual/norm/Q8_K prologue), O Q4_K, gate|up GELU Q4_K, down Q6_K",
                      "weight_bytes": layer_bytes, "us_per_layer": round(per * 1e6, 2), "launches": 4,
                      "weight_copies_rotated": ncp, "projections": parts,
                      "q5k_gateup_variant": {"weight_bytes": q5_bytes, "us_per_layer": round(q5_per * 1e6, 2),
                                             "GBps": round(q5_bytes / q5_per / 1e9, 1)}},
           "roofline": dict(roofline(layer_bytes, per, "layer projections"), kernel="the four launches of one layer",
                            bytes_per_launch=layer_bytes)}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_layer_baseline(raws, shapes, layer_bytes)
    return res


def cpu_layer_baseline(raws, shapes, layer_bytes):
    """The same projections through the reference's own functions when
    oracle/_ref is built (quantize_row_q8_K + mm_quant_dot_rows for Q4_K,
    mm_quant_rows for Q6_K), else the oracle's restatement."""
    import oracle as orc_mod
    thr = cpu_threads()
    rng = np.random.default_rng(11)
    n = 2560
    x = rng.standard_normal(n).astype(np.float32)
    xa = rng.standard_normal(2048).astype(np.float32)
    hb = rng.standard_normal(10240).astype(np.float32)
    ref = orc_mod.Ref() if orc_mod.Ref.available() else None
    orc = orc_mod.Oracle()
    kind = "reference" if ref else "port"
    L = ref.L if ref else orc.L
    pre = "ref_" if ref else "or_"
    qz, dot, rows = (getattr(L, pre + s) for s in (("quantize_row_q8_K" if ref else "quantize_q8K"),
                                                  "mm_quant_dot_rows", "mm_quant_rows"))
    P = lambda a: a.ctypes.data  # noqa: E731
    q8 = np.zeros(n // 256, orc_mod.Q8K_DTYPE)
    q8a = np.zeros(2048 // 256, orc_mod.Q8K_DTYPE)
    outs = {k: np.empty(shapes[k][2], np.float32) for k in raws}

    def run():
        qz(P(x), P(q8), n)
        for kname in ("q", "k"):
            dot(P(outs[kname]), P(raws[kname]), n, shapes[kname][2], 12, P(q8))
        rows(P(outs["v"]), P(x), P(raws["v"]), n, shapes["v"][2], 14)
        qz(P(xa), P(q8a), 2048)
        dot(P(outs["o"]), P(raws["o"]), 2048, n, 12, P(q8a))
        for kname in ("gate", "up"):
            dot(P(outs[kname]), P(raws[kname]), n, 10240, 12, P(q8))
        rows(P(outs["down"]), P(hb), P(raws["down"]), 10240, n, 14)
    run()
    ts = []
    t_end = time.perf_counter() + 10.0
    while time.perf_counter() < t_end or len(ts) < 5:
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    med = float(np.median(ts))
    return {"value": round(layer_bytes / med / 1e9, 2), "unit": "GB/s", "cores": thr, "kind": kind,
            "host": cpu_host(),
            "sample": f"one layer's projections (Q8_K of the input, Q/K/O/gate/up mm_quant_dot_rows, V/down "
                      f"mm_quant_rows), median of {len(ts)} runs, OpenMP {thr} threads"}


FP16_MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 matrix peak (the image and split-Q6_K prefill GEMMs)
INT8_MFMA_PEAK_TOPS = 5000.0     # MI355X dense int8 matrix peak (the Q4_K/Q5_K prefill GEMM on the quantized tensors)

# one E4B sliding-window layer's Q4_K matrices (rows d, inputs n): Q, K, O,
# gate, up, PLE inp_gate, PLE proj
PREFILL_MATS = [("q", 2048, 2560), ("k", 512, 2560), ("o", 2560, 2048), ("gate", 10240, 2560),
                ("up", 10240, 2560), ("inp_gate", 256, 2560), ("proj", 2560, 256)]


def bench_prefill(lib, g4, synth, args):
    """Batched prefill GEMM: 512 prompt tokens through one E4B layer's Q4_K
    matrices with pre-quantized Q8_K activations, launched as the engine
    launches them: Q|K in one launch, O, gate|up in one launch on their fp16
    weight images (g4_kq_image, built once as the engine builds them at its
    first prompt chunk), PLE inp_gate and proj; a step is the five launches.
    Reports matrix-core throughput (2 * tokens * rows * n algorithmic ops)
    against the fp16 dense peak (the kernels issue one fp16 MFMA flop per
    algorithmic flop, plus the min sums' 1/32), and the dominant launch
    (gate|up, 2 x 10240 x 2560) alone."""
    m = 512
    rng = np.random.default_rng(1)
    mats = {}
    for name, d, n in PREFILL_MATS:
        raw = synth.rand_q4K(rng, d, n)
        w = g4.upload_quant(lib, raw, g4.Q4_K, n, d)
        x = g4.DBuf.from_array(lib, rng.standard_normal((m, n)).astype(np.float32))
        q8 = g4.DBuf(lib, lib.L.g4_q8K_row_stride(n) * m)
        lib.g4_quantize_rows_q8_K(x.ptr, q8.ptr, n, m)
        out = g4.DBuf(lib, 4 * m * d)
        img = None
        if name in ("gate", "up"):
            img = g4.DBuf(lib, lib.L.g4_kq_image_bytes(n, d))
            lib.g4_kq_image(img.ptr, w.ptr, n, d, g4.Q4_K)
        mats[name] = (d, n, raw, w, q8, out, img)
    L = lib.L
    VP2, I2 = C.c_void_p * 2, C.c_int * 2
    q_, k_, gt, up = mats["q"], mats["k"], mats["gate"], mats["up"]
    qk = (VP2(q_[5].ptr, k_[5].ptr), VP2(q_[3].ptr, k_[3].ptr), I2(q_[0], k_[0]))
    gu = (VP2(gt[5].ptr, up[5].ptr), VP2(gt[6].ptr, up[6].ptr), I2(gt[0], up[0]))

    def gate_up(i):
        L.g4_mm_batch_img_multi(gu[0], gu[1], gu[2], 2, gt[4].ptr, gt[1], m, g4.Q4_K)

    def step(i):
        L.g4_mm_batch_q8_multi(qk[0], qk[1], qk[2], 2, q_[4].ptr, q_[1], m, g4.Q4_K)
        for name in ("o", "inp_gate", "proj"):
            d, n, _, w, q8, out, _ = mats[name]
            L.g4_mm_batch_q8(out.ptr, w.ptr, q8.ptr, n, d, m, g4.Q4_K)
        gate_up(i)

    ms = _time_steps(lib, step, args)
    per_step = ms / 1e3 / args.steps
    ops = sum(2.0 * m * d * n for d, n, *_ in mats.values())
    ms1 = _time_steps(lib, gate_up, args)
    per1 = ms1 / 1e3 / args.steps
    ops1 = 2.0 * m * (gt[0] + up[0]) * gt[1]
    tf1 = ops1 / per1 / 1e12
    name = "mm_batch_img_kernel gate|up 2x10240x2560, 512 tokens"
    res = {
        "value": round(m / per_step, 1), "unit": "tok/s (one layer's Q4_K GEMMs)", "higher_is_better": True,
        "ms_per_step": ms / args.steps,
        "dtype": "u4 x int8 -> int32 matrix products (gate/up: fp16 sc*q images), fp32 block combine",
        "config": {"workload": "batched prefill GEMM: 512 tokens x one E4B SWA layer's Q4_K matrices "
                               "(Q|K 2048+512, O 2560<-2048, gate|up 2x10240 on images, PLE 256/2560) (seed 1)",
                   "tokens": m, "layer_tflops": round(ops / per_step / 1e12, 2)},
        "roofline": {"bound": "mfma", "achieved": round(tf1, 2), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf1 / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": measured_traffic(name),
                     "kernel": name, "us_per_launch": round(per1 * 1e6, 2)},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_prefill_baseline(gt[2], gt[1], gt[0])
    return res


FP32_MFMA_PEAK_TFLOPS = 157.3    # MI355X dense fp32 matrix peak (the bf16 PLE projection's instruction)
Q6S_MFMA_PER_FLOP = 3     # fp16 MFMA flops the split Q6_K GEMM issues per algorithmic flop (Wh hi, Wh lo, Wl hi)


def bench_prefill_e2e(lib, g4, synth, args):
    """Batched prompt prefill through the engine at the E4B shape: a step is
    g4e_prefill of 511 tokens (chunk of 511: every layer's GEMMs, attention
    over the chunk's rows, norms, RoPE, appends, PLE).  The roofline kernel is
    the one that takes most of the time, the Q6_K GEMM on split fp16
    activations (FFN down and V), timed alone with HIP events; it issues three
    fp16 MFMA flops per algorithmic flop (the weight's fp16 rounding against
    the hi and lo activation terms, its +-1 residual against the hi term),
    reported as mfma_issued."""
    path = _gguf_e4b(synth)
    eng = g4.Engine(path, max_seq=1024)
    rng = np.random.default_rng(4)
    m = 511
    prompt = rng.integers(0, eng.vocab, m).astype(np.int32)
    for _ in range(args.warmup):
        eng.prefill(prompt, 0)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.prefill(prompt, 0)                 # returns after the work has completed
    sec = (time.perf_counter() - t0) / args.steps
    eng.close()
    # the dominant kernel, mm_batch_q6s_kernel (V of the 24 storing layers and
    # FFN down of all 42 over the chunk's rows), timed alone with HIP events in
    # the engine's proportion of launches: 20 x V 512x2560, 4 x V 1024x2560,
    # 42 x down 2560x10240 per step, on activations split once per matrix
    shapes = [(2560, 512, 20), (2560, 1024, 4), (10240, 2560, 42)]
    mats = []
    for n, d, cnt in shapes:
        raw = synth.rand_q6K(rng, d, n)
        w = g4.upload_quant(lib, raw, g4.Q6_K, n, d)
        x = g4.DBuf.from_array(lib, rng.standard_normal((m, n)).astype(np.float32))
        xs = g4.DBuf(lib, lib.L.g4_split_rows_bytes(n, m))
        lib.g4_split_rows_f16(x.ptr, xs.ptr, n, m)
        out = g4.DBuf(lib, 4 * m * d)
        mats.append((n, d, cnt, w, xs, out))
    L = lib.L

    def one(i):
        for n, d, cnt, w, xs, out in mats:
            for _ in range(cnt):
                L.g4_mm_batch_split(out.ptr, w.ptr, xs.ptr, n, d, m, g4.Q6_K)
    ms1 = _time_steps(lib, one, args)
    launches = sum(c for _, _, c, *_ in mats)
    per1 = ms1 / 1e3 / args.steps / launches
    flops = sum(2.0 * m * n * d * c for n, d, c, *_ in mats) / launches
    tf1 = flops / per1 / 1e12
    name = "mm_batch_q6s_kernel<Q6_K> (V and FFN down of one 511-token chunk)"
    res = {
        "value": round(m / sec, 1), "unit": "tok/s", "higher_is_better": True, "ms_per_step": sec * 1e3,
        "dtype": "u4/u5 x int8 -> int32 matrix products (Q4_K/Q5_K; gate/up on fp16 sc*q images), split-fp16 "
                 "matrix products (Q6_K), "
                 "fp32 matrix products (bf16), fp32 glue",
        "config": {"workload": "synthetic E4B-shape batched prefill (42 layers, hidden 2560, FFN 10240, 8q/2kv heads, "
                               "head_dim 256/512, window 512, Q4_K_M mix, seed 4): 511 prompt tokens in one chunk",
                   "tokens": m, "roofline_launches_per_step": launches},
        "roofline": {"bound": "mfma", "achieved": round(tf1, 2), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf1 / FP16_MFMA_PEAK_TFLOPS, 4),
                     "mfma_issued": round(Q6S_MFMA_PER_FLOP * tf1, 2),
                     "mfma_issued_frac": round(Q6S_MFMA_PER_FLOP * tf1 / FP16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic(name), "kernel": name, "us_per_launch": round(per1 * 1e6, 2)},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_prefill_e2e_baseline(path)
    return res


def cpu_prefill_e2e_baseline(path: str, tokens: int = 4) -> dict:
    """The reference's prompt loop (forward() per token, main.c:2366-2384) as
    the oracle's C forward on the same GGUF, over a bounded sample of tokens."""
    import oracle as orc_mod
    thr = cpu_threads()
    om = orc_mod.OracleModel(orc_mod.Oracle(), path, max_seq=64)
    prompt = np.array([2, 105, 9731, 107, 12][:tokens + 1], np.int32)
    _, pf, _ = om.generate_greedy(prompt, 1)
    om.close()
    return {"value": round(tokens / pf, 3) if pf > 0 else None, "unit": "tok/s", "cores": thr, "kind": "port",
            "sample": f"oracle forward() per prompt token (C restatement of the reference, gcc -O3 -std=c11, OpenMP "
                      f"{thr} threads): the first {tokens} prompt positions on the same GGUF"}


def cpu_prefill_baseline(raw, n, d, tokens: int = 4):
    """The reference's prefill of this matrix: quantize_row_q8_K +
    mm_quant_dot_rows once per token (forward() per prompt token)."""
    import oracle as orc_mod
    thr = cpu_threads()
    rng = np.random.default_rng(7)
    xs = rng.standard_normal((tokens, n)).astype(np.float32)
    o = np.empty(d, np.float32)
    q8 = np.zeros(n // 256, orc_mod.Q8K_DTYPE)
    if orc_mod.Ref.available():
        ref, kind = orc_mod.Ref(), "reference"

        def run():
            for t in range(tokens):
                ref.L.ref_quantize_row_q8_K(xs[t].ctypes.data, q8.ctypes.data, n)
                ref.L.ref_mm_quant_dot_rows(o.ctypes.data, raw.ctypes.data, n, d, 12, q8.ctypes.data)
    else:
        orc, kind = orc_mod.Oracle(), "port"

        def run():
            for t in range(tokens):
                orc.mm_quant_dot_rows(raw, n, d, 12, orc.quantize_q8K(xs[t]))
    run()
    ts = []
    t_end = time.perf_counter() + 10.0
    while time.perf_counter() < t_end or len(ts) < 5:
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    med = float(np.median(ts))
    return {"value": round(2.0 * tokens * d * n / med / 1e12, 4), "unit": "TFLOP/s", "cores": thr, "kind": kind,
            "sample": f"{tokens} tokens of quantize_row_q8_K + mm_quant_dot_rows (Q4_K {d}x{n}), median of "
                      f"{len(ts)} runs, OpenMP {thr} threads"}


LMHEAD_KERNEL = "gemv_q6k_xreg_kernel<Q6_K, softcap> 262144x2560"


def bench_lmhead(lib, g4, synth, args):
    """Tied LM head: Q6_K 262144x2560 x fp32 hidden, fused soft-cap (550 MB > MALL)."""
    n, d = 2560, 262144
    rng = np.random.default_rng(2)
    raw = synth.rand_q6K(rng, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    w = g4.upload_quant(lib, raw, g4.Q6_K, n, d)
    xd = g4.DBuf.from_array(lib, x)
    out = g4.DBuf(lib, 4 * d)
    L = lib.L

    def step(i):
        L.g4_mm_quant_rows_softcap(out.ptr, xd.ptr, w.ptr, n, d, g4.Q6_K, C.c_float(30.0))

    algo = raw.nbytes + 4 * n + 4 * d
    ms = _time_steps(lib, step, args)
    per = ms / 1e3 / args.steps
    res = {
        "value": round(algo / per / 1e9, 1), "unit": "GB/s", "higher_is_better": True,
        "ms_per_step": ms / args.steps, "dtype": "f32",
        "config": {"workload": "tied LM head Q6_K 262144x2560 x fp32, softcap 30 (seed 2)"},
        "roofline": dict(roofline(algo, per, LMHEAD_KERNEL), kernel=LMHEAD_KERNEL, bytes_per_launch=algo,
                         us_per_launch=round(per * 1e6, 2)),
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_lmhead_baseline(raw, x, n)
    return res


def cpu_lmhead_baseline(raw, x, n, rows: int = 32768):
    """logits_tied's product on the CPU: the reference's mm_quant_rows
    (oracle/_ref when built, else the oracle's restatement) over the first
    `rows` rows of the same table, soft-cap included, as GB/s of weights."""
    import oracle as orc_mod
    thr = cpu_threads()
    ref = orc_mod.Ref() if orc_mod.Ref.available() else None
    fn = ref.L.ref_mm_quant_rows if ref else orc_mod.Oracle().L.or_mm_quant_rows
    part = np.ascontiguousarray(raw[:rows])      # rows of 10 Q6_K blocks: the row-major GGUF layout
    o = np.empty(rows, np.float32)

    def run():
        fn(o.ctypes.data, x.ctypes.data, part.ctypes.data, n, rows, 14)
        np.tanh(o / 30.0) * 30.0
    run()
    ts = []
    t_end = time.perf_counter() + 10.0
    while time.perf_counter() < t_end or len(ts) < 5:
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    med = float(np.median(ts))
    return {"value": round(part.nbytes / med / 1e9, 2), "unit": "GB/s", "cores": thr,
            "kind": "reference" if ref else "port", "host": cpu_host(),
            "sample": f"mm_quant_rows + soft-cap over the first {rows} of the 262144 rows ({part.nbytes} B of "
                      f"weights), median of {len(ts)} runs, OpenMP {thr} threads"}


def bench_copy(lib, g4, synth, args):
    """Plain device-to-device copy of 64 MiB (read + write): the practical HBM
    ceiling, and the reference kernel for scaling rocprof byte counters."""
    nbytes = 64 << 20
    ncp = 4
    srcs = [g4.DBuf(lib, nbytes) for _ in range(ncp)]
    dst = g4.DBuf(lib, nbytes)
    L = lib.L

    def step(i):
        L.g4_memcpy_d2d_async(dst.ptr, srcs[i % ncp].ptr, nbytes)

    ms = _time_steps(lib, step, args)
    per = ms / 1e3 / args.steps
    return {"value": round(2 * nbytes / per / 1e9, 1), "unit": "GB/s (read+write)", "higher_is_better": True,
            "ms_per_step": ms / args.steps, "dtype": "u8", "config": {"workload": "device copy 64 MiB"},
            "roofline": dict(roofline(2 * nbytes, per), kernel="copy", bytes_per_launch=2 * nbytes)}


def _gguf_e4b(synth, seed: int = 4) -> str:
    """The synthetic E4B-shape GGUF (about 5.4 GB), written once per machine."""
    return synth.e4b_gguf(seed)


def _gate_up_roofline(lib, g4, synth, n_launch: int = 200):
    """The dominant decode kernel at its decode shape: fused gate/up GELU GEMV,
    Q4_K 2 x 10240x2560 against one Q8_K vector, rotating weight copies (>= 512
    MB) so every launch streams from HBM.  HIP events on the library stream."""
    n, d = 2560, 10240
    rng = np.random.default_rng(1)
    g_raw = synth.rand_q4K(rng, d, n)
    u_raw = synth.rand_q4K(rng, d, n)
    ncp = _copies(2 * g_raw.nbytes)
    gs = [g4.upload_quant(lib, g_raw, g4.Q4_K, n, d) for _ in range(ncp)]
    us = [g4.upload_quant(lib, u_raw, g4.Q4_K, n, d) for _ in range(ncp)]
    x = g4.DBuf.from_array(lib, rng.standard_normal(n).astype(np.float32))
    q8 = g4.DBuf(lib, lib.L.g4_q8K_bytes(n))
    hb = g4.DBuf(lib, 4 * d)
    lib.g4_quantize_row_q8_K(x.ptr, q8.ptr, n)
    L = lib.L

    def step(i):
        L.g4_mm_gate_up_gelu(hb.ptr, gs[i % ncp].ptr, us[i % ncp].ptr, n, d, g4.Q4_K, q8.ptr)

    class A:
        warmup, steps = 20, n_launch
    ms = _time_steps(lib, step, A)
    per = ms / 1e3 / n_launch
    algo = 2 * g_raw.nbytes + lib.L.g4_q8K_bytes(n) + 4 * d
    name = "gemv_q45_stream_kernel<gate|up, GELU> 2x10240x2560 Q4_K"
    res = dict(roofline(algo, per, name), kernel=name, bytes_per_launch=algo, us_per_launch=round(per * 1e6, 3))

    # the same GEMV as the decode step runs it: the post-attention residual
    # step, ffn_norm and Q8_K as every workgroup's prologue (g4_mm_residual_q8)
    vecs = [g4.DBuf.from_array(lib, rng.standard_normal(n).astype(np.float32)) for _ in range(4)]
    xr, yr, wp, wn = vecs
    xo = g4.DBuf(lib, 4 * n)

    def step_pro(i):
        L.g4_mm_residual_q8(hb.ptr, gs[i % ncp].ptr, us[i % ncp].ptr, n, d, g4.Q4_K, None, xr.ptr, xo.ptr, yr.ptr,
                            wp.ptr, None, wn.ptr, None, None, 0, 1e-6)
    ms = _time_steps(lib, step_pro, A)
    per_p = ms / 1e3 / n_launch
    algo_p = 2 * g_raw.nbytes + 5 * 4 * n + 4 * d
    rp = roofline(algo_p, per_p, "")
    res["in_step"] = {"kernel": "gemv_q45_stream_kernel<gate|up, GELU, residual prologue> 2x10240x2560 Q4_K",
                      "achieved": rp["achieved"], "frac": rp["frac"], "bytes_per_launch": algo_p,
                      "us_per_launch": round(per_p * 1e6, 3)}
    return res


# ISWA decode attention (8 q / 2 kv heads): (name, positions read, head_dim,
# ring slots, window, RoPE base, cache slots)
ATTN_CASES = [("sliding, ring 512, hd 256", 512, 256, 512, 512, 1e4, 512),
              ("global T=4096, hd 256", 4096, 256, 0, 0, 1e6, 4096),
              ("global T=32768, hd 256", 32768, 256, 0, 0, 1e6, 32768),
              ("global T=4096, hd 512", 4096, 512, 0, 0, 1e6, 4096),
              ("global T=32768, hd 512", 32768, 512, 0, 0, 1e6, 32768)]
ATTN_HEADLINE = 2


def _attn_chunks(cap: int) -> int:
    """chunk count the engine fixes for a cache of cap slots (engine.c attn_chunks)"""
    G = min(max((cap + 31) // 32, 1), 128)
    while (cap + G - 1) // G > 1024:
        G += 1
    return G


ATTN_KERNEL = "attn_chunk_kernel + attn_merge_wide_kernel (global T=32768, hd 256)"


def bench_attn(lib, g4, synth, args):
    """ISWA decode attention, one layer's step: q/k norms, Neox RoPE, the
    K/V append and softmax(q.K) V over the cache (g4_attn_decode_fused, the
    engine's launch pair), N(0,1) inputs (seed 3).  Caches of every case
    are rotated through >= 512 MB of copies so that the reads come from HBM.
    value: KV GB/s of the global T=32768 hd 256 case; every case in config."""
    L = lib.L
    rng = np.random.default_rng(3)
    nh, nkv, eps = 8, 2, 1e-6
    cases = []
    for name, T, hd, ring, window, theta, slots in ATTN_CASES:
        kvd = nkv * hd
        pos = T - 1 if ring == 0 else 1000                  # a sliding ring past its first wrap
        host = rng.standard_normal((slots, kvd)).astype(np.float32)
        kv_bytes = 2 * host.nbytes
        ncp = max(2, -(-MALL_BYTES // kv_bytes))
        caches = [(g4.DBuf.from_array(lib, host), g4.DBuf.from_array(lib, host)) for _ in range(ncp)]
        del host
        qr = g4.DBuf.from_array(lib, rng.standard_normal(nh * hd).astype(np.float32))
        kr = g4.DBuf.from_array(lib, rng.standard_normal(kvd).astype(np.float32))
        vr = g4.DBuf.from_array(lib, rng.standard_normal(kvd).astype(np.float32))
        qn = g4.DBuf.from_array(lib, rng.uniform(0.8, 1.2, hd).astype(np.float32))
        kn = g4.DBuf.from_array(lib, rng.uniform(0.8, 1.2, hd).astype(np.float32))
        dpos = g4.DBuf.from_array(lib, np.array([pos, 0], np.int32))
        tab = g4.DBuf(lib, hd * 4)
        lib.g4_rope_table(tab.ptr, dpos.ptr, 0, hd, C.c_float(theta), C.c_float(1.0), None)
        G = _attn_chunks(ring if ring else slots)
        part = g4.DBuf(lib, L.g4_attn_part_bytes(nh, hd, G))
        out = g4.DBuf(lib, nh * hd * 4)

        def step(i, caches=caches, qr=qr, kr=kr, vr=vr, qn=qn, kn=kn, kvd=kvd, ring=ring, dpos=dpos,
                 window=window, hd=hd, tab=tab, G=G, part=part, out=out):
            kc, vc = caches[i % len(caches)]
            L.g4_attn_decode_fused(qr.ptr, qn.ptr, kr.ptr, vr.ptr, kn.ptr, kc.ptr, vc.ptr, kc.ptr, vc.ptr, kvd, ring,
                                   dpos.ptr, window, nh, nkv, hd, hd, tab.ptr, C.c_float(eps), C.c_float(1.0), G,
                                   part.ptr, out.ptr, None)

        ms = _time_steps(lib, step, args)
        per = ms / 1e3 / args.steps
        nwin = min(pos + 1, window) if window else pos + 1
        algo = 2 * nwin * kvd * 4 + (2 * nh * hd + 2 * kvd) * 4
        cases.append({"case": name, "positions": nwin, "chunks": G, "us": round(per * 1e6, 2),
                      "GBps": round(algo / per / 1e9, 1), "frac": round(algo / per / 1e9 / HBM_PEAK_GBS, 4),
                      "kv_bytes": 2 * nwin * kvd * 4, "copies_rotated": ncp})
        _log(f"attention {name}: {per * 1e6:.2f} us, {algo / per / 1e9:.0f} GB/s")
        del caches
        lib.g4_sync()
    h = cases[ATTN_HEADLINE]
    res = {
        "value": h["GBps"], "unit": "GB/s (KV read)", "higher_is_better": True, "ms_per_step": h["us"] / 1e3,
        "dtype": "f32",
        "config": {"workload": "ISWA decode attention step (q/k norms, Neox RoPE, K/V append, softmax(qK)V), 8 q / 2 "
                               "kv heads, fp32 KV cache, N(0,1) inputs (seed 3); value: global T=32768 hd 256",
                   "cases": cases},
        "roofline": {"bound": "hbm", "achieved": h["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": h["frac"],
                     "traffic": measured_traffic(ATTN_KERNEL),
                     "kernel": ATTN_KERNEL,
                     "bytes_per_launch": h["kv_bytes"], "us_per_launch": h["us"]},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_attn_baseline()
    return res


def cpu_attn_baseline() -> dict:
    """The attention block of main.c:1909-1950 as the oracle's plain loops
    (per head q.K, softmax, p.V) over the global T=4096 hd 256 case."""
    import oracle as orc_mod
    orc = orc_mod.Oracle()
    rng = np.random.default_rng(3)
    T, hd, nh, nkv = 4096, 256, 8, 2
    kc = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    orc.attn(q, kc, vc, nkv * hd, 0, T, nh, nkv, hd, 1.0)
    ts = []
    t_end = time.perf_counter() + 10.0
    while time.perf_counter() < t_end or len(ts) < 20:
        t0 = time.perf_counter()
        orc.attn(q, kc, vc, nkv * hd, 0, T, nh, nkv, hd, 1.0)
        ts.append(time.perf_counter() - t0)
    med = float(np.median(ts))
    return {"value": round(2 * T * nkv * hd * 4 / med / 1e9, 3), "unit": "GB/s (KV read)", "cores": 1,
            "kind": "port", "host": cpu_host(),
            "sample": f"oracle or_attn_decode (the attention block as plain loops, one thread) over the global "
                      f"T=4096 hd 256 case, median of {len(ts)} runs"}


def _log(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def bench_gateup(lib, g4, synth, args):
    """The dominant decode kernel alone: fused gate|up GELU GEMV at its decode
    shape (Q4_K 2 x 10240x2560), weight copies rotated through >= 512 MB."""
    r = _gate_up_roofline(lib, g4, synth, n_launch=args.steps)
    return {"value": r["achieved"], "unit": "GB/s", "higher_is_better": True,
            "ms_per_step": r["us_per_launch"] / 1e3, "dtype": "int8xu4->int32, fp32 combine",
            "config": {"workload": "fused gate|up GELU GEMV, Q4_K 2 x 10240x2560, batch 1 (seed 1)"}, "roofline": r}


def bench_decode(lib, g4, synth, args):
    """Full synthetic E4B-shape decode: 42 layers, dim 2560, FFN 10240, vocab
    262144, Q4_K_M mix; 511 prompt tokens prefilled in one chunk (batched
    GEMMs, attention over the chunk's rows), then greedy decode steps replayed
    as one HIP graph per token.  The prefill rate of the chunk and of the
    token-by-token loop are reported beside the decode rate."""
    t0 = time.perf_counter()
    _log("synthetic E4B-shape GGUF (seed 4)")
    path = _gguf_e4b(synth)
    t_gen = time.perf_counter() - t0
    _log(f"GGUF ready in {t_gen:.1f} s; loading into HBM")
    eng = g4.Engine(path, max_seq=1024)
    rng = np.random.default_rng(4)
    n_prompt = 512
    prompt = rng.integers(0, eng.vocab, n_prompt).astype(np.int32)
    # prefill in one 511-token chunk (the first call sizes the chunk buffers
    # and builds the FFN gate/up fp16 images, reported separately; the
    # second, timed, rewrites the same positions), then the timed decode
    _log("prefill 511 tokens in one chunk")
    t1 = time.perf_counter()
    eng.prefill(prompt[:-1], 0)
    t_prefill_first = time.perf_counter() - t1
    t1 = time.perf_counter()
    eng.prefill(prompt[:-1], 0)
    t_prefill = time.perf_counter() - t1
    # the reference's prompt loop, token by token, over the first 64 positions
    n_serial = 64
    t2 = time.perf_counter()
    for pos in range(n_serial):
        eng.forward(int(prompt[pos]), pos, 0)
    t_serial = time.perf_counter() - t2
    eng.prefill(prompt[:-1], 0)
    assert n_prompt - 1 + args.warmup + args.steps <= eng.max_seq
    tok = int(prompt[-1])
    use_graph = not args.no_graph
    _, _ = eng.decode_steps(tok, n_prompt - 1, args.warmup, use_graph=use_graph)
    # timed: K graph replays from position 511 + W; events bracket the region
    lib.L.g4_set_stream(None)
    toks, sec = eng.decode_steps(tok, n_prompt - 1 + args.warmup, args.steps, use_graph=use_graph, record=False)
    tps = args.steps / sec
    _log(f"decode {args.steps} steps: {tps:.1f} tok/s")
    # the same steps with the reference's default sampling (temp 0.6, top-p
    # 0.9, top-k 40) on the device after each forward, in the graph
    _, _ = eng.decode_steps_sampled(tok, n_prompt - 1, args.warmup, use_graph=use_graph)
    _, sec_s = eng.decode_steps_sampled(tok, n_prompt - 1 + args.warmup, args.steps, use_graph=use_graph)
    tps_s = args.steps / sec_s
    _log(f"sampled decode {args.steps} steps: {tps_s:.1f} tok/s")
    eng.close()
    res = {
        "value": round(tps, 2), "unit": "tok/s", "higher_is_better": True,
        "ms_per_step": sec * 1e3 / args.steps, "dtype": "int8xu4/u6->int32 + f32 (Q4_K_M weights)",
        "config": {"workload": "synthetic E4B-shape greedy decode (42 layers, hidden 2560, FFN 10240, 8q/2kv heads, "
                               "head_dim 256/512, window 512, last 18 layers shared-KV, vocab 262144 tied Q6_K head, "
                               "Q4_K_M mix, seed 4); prompt 512 tokens, 511 prefilled in one chunk, then decode",
                   "positions": [n_prompt - 1 + args.warmup, n_prompt - 1 + args.warmup + args.steps],
                   "graph": use_graph, "weights_bytes_per_token": synth.decode_weight_bytes(synth.E4B),
                   "decode_tok_s_sampled": round(tps_s, 2),
                   "prefill_tok_s": round((n_prompt - 1) / t_prefill, 1),
                   "prefill_first_call_ms": round(t_prefill_first * 1e3, 1),
                   "prefill_tok_s_token_serial": round(n_serial / t_serial, 1),
                   "gguf_write_s": round(t_gen, 1)},
    }
    # matrix-core use of the batched prefill: algorithmic GEMM flops of the
    # 511 tokens over the prefill's wall time, and the share of that time the
    # issued matrix-core work would take at its instructions' peaks: int8
    # MFMA for the Q4_K/Q5_K GEMMs on the quantized tensors (one issued op
    # per op), fp16 MFMA for the FFN gate/up on their fp16 images (one per
    # flop) and for the split Q6_K (three per flop), fp32 MFMA for the bf16
    # PLE projection
    mm = synth.prefill_matmuls(synth.E4B)
    flops = sum(2.0 * n * d for _, _, n, d in mm) * (n_prompt - 1)

    def peak(name, t):
        if t == synth.BF16:
            return FP32_MFMA_PEAK_TFLOPS
        if t in (g4.Q4_K, g4.Q5_K) and not name.endswith(("ffn_gate.weight", "ffn_up.weight")):
            return INT8_MFMA_PEAK_TOPS
        return FP16_MFMA_PEAK_TFLOPS
    issued_s = sum(2.0 * n * d * (n_prompt - 1) * (3 if t == g4.Q6_K else 1) / (peak(nm, t) * 1e12)
                   for nm, t, n, d in mm)
    res["config"]["prefill_gemm_tflops"] = round(flops / t_prefill / 1e12, 1)
    res["config"]["prefill_mfma_util"] = round(issued_s / t_prefill, 4)
    _log("dominant-kernel roofline")
    res["roofline"] = _gate_up_roofline(lib, g4, synth)
    res["decode_hbm_GBps"] = round(synth.decode_weight_bytes(synth.E4B) * tps / 1e9, 1)
    if not args.no_cpu:
        _log("CPU baseline (oracle forward)")
        res["cpu_baseline"] = cpu_decode_baseline(path, (n_prompt - 1 + args.warmup, n_prompt - 1 + args.warmup
                                                          + args.steps))
    return res


def cpu_decode_baseline(path: str, positions: tuple, steps: int = 4) -> dict:
    """The oracle's forward() (the C restatement of main.c:1838-2029, OpenMP)
    on the same GGUF at the decode positions the GPU leg times: its caches
    hold zeros there instead of a prompt's K/V, which costs the same
    arithmetic (the attention spans the same windows); then one step on one
    thread."""
    import oracle as orc_mod
    thr = cpu_threads()
    p0 = positions[0]
    om = orc_mod.OracleModel(orc_mod.Oracle(), path, max_seq=p0 + steps + 8)
    om.forward(2, p0 - 1, 1)                                 # warm-up (page-in of the mapped weights)
    t0 = time.perf_counter()
    for i in range(steps):
        om.forward(2 + i, p0 + i, 1)
    sec = (time.perf_counter() - t0) / steps
    omp_threads(1)
    t1 = time.perf_counter()
    om.forward(3, p0 + steps, 1)
    sec1 = time.perf_counter() - t1
    omp_threads(thr)
    om.close()
    return {"value": round(1.0 / sec, 3), "unit": "tok/s", "cores": thr, "kind": "port",
            "tok_s_1_thread": round(1.0 / sec1, 4), "host": cpu_host(),
            "sample": f"oracle forward() with logits (C restatement of the reference, gcc -O3 -std=c11, OpenMP {thr} "
                      f"threads, plain-loop sgemv): {steps} decode steps at positions {p0}..{p0 + steps - 1} of the "
                      f"same GGUF, then 1 step on 1 thread"}


_STREAM = [None]    # the stream the kernel workloads run on (created in main)


def _time_steps(lib, step, args) -> float:
    """W eager warm-up launches, then the K timed launches captured as one
    graph on the library stream and replayed: the host's launch cost stays
    out of the timed region, which spans the kernels back to back (each
    launch's fixed dependent-kernel gap included).  Returns milliseconds."""
    if _STREAM[0] is not None:
        lib.check(lib.L.g4_set_stream(_STREAM[0]))   # an engine may have left the library on its own stream
    for i in range(args.warmup):
        step(i)
    lib.g4_sync()
    g = C.c_void_p()
    lib.check(lib.L.g4_graph_begin())
    for i in range(args.steps):
        step(i)
    lib.check(lib.L.g4_graph_end(C.byref(g)))
    try:
        lib.check(lib.L.g4_graph_launch(g))       # first replay: instantiation costs out of the timing
        lib.g4_sync()
        t = Timer(lib)
        t.start()
        lib.check(lib.L.g4_graph_launch(g))
        ms = t.stop_ms()
        lib.g4_sync()
    finally:
        lib.L.g4_graph_destroy(g)
    return ms


def bench_floors(lib, g4, synth, args):
    """The floors the decode step's kernels are sized against (probe kernels
    that compute nothing of the model): a dependent launch with no work, a
    streaming read at the byte counts of the step's kernels (weights rotated
    over more than the 256 MB Infinity Cache, so every launch reads HBM), and
    a last-workgroup hand-off inside a kernel against the same kernel
    without it.  Each is a graph of K launches timed with HIP events."""
    L = lib.L
    ncu, arch = C.c_int(), C.create_string_buffer(64)
    lib.check(L.g4_device_info(C.byref(ncu), arch, 64))
    cus = ncu.value
    res_cfg = {"cus": cus}
    # 1. chained empty kernels
    for wg in (1, 256, 1024):
        ms = _time_steps(lib, lambda i, wg=wg: L.g4_probe_empty(wg), args)
        res_cfg[f"empty_launch_us_{wg}wg"] = round(ms * 1e3 / args.steps, 3)
    # 2. streaming reads
    sink = g4.DBuf(lib, 4 * 4096)
    reads = {}
    for mb, label in ((2.95, "2.95MB (O Q4_K 2560x2048)"), (14.79, "14.8MB (Q4_K 10240x2560)"),
                      (21.54, "21.5MB (FFN down Q6_K 2560x10240)"), (29.54, "29.5MB (gate|up 2x10240x2560)"),
                      (551.6, "551.6MB (LM head Q6_K 262144x2560)")):
        nbytes = int(mb * 1e6) // 16 * 16
        ncp = _copies(nbytes)
        bufs = [g4.DBuf(lib, nbytes) for _ in range(ncp)]
        for b in bufs:
            lib.check(L.g4_memset(b.ptr, 0, nbytes))
        for wg in (4 * cus,):
            ms = _time_steps(lib, lambda i, b=bufs, n=nbytes, wg=wg: L.g4_probe_read(b[i % len(b)].ptr, n, sink.ptr, wg),
                             args)
            us = ms * 1e3 / args.steps
            reads[label] = {"us": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1), "copies_rotated": ncp}
        del bufs
    # 3. last-workgroup hand-off: 16 values per workgroup, fenced and as
    # device-scope atomics, against the same launch without it
    vals = g4.DBuf(lib, 4 * 16 * 640)
    cnt = g4.DBuf(lib, 256)
    out = g4.DBuf(lib, 256)
    lib.check(L.g4_memset(cnt.ptr, 0, 256))
    hand = {}
    got = np.zeros(1, np.float32)
    for wg in (13, 32, 160, 256, 640):
        t = []
        for mode in (0, 1, 2):
            ms = _time_steps(lib, lambda i, wg=wg, mode=mode: L.g4_probe_handoff(vals.ptr, cnt.ptr, out.ptr, wg, mode),
                             args)
            t.append(ms * 1e3 / args.steps)
            if mode:
                lib.check(L.g4_memcpy_d2h(got.ctypes.data, out.ptr, 4))
                want = float(np.sum(np.arange(16 * wg, dtype=np.float64)))
                assert abs(float(got[0]) - want) <= 1e-6 * want, (got, want)   # every value seen
        hand[f"{wg}wg"] = {"plain_us": round(t[0], 3), "fenced_us": round(t[1], 3), "atomic_us": round(t[2], 3),
                           "cost_fenced_us": round(t[1] - t[0], 3), "cost_atomic_us": round(t[2] - t[0], 3)}
    big = reads["551.6MB (LM head Q6_K 262144x2560)"]
    return {"value": big["GB_s"], "unit": "GB/s", "higher_is_better": True,
            "ms_per_step": big["us"] / 1e3, "dtype": "f32",
            "config": dict({"workload": "floors: chained empty launches, streaming reads, last-workgroup hand-off "
                            "(graphs of K launches, HIP events)", "streaming_read": reads, "handoff": hand},
                           **res_cfg)}


WORKLOADS = {"decode": bench_decode, "gemv": bench_gemv, "gateup": bench_gateup, "lmhead": bench_lmhead,
             "copy": bench_copy, "prefill": bench_prefill, "prefill_e2e": bench_prefill_e2e, "attn": bench_attn,
             "layer": bench_layer, "floors": bench_floors}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="decode with eager launches instead of one HIP graph "
                    "per token (same kernels; for profilers that do not follow graph launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the decode path is single-GPU; multi-GPU sharding is a design note only)", file=sys.stderr)
        return 2
    if args.steps is None:
        args.steps = {"decode": 128, "prefill_e2e": 10}.get(args.workload, 200)
    if args.warmup is None:
        args.warmup = {"decode": 8, "prefill_e2e": 2}.get(args.workload, 20)
    import g4
    import synth
    lib = g4.Lib.get()
    lib.init(0)
    stream = C.c_void_p()
    lib.check(lib.L.g4_stream_create(C.byref(stream)))
    lib.check(lib.L.g4_set_stream(stream))      # the kernel workloads' launches are captured on it
    _STREAM[0] = stream
    t0 = time.perf_counter()
    res = WORKLOADS[args.workload](lib, g4, synth, args)
    line = {"metric": METRIC, "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(res.pop("ms_per_step"), 6),
            "higher_is_better": res.pop("higher_is_better"), "scaling": "weak", "vs_baseline": None,
            "dtype": res.pop("dtype"), "data": "synthetic"}
    line.update(res)
    line["wall_s"] = round(time.perf_counter() - t0, 1)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
