// g4_device.h -- device-side formats and helpers shared by the gfx950 kernels.
//
// HBM layouts (all tensors are "planar": the bytes of every GGUF super-block
// are kept, only their placement changes, so the download transform gives
// back the GGUF bytes exactly):
//
//   Q4_K [d rows x nb blocks], 144 B/block (gemma4-4b/cpu-blas/main.c:95-100)
//     qs plane  : d*nb*128 B.  Block word 4l+j holds GGUF qs word 8j+l, so the
//                 8 lanes of a block read 16 contiguous bytes each and lane l
//                 owns bytes 4l..4l+3 of every 32-byte chunk -- the lane
//                 partition of the reference's AVX2 dot (main.c:500-523).
//     hdr plane : d*nb*16 B, GGUF bytes 0..15 (d, dmin, scales[12]) verbatim.
//   Q5_K [.. 176 B/block] (main.c:102-108): qs plane as Q4_K, qh plane
//                 d*nb*32 B verbatim, hdr plane d*nb*16 B.
//   Q6_K [.. 210 B/block] (main.c:110-115):
//     ql plane  : d*nb*128 B; lane L=4h+u of a block owns 16 contiguous bytes
//                 = GGUF ql[64h+8u .. +7] followed by ql[64h+32+8u .. +7].
//     qh plane  : d*nb*64 B verbatim (lane L reads bytes 8L..8L+7).
//     sc plane  : d*nb*16 B verbatim (int8 scales).
//     d plane   : d*nb*2 B verbatim (fp16 d).
//   Q8_K activations, nb blocks (main.c:118-122, private layout):
//     qs plane  : nb*256 B; block word 8l + 4h + j holds GGUF-order word
//                 16j + 8h + l (lane l's 32 bytes are contiguous).
//     bsums     : nb*16 int16, then d: nb fp32.   Total nb*292 B.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define G4_QK 256

namespace g4 {

// ---- plane offsets ---------------------------------------------------------
struct Q4KPlanes { size_t qs, hdr; };
struct Q5KPlanes { size_t qs, qh, hdr; };
struct Q6KPlanes { size_t ql, qh, sc, d; };

__host__ __device__ inline Q4KPlanes q4k_planes(size_t nblocks) { return {0, nblocks * 128}; }
__host__ __device__ inline Q5KPlanes q5k_planes(size_t nblocks) { return {0, nblocks * 128, nblocks * 160}; }
__host__ __device__ inline Q6KPlanes q6k_planes(size_t nblocks) {
    return {0, nblocks * 128, nblocks * 192, nblocks * 208};
}
__host__ __device__ inline size_t q8k_bsums_off(int nb) { return (size_t)nb * 256; }
__host__ __device__ inline size_t q8k_d_off(int nb) { return (size_t)nb * 288; }

// Q8_K qs permutation: GGUF word w = 16j + 8h + l  ->  device word 8l + 4h + j
__host__ __device__ inline int q8k_word_dev(int w) {
    const int j = w >> 4, h = (w >> 3) & 1, l = w & 7;
    return 8 * l + 4 * h + j;
}
// Q4_K qs permutation: GGUF word 8j + l -> device word 4l + j
__host__ __device__ inline int q4k_word_dev(int w) { return 4 * (w & 7) + (w >> 3); }

// ---- exact fp16 -> fp32 (main.c:128-149) -----------------------------------
// Integer decode so the result never depends on the hardware denorm mode:
// a binary16 subnormal is man * 2^-24, exact in binary32.
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, man = h & 1023u;
    if (e == 0) {
        const float v = (float)man * 5.9604644775390625e-8f;   // 2^-24
        return __uint_as_float(__float_as_uint(v) | sign);
    }
    const uint32_t bits = (e == 31) ? (sign | 0x7F800000u | (man << 13))
                                    : (sign | ((e + 112u) << 23) | (man << 13));
    return __uint_as_float(bits);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// 6-bit scale/min unpack in word form (main.c:490-495); sc[0..7], mn[0..7] as bytes
__device__ __forceinline__ void unpack_scales(const uint32_t s0, const uint32_t s1, const uint32_t s2,
                                              uint32_t& sc_lo, uint32_t& sc_hi, uint32_t& mn_lo, uint32_t& mn_hi) {
    sc_lo = s0 & 0x3f3f3f3fu;
    sc_hi = (s2 & 0x0f0f0f0fu) | (((s0 >> 6) & 0x03030303u) << 4);
    mn_lo = s1 & 0x3f3f3f3fu;
    mn_hi = ((s2 >> 4) & 0x0f0f0f0fu) | (((s1 >> 6) & 0x03030303u) << 4);
}
__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xff; }

// ---- RoPE angles (main.c:1725-1742) ------------------------------------------
// (cos, sin) of pair j at position p: the reference's angle chain theta_0 = p,
// theta_j = theta_{j-1} * ts (one rounding per step), angle = (fs * theta_j) / ff[j]
__device__ __forceinline__ float2 rope_pair_cs(int p, int j, float ts, float fs, const float* __restrict__ ff) {
    const float f = ff ? ff[j] : 1.0f;   // in flight during the product chain
    float theta = (float)p;
    for (int i = 0; i < j; i++) theta *= ts;
    const float angle = (fs * theta) / f;
    return make_float2(cosf(angle), sinf(angle));
}

// ---- cross-lane helpers (64-wide wavefronts) --------------------------------
template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) { return __shfl_xor(v, mask, 64); }

// Wave-wide reductions on DPP lane moves inside each 16-lane row (xor 1,
// xor 2 by quad permutes; then the mirrors, which pair a lane with one that
// holds the same partial value as its xor-4 / xor-8 partner) and four
// readlanes across the rows: (r0 + r1) + (r2 + r3).  The result is the same,
// bit for bit, as the xor butterfly v += shfl_xor(v, 1), (2), ..., (32), in
// every lane.  All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppXor1 = 0xB1;         // quad_perm(1,0,3,2)
constexpr int kDppXor2 = 0x4E;         // quad_perm(2,3,0,1)
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i within 16
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    v += dpp_f<kDppMirror>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppMirror>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Sum over the whole workgroup (blockDim.x a multiple of 64, <= 1024); every
// thread gets the total.  red must hold 16 floats; it is reusable after return.
// workgroup barrier for LDS hand-offs only: this wave's LDS operations are
// complete, then s_barrier.  __syncthreads() also waits for every
// outstanding global load; this keeps them in flight.  The asm is a
// compiler barrier for memory operations as well.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// GELU, tanh form, evaluated in the reference's operation order (main.c:1490-1492)
// ---- argmax keys: first index of the maximum -------------------------------
// key = order-preserving bits of the value (high word) and ~index (low word):
// the largest key is the largest value at its smallest index.  -0.0 is taken
// as +0.0 so that equal values compare equal, as the C comparison does.  The
// reference's scan (main.c:2046-2048) never moves to a NaN and never leaves
// one at index 0 (every comparison with it is false): a NaN gets the lowest
// key, or the highest at index 0.
__device__ __forceinline__ unsigned long long argmax_key(float v, int i) {
    if (v != v) return i == 0 ? ~0ull : 0ull;
    uint32_t u = __float_as_uint(v + 0.0f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)(~(uint32_t)i);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(k, m, 64);
        k = o > k ? o : k;
    }
    return k;
}

__device__ inline unsigned long long block_max_u64(unsigned long long k, unsigned long long* red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    k = wave_max_u64(k);
    if (lane == 0) red[w] = k;
    __syncthreads();
    unsigned long long t = 0;
    for (int i = 0; i < nw; i++) t = red[i] > t ? red[i] : t;
    return t;
}


__device__ __forceinline__ float gelu_ref(float x) {
    const float inner = 0.7978845608028654f * x * (1.0f + 0.044715f * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

// ---- Q8_K quantization of one 256-element block by one wavefront ----------
// (quantize_row_q8_K, gemma4-4b/cpu-blas/main.c:247-340)
// Quantize one 256-block held as 4 floats per lane; writes the device Q8_K
// layout (qs permuted, bsums, d).  Every lane of the wave must call it.
__device__ __forceinline__ void quantize_block_wave(const float v[4], int lane, uint8_t* __restrict__ y,
                                                    int nb, int b) {
    // amax = max |x|; maxv = the element of smallest index with |x| == amax
    // (lane l owns elements 4l..4l+3, so the first such lane holds it)
    float al = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) al = fmaxf(al, fabsf(v[e]));
    const float amax = wave_max(al);
    float cand = v[3];
    bool hit = fabsf(v[3]) == amax;
#pragma unroll
    for (int e = 2; e >= 0; e--) {
        if (fabsf(v[e]) == amax) { cand = v[e]; hit = true; }
    }
    const unsigned long long hits = __ballot(hit);
    const float maxv = hits ? lane_f(cand, (int)__builtin_ctzll(hits)) : 0.0f;
    int8_t q[4];
    float dval = 0.0f;
    if (amax == 0.0f) {
        q[0] = q[1] = q[2] = q[3] = 0;
    } else {
        const float iscale = -127.0f / maxv;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int r = (int)rintf(iscale * v[e]);
            q[e] = (int8_t)(r > 127 ? 127 : r);
        }
        dval = 1.0f / iscale;
    }
    const uint32_t word = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                          ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
    reinterpret_cast<uint32_t*>(y + (size_t)b * 256)[q8k_word_dev(lane)] = word;
    // bsums: 16 elements = 4 lanes
    int s = (int)q[0] + q[1] + q[2] + q[3];
    s += dpp_i<kDppXor1>(s);
    s += dpp_i<kDppXor2>(s);
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(y + q8k_bsums_off(nb))[b * 16 + (lane >> 2)] = (int16_t)s;
    if (lane == 0) reinterpret_cast<float*>(y + q8k_d_off(nb))[b] = dval;
}


// ---- residual step + next norm + Q8_K (one workgroup) ----------------------
//   if y:       x'[i] = x[i] + (y[i] * s_y) * w_post[i]       (main.c:1960-1962,
//               1982-1984, 1995-1997: post-norm then residual add)
//   if oscale:  x'[i] = x'[i] * oscale[0]                     (main.c:1999-2003)
//   if w_next:  xb2[i] = (x'[i] * s_x) * w_next[i]            (main.c:1878, 1973)
//   q8 = quantize_row_q8_K(qsrc == 0 ? xb2 : x')              (main.c:1884, 1975)
// s_v = 1/sqrtf(sum(v^2)/n + eps) (main.c:1451-1456; the sum is a tree).
struct ResidualArgs {
    const float* x;        // residual stream in
    float* x_out;          // residual stream out (may be x; nullptr: not stored)
    const float* y;        // sub-layer output (nullptr: no residual step)
    const float* w_post;
    const float* oscale;
    const float* w_next;   // nullptr: no second norm (the vector is x')
    float* xb2;            // nullable
    uint8_t* q8;           // nullable (global Q8_K of the vector)
    int qsrc;
    int n;
    float eps;
};

// The whole workgroup (n <= EPT * blockDim.x).  residual_load issues every
// global load of the step; residual_finish leaves the vector to quantize in
// buf (n floats of LDS) and, if store, writes x_out and xb2.  A caller may
// issue other loads between the two (they then overlap the norm's latency).
// red: 16 floats of LDS.
template <int EPT>
struct ResidualRegs {
    float xv[EPT], yv[EPT], wp[EPT], wn[EPT];
};

template <int EPT>
__device__ __forceinline__ void residual_load(const ResidualArgs& a, ResidualRegs<EPT>& r) {
    const int n = a.n, tid = threadIdx.x, nt = blockDim.x;
#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int i = tid + k * nt;
        const bool ok = i < n;
        r.xv[k] = ok ? a.x[i] : 0.0f;
        r.yv[k] = (ok && a.y) ? a.y[i] : 0.0f;
        r.wp[k] = (ok && a.y) ? a.w_post[i] : 0.0f;
        r.wn[k] = (ok && a.w_next) ? a.w_next[i] : 0.0f;
    }
}

template <int EPT>
__device__ __forceinline__ void residual_finish(const ResidualArgs& a, ResidualRegs<EPT>& r, float* buf, float* red,
                                                bool store) {
    const int n = a.n, tid = threadIdx.x, nt = blockDim.x;
    float* xv = r.xv;
    const float sc = a.oscale ? a.oscale[0] : 1.0f;
    if (a.y) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < EPT; k++) ss += r.yv[k] * r.yv[k];
        ss = block_sum(ss, red);
        const float sy = 1.0f / sqrtf(ss / (float)n + a.eps);
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            float v = xv[k] + (r.yv[k] * sy) * r.wp[k];
            if (a.oscale) v = v * sc;
            xv[k] = v;
        }
    }
    if (store && a.x_out && (a.y || a.x_out != a.x)) {
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            const int i = tid + k * nt;
            if (i < n) a.x_out[i] = xv[k];
        }
    }
    if (a.w_next) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < EPT; k++) ss += xv[k] * xv[k];
        ss = block_sum(ss, red);
        const float sx = 1.0f / sqrtf(ss / (float)n + a.eps);
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            const int i = tid + k * nt;
            const float t = (xv[k] * sx) * r.wn[k];
            if (i < n) {
                if (store && a.xb2) a.xb2[i] = t;
                buf[i] = a.qsrc == 0 ? t : xv[k];
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            const int i = tid + k * nt;
            if (i < n) buf[i] = xv[k];
        }
    }
}

// The same step with one float4 of each vector per thread (n/4 threads):
// thread t owns elements 4t .. 4t+3, so wave w holds Q8_K block w.  Every
// load is issued unconditionally (an absent vector is read from x in its
// place and not used), and each norm's sum of squares takes one LDS-only
// barrier: per thread ((a^2 + b^2) + c^2) + d^2, a wave butterfly, then the
// waves' sums in wave order.  off: the row's offset (rows of n floats).
struct Res4 {
    float4 x, y, wp, wn;
    float sc;
};

__device__ __forceinline__ void residual4_load(const ResidualArgs& a, Res4& r, size_t off) {
    const int tid = threadIdx.x;
    r.x = reinterpret_cast<const float4*>(a.x + off)[tid];
    r.y = reinterpret_cast<const float4*>(a.y ? a.y + off : a.x + off)[tid];
    r.wp = reinterpret_cast<const float4*>(a.y ? a.w_post : a.x)[tid];
    r.wn = reinterpret_cast<const float4*>(a.w_next ? a.w_next : a.x)[tid];
    r.sc = a.oscale ? a.oscale[0] : 1.0f;
}

// q: the thread's 4 values to quantize (qsrc 0: the normed vector, else x');
// nv: the normed vector (x' without w_next).  store: x_out and xb2 are
// written (one workgroup of a prologue kernel).  red: [2][16] floats of LDS.
__device__ __forceinline__ void residual4_finish(const ResidualArgs& a, const Res4& r, float (*red)[16], bool store,
                                                 size_t off, float q[4], float nv[4]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    float v[4] = {r.x.x, r.x.y, r.x.z, r.x.w};
    if (a.y) {
        const float y[4] = {r.y.x, r.y.y, r.y.z, r.y.w}, w[4] = {r.wp.x, r.wp.y, r.wp.z, r.wp.w};
        float ss = ((y[0] * y[0] + y[1] * y[1]) + y[2] * y[2]) + y[3] * y[3];
        ss = wave_sum(ss);
        if (lane == 0) red[0][wave] = ss;
        lds_sync();
        float t = 0.0f;
        for (int i = 0; i < nw; i++) t += red[0][i];
        const float sy = 1.0f / sqrtf(t / (float)a.n + a.eps);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float u = v[k] + (y[k] * sy) * w[k];
            if (a.oscale) u = u * r.sc;
            v[k] = u;
        }
    }
    if (store && a.x_out && (a.y || a.x_out != a.x))
        reinterpret_cast<float4*>(a.x_out + off)[tid] = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
    for (int k = 0; k < 4; k++) q[k] = nv[k] = v[k];
    if (a.w_next) {
        const float w[4] = {r.wn.x, r.wn.y, r.wn.z, r.wn.w};
        float ss = ((v[0] * v[0] + v[1] * v[1]) + v[2] * v[2]) + v[3] * v[3];
        ss = wave_sum(ss);
        if (lane == 0) red[1][wave] = ss;
        lds_sync();
        float t = 0.0f;
        for (int i = 0; i < nw; i++) t += red[1][i];
        const float sx = 1.0f / sqrtf(t / (float)a.n + a.eps);
#pragma unroll
        for (int k = 0; k < 4; k++) nv[k] = (v[k] * sx) * w[k];
        if (store && a.xb2) reinterpret_cast<float4*>(a.xb2 + off)[tid] = make_float4(nv[0], nv[1], nv[2], nv[3]);
        if (a.qsrc == 0) {
#pragma unroll
            for (int k = 0; k < 4; k++) q[k] = nv[k];
        }
    }
}

template <int EPT>
__device__ __forceinline__ void residual_core(const ResidualArgs& a, float* buf, float* red, bool store) {
    ResidualRegs<EPT> r;
    residual_load<EPT>(a, r);
    residual_finish<EPT>(a, r, buf, red, store);
}

// element e (0..255) of block blk of a planar K-quant tensor with nblk blocks;
// the fp32 value dequant_q*_k produces (main.c:172-237)
__device__ inline float dequant_elem(const uint8_t* __restrict__ w, int type, size_t nblk, size_t blk, int e) {
    if (type == 14) {   // Q6_K
        const Q6KPlanes p = q6k_planes(nblk);
        const int h = e >> 7, idx = e & 127, k = idx >> 5, l = idx & 31;
        const int gq = 64 * h + (k & 1) * 32 + l;            // GGUF ql byte
        const int r = gq & 63, u = (r & 31) >> 3, c = (r & 7) + (r >= 32 ? 8 : 0);
        const uint8_t qlb = w[p.ql + blk * 128 + 16 * (4 * h + u) + c];
        const uint8_t qhb = w[p.qh + blk * 64 + 32 * h + l];
        const int lo = k < 2 ? (qlb & 15) : (qlb >> 4);
        const int q = (int)(int8_t)(lo | (((qhb >> (2 * k)) & 3) << 4)) - 32;
        const int8_t sc = (int8_t)w[p.sc + blk * 16 + 8 * h + (l >> 4) + 2 * k];
        const float d = f16_to_f32(*reinterpret_cast<const uint16_t*>(w + p.d + blk * 2));
        return d * (float)sc * (float)q;
    }
    // Q4_K / Q5_K: element e is in 64-group c = e/64, nibble half hi = (e/32)&1
    const bool q5 = type == 13;   // Q5_K
    const size_t hdr_off = q5 ? q5k_planes(nblk).hdr : q4k_planes(nblk).hdr;
    const uint8_t* hdr = w + hdr_off + blk * 16;
    const int c = e >> 6, hi = (e >> 5) & 1, l = e & 31;
    const int gw = (32 * c + l) >> 2;                          // GGUF qs word
    const uint8_t qb = w[blk * 128 + 4 * q4k_word_dev(gw) + (l & 3)];
    int q = hi ? (qb >> 4) : (qb & 15);
    if (q5) {
        const uint8_t qh = w[q5k_planes(nblk).qh + blk * 32 + l];
        if (qh & (1u << (2 * c + hi))) q += 16;
    }
    const int j = 2 * c + hi;
    int sc, m;
    const uint8_t* s = hdr + 4;
    if (j < 4) { sc = s[j] & 63; m = s[j + 4] & 63; }
    else { sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
    const float d = f16_to_f32(*reinterpret_cast<const uint16_t*>(hdr));
    const float mn = f16_to_f32(*reinterpret_cast<const uint16_t*>(hdr + 2));
    const float d1 = d * (float)sc, m1 = mn * (float)m;
    return d1 * (float)q - m1;
}

// ---- BF16 x fp32 rows (mm_bf16, main.c:1529-1537) ---------------------------
// A wave's RPW rows of nch 16-byte chunks (8 bf16 each), chunk lane + 64c of
// row r in v[r][c] (zero past nch), against x in LDS: lane partial sums in
// chunk order, then the wave sum.  Every lane gets each row's dot.
template <int RPW, int CPL>
__device__ __forceinline__ void bf16_rows_dot(const uint4 (&v)[RPW][CPL], const float* xs, int nch, int lane,
                                              float (&res)[RPW]) {
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ch = lane + 64 * c;
            if (ch < nch) {
                const float4 xa = reinterpret_cast<const float4*>(xs)[2 * ch];
                const float4 xb = reinterpret_cast<const float4*>(xs)[2 * ch + 1];
                acc = __builtin_fmaf(xa.x, bf16_to_f32(v[r][c].x & 0xffffu), acc);
                acc = __builtin_fmaf(xa.y, bf16_to_f32(v[r][c].x >> 16), acc);
                acc = __builtin_fmaf(xa.z, bf16_to_f32(v[r][c].y & 0xffffu), acc);
                acc = __builtin_fmaf(xa.w, bf16_to_f32(v[r][c].y >> 16), acc);
                acc = __builtin_fmaf(xb.x, bf16_to_f32(v[r][c].z & 0xffffu), acc);
                acc = __builtin_fmaf(xb.y, bf16_to_f32(v[r][c].z >> 16), acc);
                acc = __builtin_fmaf(xb.z, bf16_to_f32(v[r][c].w & 0xffffu), acc);
                acc = __builtin_fmaf(xb.w, bf16_to_f32(v[r][c].w >> 16), acc);
            }
        }
        res[r] = wave_sum(acc);
    }
}

// the loads of those rows (rows past d and chunks past nch: zero)
template <int RPW, int CPL>
__device__ __forceinline__ void bf16_rows_load(const uint16_t* __restrict__ w, int n, int d, int row0, int lane,
                                               uint4 (&v)[RPW][CPL]) {
    const int nch = n / 8;
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ch = lane + 64 * c, row = row0 + r;
            v[r][c] = (row < d && ch < nch) ? reinterpret_cast<const uint4*>(w + (size_t)row * n)[ch]
                                            : make_uint4(0, 0, 0, 0);
        }
}

// Q8_K of the nb blocks in buf (LDS) into y (global or LDS, device layout),
// one wave per block
__device__ __forceinline__ void quantize_blocks_wg(const float* buf, uint8_t* y, int nb) {
    const int lane = threadIdx.x & 63;
    for (int b = threadIdx.x >> 6; b < nb; b += blockDim.x >> 6) {
        const float4 f = reinterpret_cast<const float4*>(buf + (size_t)b * 256)[lane];
        const float v[4] = {f.x, f.y, f.z, f.w};
        quantize_block_wave(v, lane, y, nb, b);
    }
}

}  // namespace g4
