// gemv.hip -- K-quant GEMV kernels for gfx950 (decode, batch 1).
//
// o[d] = W[d x n] . x   (W row-major, ne[0] = n; gemma4-4b/cpu-blas/main.c:1669)
//
// Work decomposition shared by all kernels: a 256-thread workgroup owns R
// consecutive rows; its 32 groups of 8 lanes walk (row, block) tasks in
// block-major order, so the groups of a wave read the same activation block
// from LDS (broadcast) while each streams a different row's 16-byte weight
// slices from HBM.  All weight loads of a group are issued before the
// activation is staged into LDS, so HBM latency overlaps the staging.
//
// Q4_K / Q5_K x Q8_K: per-block integer sums are computed in the lane
// partition of the reference's AVX2 dot (lane l = bytes 4l..4l+3 of every
// 32-byte chunk, main.c:500-523) and parked in LDS; the fp32 combine then
// replays main.c:476-529 (Q4_K) / 531-593 (Q5_K) exactly: eight FMA lanes
// over the blocks in order, the min term (four FMA lanes, or one scalar for
// Q5_K), and the fixed horizontal-add tree.  The result is bit-identical to
// the reference for the same Q8_K input.
//
// Q6_K x fp32 (mm_quant_rows, main.c:1539-1556): weights are dequantized to
// the reference's fp32 values ((d*sc)*q, main.c:226-229) and accumulated with
// FMA in a parallel order (tolerance, not bit-exact).
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

constexpr int kWG = 256;      // threads per workgroup
constexpr int kGroups = 32;   // 8-lane groups per workgroup

__device__ __forceinline__ uint32_t word_of(const uint4& v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// ------------------------------------------------------------------------
// Q4_K / Q5_K x Q8_K
// ------------------------------------------------------------------------
// LDS: [q8 copy: nb*292 B, padded to 16][S: Tmax*8 i32][P: Tmax*4 i32][D, DM: Tmax f32][res: 2R f32]
template <int TPG, bool Q5, int NMAT, bool DBG>
__global__ __launch_bounds__(kWG) void gemv_q45k_kernel(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                                        const uint8_t* __restrict__ q8, float* __restrict__ out, int nb,
                                                        int d, int R, int32_t* __restrict__ dbgS,
                                                        int32_t* __restrict__ dbgM) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int Tmax = kGroups * TPG;
    const int tid = threadIdx.x, l = tid & 7, g = tid >> 3;
    const int r0 = blockIdx.x * R;
    const int rows = min(R, d - r0);
    const int per_mat = rows * nb;
    const int T = NMAT * per_mat;
    const size_t nblk = (size_t)d * nb;
    const size_t hdr_off = Q5 ? q5k_planes(nblk).hdr : q4k_planes(nblk).hdr;
    const size_t qh_off = q5k_planes(nblk).qh;

    // ---- 1. issue every weight load of this group
    uint4 wq[TPG], hd[TPG];
    uint32_t qh[TPG];
#pragma unroll
    for (int i = 0; i < TPG; i++) {
        const int t = g + kGroups * i;
        wq[i] = make_uint4(0, 0, 0, 0);
        hd[i] = make_uint4(0, 0, 0, 0);
        qh[i] = 0;
        if (t < T) {
            const int m = NMAT == 2 ? t / per_mat : 0;
            const int tt = t - m * per_mat;
            const int b = tt / rows, rr = tt - b * rows;
            const uint8_t* base = m ? w1 : w0;
            const size_t blk = (size_t)(r0 + rr) * nb + b;
            wq[i] = *reinterpret_cast<const uint4*>(base + blk * 128 + 16 * l);
            hd[i] = *reinterpret_cast<const uint4*>(base + hdr_off + blk * 16);
            if (Q5) qh[i] = *reinterpret_cast<const uint32_t*>(base + qh_off + blk * 32 + 4 * l);
        }
    }
    // ---- 2. stage the Q8_K activation (qs | bsums | d) into LDS
    const int q8w = nb * 73;   // 292 B per block
    for (int k = tid; k < q8w; k += kWG) reinterpret_cast<uint32_t*>(smem)[k] = reinterpret_cast<const uint32_t*>(q8)[k];
    const int q8bytes = (nb * 292 + 15) & ~15;
    int32_t* S = reinterpret_cast<int32_t*>(smem + q8bytes);
    int32_t* P = S + Tmax * 8;
    float* D = reinterpret_cast<float*>(P + Tmax * 4);
    float* DM = D + Tmax;
    float* res = DM + Tmax;
    const int16_t* bsums = reinterpret_cast<const int16_t*>(smem + q8k_bsums_off(nb));
    const float* yd = reinterpret_cast<const float*>(smem + q8k_d_off(nb));
    __syncthreads();

    // ---- 3. exact per-block integer sums in the AVX2 lane partition
#pragma unroll
    for (int i = 0; i < TPG; i++) {
        const int t = g + kGroups * i;
        if (t < T) {
            const int m = NMAT == 2 ? t / per_mat : 0;
            const int tt = t - m * per_mat;
            const int b = tt / rows;
            uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
            unpack_scales(hd[i].y, hd[i].z, hd[i].w, sc_lo, sc_hi, mn_lo, mn_hi);
            const uint4 a0 = *reinterpret_cast<const uint4*>(smem + b * 256 + 32 * l);
            const uint4 a1 = *reinterpret_cast<const uint4*>(smem + b * 256 + 32 * l + 16);
            int32_t sumi = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t qw = word_of(wq[i], j);
                uint32_t lo = qw & 0x0f0f0f0fu, hi = (qw >> 4) & 0x0f0f0f0fu;
                if (Q5) {
                    lo |= ((qh[i] >> (2 * j)) & 0x01010101u) << 4;
                    hi |= ((qh[i] >> (2 * j + 1)) & 0x01010101u) << 4;
                }
                const int dl = __builtin_amdgcn_sdot4((int)lo, (int)word_of(a0, j), 0, false);
                const int dh = __builtin_amdgcn_sdot4((int)hi, (int)word_of(a1, j), 0, false);
                const uint32_t scw = j < 2 ? sc_lo : sc_hi;
                sumi += byte_of(scw, 2 * (j & 1)) * dl + byte_of(scw, 2 * (j & 1) + 1) * dh;
            }
            const int k = l & 3;
            const uint32_t mnw = k < 2 ? mn_lo : mn_hi;
            const int16_t* bs = bsums + b * 16 + 4 * k;
            const int32_t prod = byte_of(mnw, 2 * (k & 1)) * ((int)bs[0] + bs[1]) +
                                 byte_of(mnw, 2 * (k & 1) + 1) * ((int)bs[2] + bs[3]);
            if (DBG) {
                int32_t s = sumi;
                s += __shfl_xor(s, 1, 64);
                s += __shfl_xor(s, 2, 64);
                s += __shfl_xor(s, 4, 64);
                int32_t p = l < 4 ? prod : 0;
                p += __shfl_xor(p, 1, 64);
                p += __shfl_xor(p, 2, 64);
                p += __shfl_xor(p, 4, 64);
                if (l == 0) {
                    const int rr = tt - b * rows;
                    dbgS[(size_t)(r0 + rr) * nb + b] = s;
                    dbgM[(size_t)(r0 + rr) * nb + b] = p;
                }
            }
            S[t * 8 + l] = sumi;
            if (l < 4) P[t * 4 + l] = prod;
            if (l == 0) {
                const float y = yd[b];
                D[t] = y * f16_to_f32(hd[i].x & 0xffffu);
                DM[t] = -y * f16_to_f32(hd[i].x >> 16);
            }
        }
    }
    __syncthreads();
    if (DBG) return;

    // ---- 4. per-row fp32 combine, in the reference's order
    for (int ra = g; ra < NMAT * rows; ra += kGroups) {
        const int m = NMAT == 2 ? ra / rows : 0;
        const int rr = ra - m * rows;
        float acc = 0.0f, accm = 0.0f, summs = 0.0f;
        for (int b = 0; b < nb; b++) {
            const int t = m * per_mat + b * rows + rr;
            acc = __builtin_fmaf(D[t], (float)S[t * 8 + l], acc);
            if (Q5) {
                const int32_t pm = (P[t * 4 + 0] + P[t * 4 + 1]) + (P[t * 4 + 2] + P[t * 4 + 3]);
                const float tm = DM[t] * (float)pm;
                summs = summs + tm;
            } else if (l < 4) {
                accm = __builtin_fmaf(DM[t], (float)P[t * 4 + l], accm);
            }
        }
        const float t1 = acc + __shfl_xor(acc, 4, 64);
        const float t2 = t1 + __shfl_xor(t1, 2, 64);
        const float h = t2 + __shfl_xor(t2, 1, 64);
        float r;
        if (Q5) {
            r = h + summs;
        } else {
            const float v1 = accm + __shfl_xor(accm, 2, 64);
            const float hm = v1 + __shfl_xor(v1, 1, 64);
            r = h + hm;
        }
        if (l == 0) {
            if (NMAT == 1) out[r0 + rr] = r;
            else res[m * R + rr] = r;
        }
    }
    if (NMAT == 2) {
        __syncthreads();
        for (int rr = tid; rr < rows; rr += kWG) out[r0 + rr] = gelu_ref(res[rr]) * res[R + rr];
    }
}

// ------------------------------------------------------------------------
// Q6_K x fp32 (reference semantics of mm_quant_rows)
// ------------------------------------------------------------------------
// LDS: [x: n floats][part: Tmax floats]
template <int TPG, bool SOFTCAP>
__global__ __launch_bounds__(kWG) void gemv_q6k_f32_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                           float* __restrict__ out, int nb, int d, int R, float cap) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, L = tid & 7, g = tid >> 3, h = L >> 2, u = L & 3;
    const int r0 = blockIdx.x * R;
    const int rows = min(R, d - r0);
    const int T = rows * nb;
    const size_t nblk = (size_t)d * nb;
    const Q6KPlanes p = q6k_planes(nblk);

    uint4 qlv[TPG];
    uint2 qhv[TPG], scv[TPG];
    uint32_t dv[TPG];
#pragma unroll
    for (int i = 0; i < TPG; i++) {
        const int t = g + kGroups * i;
        qlv[i] = make_uint4(0, 0, 0, 0);
        qhv[i] = make_uint2(0, 0);
        scv[i] = make_uint2(0, 0);
        dv[i] = 0;
        if (t < T) {
            const int b = t / rows, rr = t - b * rows;
            const size_t blk = (size_t)(r0 + rr) * nb + b;
            qlv[i] = *reinterpret_cast<const uint4*>(w + p.ql + blk * 128 + 16 * L);
            qhv[i] = *reinterpret_cast<const uint2*>(w + p.qh + blk * 64 + 8 * L);
            scv[i] = *reinterpret_cast<const uint2*>(w + p.sc + blk * 16 + 8 * h);
            dv[i] = *reinterpret_cast<const uint16_t*>(w + p.d + blk * 2);
        }
    }
    float* xs = reinterpret_cast<float*>(smem);
    const int n4 = nb * 64;
    for (int k = tid; k < n4; k += kWG) reinterpret_cast<float4*>(xs)[k] = reinterpret_cast<const float4*>(x)[k];
    float* part = xs + nb * 256;
    __syncthreads();

#pragma unroll
    for (int i = 0; i < TPG; i++) {
        const int t = g + kGroups * i;
        if (t < T) {
            const int b = t / rows;
            const float df = f16_to_f32(dv[i]);
            float ds[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int sb = (u >> 1) + 2 * k;   // byte within the 8-byte half
                const uint32_t sw = sb < 4 ? scv[i].x : scv[i].y;
                ds[k] = df * (float)(int8_t)byte_of(sw, sb & 3);
            }
            const float* xb = xs + b * 256 + 128 * h + 8 * u;
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t qa = (k & 1) ? qlv[i].z : qlv[i].x;   // bytes 0..3 of the run
                const uint32_t qb = (k & 1) ? qlv[i].w : qlv[i].y;   // bytes 4..7
                const float4 x0 = *reinterpret_cast<const float4*>(xb + 32 * k);
                const float4 x1 = *reinterpret_cast<const float4*>(xb + 32 * k + 4);
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t qlb = byte_of(e < 4 ? qa : qb, e & 3);
                    const uint32_t lo = k < 2 ? (qlb & 15u) : (qlb >> 4);
                    const uint32_t hb = (byte_of(e < 4 ? qhv[i].x : qhv[i].y, e & 3) >> (2 * k)) & 3u;
                    const int q = (int)(lo | (hb << 4)) - 32;
                    const float wv = ds[k] * (float)q;
                    acc = __builtin_fmaf(xv[e], wv, acc);
                }
            }
            acc += __shfl_xor(acc, 1, 64);
            acc += __shfl_xor(acc, 2, 64);
            acc += __shfl_xor(acc, 4, 64);
            if (L == 0) part[t] = acc;
        }
    }
    __syncthreads();
    const float inv = SOFTCAP ? 1.0f / cap : 0.0f;
    for (int rr = tid; rr < rows; rr += kWG) {
        float s = 0.0f;
        for (int b = 0; b < nb; b++) s += part[b * rows + rr];
        if (SOFTCAP) s = cap * tanhf(s * inv);
        out[r0 + rr] = s;
    }
}

// ------------------------------------------------------------------------
// Q6_K x Q8_K (integer; no reference counterpart)
// ------------------------------------------------------------------------
template <int TPG>
__global__ __launch_bounds__(kWG) void gemv_q6k_q8k_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ q8,
                                                           float* __restrict__ out, int nb, int d, int R) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int Tmax = kGroups * TPG;
    const int tid = threadIdx.x, L = tid & 7, g = tid >> 3, h = L >> 2, u = L & 3;
    const int r0 = blockIdx.x * R;
    const int rows = min(R, d - r0);
    const int T = rows * nb;
    const size_t nblk = (size_t)d * nb;
    const Q6KPlanes p = q6k_planes(nblk);

    uint4 qlv[TPG];
    uint2 qhv[TPG], scv[TPG];
    uint32_t dv[TPG];
#pragma unroll
    for (int i = 0; i < TPG; i++) {
        const int t = g + kGroups * i;
        qlv[i] = make_uint4(0, 0, 0, 0);
        qhv[i] = make_uint2(0, 0);
        scv[i] = make_uint2(0, 0);
        dv[i] = 0;
        if (t < T) {
            const int b = t / rows, rr = t - b * rows;
            const size_t blk = (size_t)(r0 + rr) * nb + b;
            qlv[i] = *reinterpret_cast<const uint4*>(w + p.ql + blk * 128 + 16 * L);
            qhv[i] = *reinterpret_cast<const uint2*>(w + p.qh + blk * 64 + 8 * L);
            scv[i] = *reinterpret_cast<const uint2*>(w + p.sc + blk * 16 + 8 * h);
            dv[i] = *reinterpret_cast<const uint16_t*>(w + p.d + blk * 2);
        }
    }
    const int q8w = nb * 73;
    for (int k = tid; k < q8w; k += kWG) reinterpret_cast<uint32_t*>(smem)[k] = reinterpret_cast<const uint32_t*>(q8)[k];
    const int q8bytes = (nb * 292 + 15) & ~15;
    int32_t* Sb = reinterpret_cast<int32_t*>(smem + q8bytes);
    float* Db = reinterpret_cast<float*>(Sb + Tmax);
    const float* yd = reinterpret_cast<const float*>(smem + q8k_d_off(nb));
    __syncthreads();

#pragma unroll
    for (int i = 0; i < TPG; i++) {
        const int t = g + kGroups * i;
        if (t < T) {
            const int b = t / rows;
            const uint32_t* a = reinterpret_cast<const uint32_t*>(smem + b * 256);
            int32_t s = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t qa = (k & 1) ? qlv[i].z : qlv[i].x;
                const uint32_t qb = (k & 1) ? qlv[i].w : qlv[i].y;
                uint32_t lo_a = k < 2 ? (qa & 0x0f0f0f0fu) : ((qa >> 4) & 0x0f0f0f0fu);
                uint32_t lo_b = k < 2 ? (qb & 0x0f0f0f0fu) : ((qb >> 4) & 0x0f0f0f0fu);
                lo_a |= ((qhv[i].x >> (2 * k)) & 0x03030303u) << 4;
                lo_b |= ((qhv[i].y >> (2 * k)) & 0x03030303u) << 4;
                // bytes q in [0,63] -> (q - 32) as int8, per byte without borrows
                const uint32_t sa = ((lo_a | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                const uint32_t sb2 = ((lo_b | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
                const int gw = 32 * h + 8 * k + 2 * u;   // GGUF-order q8 word of this run
                const int dot = __builtin_amdgcn_sdot4((int)sa, (int)a[q8k_word_dev(gw)], 0, false) +
                                __builtin_amdgcn_sdot4((int)sb2, (int)a[q8k_word_dev(gw + 1)], 0, false);
                const int sbi = (u >> 1) + 2 * k;
                const int8_t sc = (int8_t)byte_of(sbi < 4 ? scv[i].x : scv[i].y, sbi & 3);
                s += sc * dot;
            }
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            s += __shfl_xor(s, 4, 64);
            if (L == 0) {
                Sb[t] = s;
                Db[t] = f16_to_f32(dv[i]) * yd[b];
            }
        }
    }
    __syncthreads();
    for (int rr = tid; rr < rows; rr += kWG) {
        float acc = 0.0f;
        for (int b = 0; b < nb; b++) acc = __builtin_fmaf(Db[b * rows + rr], (float)Sb[b * rows + rr], acc);
        out[r0 + rr] = acc;
    }
}

// ------------------------------------------------------------------------
// BF16 x fp32 (mm_bf16, main.c:1529-1537)
// ------------------------------------------------------------------------
// one wave per row, RPW rows per wave, CPL 16-byte chunks per lane
template <int RPW, int CPL>
__global__ __launch_bounds__(kWG) void gemv_bf16_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                        float* __restrict__ out, int n, int d) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nch = n / 8;
    const int row0 = (blockIdx.x * 4 + wave) * RPW;
    uint4 v[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int ch = lane + 64 * c, row = row0 + r;
            v[r][c] = (row < d && ch < nch) ? reinterpret_cast<const uint4*>(w + (size_t)row * n)[ch] : make_uint4(0, 0, 0, 0);
        }
    for (int k = tid; k < n / 4; k += kWG) reinterpret_cast<float4*>(xs)[k] = reinterpret_cast<const float4*>(x)[k];
    __syncthreads();
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
        acc = wave_sum(acc);
        if (lane == 0 && row0 + r < d) out[row0 + r] = acc;
    }
}

}  // namespace g4

using namespace g4;

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------
namespace {

int g_wg_per_cu = 4;   // occupancy target for the tiling choice

// Choose TPG (tasks per 8-lane group, a template value) and R (rows per
// workgroup) so that the grid has >= g_wg_per_cu workgroups per CU where the
// matrix allows it, with as many loads in flight per lane as possible.
bool pick_tiling(int nb, int d, int nmat, int* tpg, int* R) {
    const int target = g_wg_per_cu * g4_num_cus();
    static const int cand[4] = {8, 4, 2, 1};
    for (int t : cand) {
        const int r = kGroups * t / (nmat * nb);
        if (r < 1) continue;
        if ((d + r - 1) / r >= target) { *tpg = t; *R = r; return true; }
    }
    for (int i = 3; i >= 0; i--) {
        const int t = cand[i];
        const int r = kGroups * t / (nmat * nb);
        if (r >= 1) { *tpg = t; *R = r; return true; }
    }
    return false;
}

size_t q45_lds(int nb, int tpg, int R) {
    return (size_t)((nb * 292 + 15) & ~15) + (size_t)kGroups * tpg * 56 + (size_t)2 * R * 4;
}

template <bool Q5, int NMAT, bool DBG>
int launch_q45(const void* w0, const void* w1, const void* q8, float* o, int nb, int d, int32_t* S, int32_t* M) {
    int tpg = 1, R = 1;
    if (!pick_tiling(nb, d, NMAT, &tpg, &R)) return g4_fail(G4_ERR_ARG, "GEMV: row length %d blocks too long", nb);
    const dim3 grid((d + R - 1) / R);
    const size_t lds = q45_lds(nb, tpg, R);
    const uint8_t *a = (const uint8_t*)w0, *b = (const uint8_t*)w1, *q = (const uint8_t*)q8;
    switch (tpg) {
    case 8: hipLaunchKernelGGL((gemv_q45k_kernel<8, Q5, NMAT, DBG>), grid, dim3(kWG), lds, g4_stream(), a, b, q, o, nb, d, R, S, M); break;
    case 4: hipLaunchKernelGGL((gemv_q45k_kernel<4, Q5, NMAT, DBG>), grid, dim3(kWG), lds, g4_stream(), a, b, q, o, nb, d, R, S, M); break;
    case 2: hipLaunchKernelGGL((gemv_q45k_kernel<2, Q5, NMAT, DBG>), grid, dim3(kWG), lds, g4_stream(), a, b, q, o, nb, d, R, S, M); break;
    default: hipLaunchKernelGGL((gemv_q45k_kernel<1, Q5, NMAT, DBG>), grid, dim3(kWG), lds, g4_stream(), a, b, q, o, nb, d, R, S, M); break;
    }
    return g4_check_launch("gemv_q45k_kernel");
}

template <bool SOFTCAP>
int launch_q6_f32(const void* w, const float* x, float* o, int nb, int d, float cap) {
    int tpg = 1, R = 1;
    if (!pick_tiling(nb, d, 1, &tpg, &R)) return g4_fail(G4_ERR_ARG, "GEMV: row length %d blocks too long", nb);
    const dim3 grid((d + R - 1) / R);
    const size_t lds = (size_t)nb * 1024 + (size_t)kGroups * tpg * 4;
    const uint8_t* a = (const uint8_t*)w;
    switch (tpg) {
    case 8: hipLaunchKernelGGL((gemv_q6k_f32_kernel<8, SOFTCAP>), grid, dim3(kWG), lds, g4_stream(), a, x, o, nb, d, R, cap); break;
    case 4: hipLaunchKernelGGL((gemv_q6k_f32_kernel<4, SOFTCAP>), grid, dim3(kWG), lds, g4_stream(), a, x, o, nb, d, R, cap); break;
    case 2: hipLaunchKernelGGL((gemv_q6k_f32_kernel<2, SOFTCAP>), grid, dim3(kWG), lds, g4_stream(), a, x, o, nb, d, R, cap); break;
    default: hipLaunchKernelGGL((gemv_q6k_f32_kernel<1, SOFTCAP>), grid, dim3(kWG), lds, g4_stream(), a, x, o, nb, d, R, cap); break;
    }
    return g4_check_launch("gemv_q6k_f32_kernel");
}

int launch_q6_q8(const void* w, const void* q8, float* o, int nb, int d) {
    int tpg = 1, R = 1;
    if (!pick_tiling(nb, d, 1, &tpg, &R)) return g4_fail(G4_ERR_ARG, "GEMV: row length %d blocks too long", nb);
    const dim3 grid((d + R - 1) / R);
    const size_t lds = (size_t)((nb * 292 + 15) & ~15) + (size_t)kGroups * tpg * 8;
    const uint8_t *a = (const uint8_t*)w, *q = (const uint8_t*)q8;
    switch (tpg) {
    case 8: hipLaunchKernelGGL((gemv_q6k_q8k_kernel<8>), grid, dim3(kWG), lds, g4_stream(), a, q, o, nb, d, R); break;
    case 4: hipLaunchKernelGGL((gemv_q6k_q8k_kernel<4>), grid, dim3(kWG), lds, g4_stream(), a, q, o, nb, d, R); break;
    case 2: hipLaunchKernelGGL((gemv_q6k_q8k_kernel<2>), grid, dim3(kWG), lds, g4_stream(), a, q, o, nb, d, R); break;
    default: hipLaunchKernelGGL((gemv_q6k_q8k_kernel<1>), grid, dim3(kWG), lds, g4_stream(), a, q, o, nb, d, R); break;
    }
    return g4_check_launch("gemv_q6k_q8k_kernel");
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_gemv(const char* who, const void* o, const void* w, const void* x, int n, int d) {
    if (!o || !w || !x) return g4_fail(G4_ERR_ARG, "%s: null pointer", who);
    if (!aligned16(w) || !aligned16(x)) return g4_fail(G4_ERR_ARG, "%s: w and x must be 16-byte aligned", who);
    if (n <= 0 || d <= 0 || n % 256) return g4_fail(G4_ERR_ARG, "%s: n=%d not a positive multiple of QK_K, d=%d", who, n, d);
    if (n > 256 * 48) return g4_fail(G4_ERR_ARG, "%s: n=%d exceeds 12288", who, n);
    return G4_OK;
}

}  // namespace

extern "C" int g4_set_gemv_occupancy(int wg_per_cu) {
    G4_CHECK_ARG(wg_per_cu >= 1 && wg_per_cu <= 64, "g4_set_gemv_occupancy: %d out of range", wg_per_cu);
    g_wg_per_cu = wg_per_cu;
    return G4_OK;
}

extern "C" int g4_mm_quant_dot_rows(float* o, const void* w, int n, int d, int type, const void* q8) {
    int rc = check_gemv("g4_mm_quant_dot_rows", o, w, q8, n, d);
    if (rc) return rc;
    const int nb = n / 256;
    switch (type) {
    case G4_Q4_K: return launch_q45<false, 1, false>(w, nullptr, q8, o, nb, d, nullptr, nullptr);
    case G4_Q5_K: return launch_q45<true, 1, false>(w, nullptr, q8, o, nb, d, nullptr, nullptr);
    case G4_Q6_K: return launch_q6_q8(w, q8, o, nb, d);
    default: return g4_fail(G4_ERR_TYPE, "vec_dot_row_q8_K: unsupported type %d", type);
    }
}

extern "C" int g4_vec_dot_q4_K_q8_K(int n, const void* x, const void* y, float* out) {
    return g4_mm_quant_dot_rows(out, x, n, 1, G4_Q4_K, y);
}
extern "C" int g4_vec_dot_q5_K_q8_K(int n, const void* x, const void* y, float* out) {
    return g4_mm_quant_dot_rows(out, x, n, 1, G4_Q5_K, y);
}
extern "C" int g4_vec_dot_q6_K_q8_K(int n, const void* x, const void* y, float* out) {
    return g4_mm_quant_dot_rows(out, x, n, 1, G4_Q6_K, y);
}

extern "C" int g4_mm_quant_rows(float* o, const float* x, const void* w, int n, int d, int type) {
    int rc = check_gemv("g4_mm_quant_rows", o, w, x, n, d);
    if (rc) return rc;
    if (type != G4_Q6_K) return g4_fail(G4_ERR_TYPE, "g4_mm_quant_rows: type %d not supported (Q6_K only)", type);
    return launch_q6_f32<false>(w, x, o, n / 256, d, 0.0f);
}

// LM head: mm_quant_rows followed by the logit soft-cap (main.c:1788-1795)
extern "C" int g4_mm_quant_rows_softcap(float* o, const float* x, const void* w, int n, int d, int type, float cap) {
    int rc = check_gemv("g4_mm_quant_rows_softcap", o, w, x, n, d);
    if (rc) return rc;
    if (type != G4_Q6_K) return g4_fail(G4_ERR_TYPE, "g4_mm_quant_rows_softcap: type %d not supported", type);
    if (!(cap > 0.0f)) return launch_q6_f32<false>(w, x, o, n / 256, d, 0.0f);
    return launch_q6_f32<true>(w, x, o, n / 256, d, cap);
}

extern "C" int g4_mm_bf16(float* o, const float* x, const void* w, int n, int d) {
    if (!o || !x || !w) return g4_fail(G4_ERR_ARG, "g4_mm_bf16: null pointer");
    if (!aligned16(w) || !aligned16(x)) return g4_fail(G4_ERR_ARG, "g4_mm_bf16: w and x must be 16-byte aligned");
    if (n <= 0 || d <= 0 || n % 8 || n > 4096) return g4_fail(G4_ERR_ARG, "g4_mm_bf16: n=%d unsupported (multiple of 8, <= 4096)", n);
    const int cpl = (n / 8 + 63) / 64;
    const size_t lds = (size_t)n * 4;
    const dim3 grid((d + 7) / 8);
    const uint16_t* wp = (const uint16_t*)w;
    if (cpl <= 4) hipLaunchKernelGGL((gemv_bf16_kernel<2, 4>), grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    else hipLaunchKernelGGL((gemv_bf16_kernel<2, 8>), grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    return g4_check_launch("gemv_bf16_kernel");
}

extern "C" int g4_mm(float* o, const float* x, const void* w, int n, int d, int type, void* q8, int q8_ready) {
    switch (type) {
    case G4_Q4_K:
    case G4_Q5_K: {
        if (n % 256) return g4_fail(G4_ERR_ARG, "mm: n=%d not multiple of QK_K", n);
        if (!q8_ready) {
            int rc = g4_quantize_row_q8_K(x, q8, n);
            if (rc) return rc;
        }
        return g4_mm_quant_dot_rows(o, w, n, d, type, q8);
    }
    case G4_Q6_K: return g4_mm_quant_rows(o, x, w, n, d, type);
    case G4_BF16: return g4_mm_bf16(o, x, w, n, d);
    default: return g4_fail(G4_ERR_TYPE, "Unsupported tensor type %d in matmul", type);
    }
}

extern "C" int g4_mm_gate_up_gelu(float* hb, const void* gate, const void* up, int n, int d, int type, const void* q8) {
    int rc = check_gemv("g4_mm_gate_up_gelu", hb, gate, q8, n, d);
    if (rc) return rc;
    if (!up || !aligned16(up)) return g4_fail(G4_ERR_ARG, "g4_mm_gate_up_gelu: bad up pointer");
    const int nb = n / 256;
    if (type == G4_Q4_K) return launch_q45<false, 2, false>(gate, up, q8, hb, nb, d, nullptr, nullptr);
    if (type == G4_Q5_K) return launch_q45<true, 2, false>(gate, up, q8, hb, nb, d, nullptr, nullptr);
    return g4_fail(G4_ERR_TYPE, "g4_mm_gate_up_gelu: type %d not supported", type);
}

extern "C" int g4_debug_block_sums(const void* w, int n, int d, int type, const void* q8, int32_t* S, int32_t* M) {
    int rc = check_gemv("g4_debug_block_sums", S, w, q8, n, d);
    if (rc) return rc;
    if (!M) return g4_fail(G4_ERR_ARG, "g4_debug_block_sums: null M");
    const int nb = n / 256;
    if (type == G4_Q4_K) return launch_q45<false, 1, true>(w, nullptr, q8, nullptr, nb, d, S, M);
    if (type == G4_Q5_K) return launch_q45<true, 1, true>(w, nullptr, q8, nullptr, nb, d, S, M);
    return g4_fail(G4_ERR_TYPE, "g4_debug_block_sums: type %d not supported", type);
}
