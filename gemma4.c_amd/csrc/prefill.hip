// prefill.hip -- many tokens through one weight matrix at once (prefill):
// Y[m x d] = X[m x n] . W[d x n]^T on the gfx950 matrix cores.  The
// reference has no batched path: generate() calls forward() once per prompt
// token (gemma4-4b/cpu-blas/main.c:2366-2384), i.e. quantize_row_q8_K +
// mm_quant_dot_rows per token for Q4_K / Q5_K and mm_quant_rows / mm_bf16 on
// the fp32 activations for Q6_K / bf16.  Every kernel here computes the same
// sums from the same integer codes and scales; only the fp32 rounding of the
// partial sums differs from the per-token dot, so the bar is the GEMVs' one,
// 1e-5 of sum |w x|.  Each token's outputs are a fixed function of that
// token's activations (no split over tokens or K that depends on the batch),
// so a prompt gives the same bits in any chunking.
//
// Q4_K / Q5_K (mm_batch_kq8_kernel).  The reference's dot per block is
//   y.d * d * sum_j sc_j * sum_e q_e * q8_e  -  y.d * dmin * sum_j m_j * bs_j
// (vec_dot_q4_K_q8_K / vec_dot_q5_K_q8_K, main.c:476-529, 531-593; bs_j =
// the two 16-element bsums of sub-block j).  The inner sums run on the int8
// matrix cores, v_mfma_i32_32x32x32_i8, one product per sub-block (K = its
// 32 codes: the 4/5-bit q against the int8 q8), exact in int32; the 6-bit
// sub-block scale cannot ride in an int8 operand (sc * q reaches 1953), so
// S_b = sum_j sc_j * acc_j is formed in int32 (|S_b| <= 256 * 63 * 31 * 128
// = 6.4e7).  The min sum M_b (|M_b| <= 16 * 63 * 2048, exact) is two
// v_mfma_f32_32x32x8_f16 on the bsums and mins, and the block is folded into
// the fp32 accumulator with three VALU operations per output:
// fma(y.d, fma(d, S_b, -(dmin * M_b)), acc).  MODE 2 stores the int32 S_b
// and M_b of every (token, row, block) instead (g4_debug_batch_block_sums).
// The weights are the B operand, so a lane's outputs share one weight row
// and its d, dmin and scales come from the block header the lane loads
// itself.  Work split: a workgroup of 4 or 5 waves owns 32 weight rows per
// wave x 32 tokens; per block it stages its tokens' Q8_K codes in LDS as
// they are, each sub-block's 32 positions contiguous, and each wave builds
// its weight operands (nibbles as bytes) in registers from 64 contiguous
// bytes per lane, loaded one block ahead.  Against the same kernel on the
// fp16 matrix cores (codes * scale as fp16, chained in exact pieces): the
// same bits, Q4_K 4-12 % and Q5_K 11-25 % less time at the E4B prompt
// shapes (511 tokens).
//
// Q6_K (mm_batch_q6s_kernel).  The reference dequantizes each weight to
// d * sc * (q - 32) in fp32 (exact: 11 + 7 + 5 significant bits) and
// multiplies by the fp32 activations (mm_quant_rows, main.c:1539-1556,
// dequant_q6_k main.c:213-236).  Here:
//   * each activation row is split (g4_split_rows_f16) into two fp16 terms
//     after scaling by a power of two that brings its largest |x| into
//     [2^14, 2^15): x * 2^-s = hi + lo + r with |r| <= 2^-22 |x * 2^-s| (or
//     below 2^-25 in the scaled units, for elements in fp16's subnormal range);
//   * the integer weight w = sc * (q - 32) (|w| <= 4096) is split exactly
//     into Wh = fp16(w) and Wl = w - Wh in {-1, 0, 1} (nonzero only for odd
//     |w| > 2048);
//   * three fp16 MFMAs per 32 weights, Wh hi + Wh lo + Wl hi, give
//     sum sc * (q - 32) * x over a block with exact products (the dropped
//     Wl lo is below 2^-22 of its term), chained in one fp32 accumulator; the
//     block's fp16 d is applied with one FMA per output, and the token's 2^s
//     at the end (exact).
// The bf16 matrices and the workspace-free g4_mm_batch entry keep the fp32
// MFMA kernel (mm_batch_f32_kernel, below).
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));


__device__ __forceinline__ uint32_t h2_bits(h2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ h2_t bits_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }

// fp16 of the half-word pattern 0x64XX is 1024 + XX (XX < 256)
constexpr uint32_t kMagic = 0x64646464u;
constexpr uint32_t kSelLo = 0x04010400u;   // bytes (c0, 0x64, c1, 0x64)
constexpr uint32_t kSelHi = 0x04030402u;   // bytes (c2, 0x64, c3, 0x64)

// four int8 (one little-endian word) -> four exact fp16: q ^ 0x80 = q + 128
__device__ __forceinline__ uint2 i8x4_to_h4(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const h2_t c = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2_t lo = bits_h2(__builtin_amdgcn_perm(kMagic, u, kSelLo)) + c;
    const h2_t hi = bits_h2(__builtin_amdgcn_perm(kMagic, u, kSelHi)) + c;
    return make_uint2(h2_bits(lo), h2_bits(hi));
}

__device__ __forceinline__ float hbits_to_f32(uint32_t h) {
    _Float16 v;
    const uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// XCD-aware tile order.  Workgroups go to the 8 XCDs round robin by their
// linear id; tile t = (row group t / gy, token group t % gy) is given to id
// so that each XCD takes a contiguous run of tiles, i.e. a few row groups
// with all their token groups: the weights of those rows stay in that XCD's
// L2 while its workgroups stream the activations.  (A bijection on ids for
// any tile count; grid = gx * gy workgroups in x.)
__device__ __forceinline__ void xcd_tile(int gy, int& bx, int& by) {
    const int n = gridDim.x, id = blockIdx.x;
    const int q = n >> 3, r = n & 7, x = id & 7, l = id >> 3;
    const int t = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + l;
    bx = t / gy;
    by = t - bx * gy;
}

// buffer-resource loads (word 3 of the descriptor: 32-bit data format, the
// value the gfx9 family takes for raw byte-addressed buffers)
constexpr int kBufWord3 = 0x00020000;
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ uint2 buf_load8(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// Workgroup barrier for LDS hand-offs: this wave's LDS operations complete,
// then s_barrier.  __syncthreads() also waits for every outstanding global
// load (its release fence), which would make each block wait for the next
// block's prefetch; here the loads stay in flight across the barrier.  The
// asm is a compiler barrier for memory operations as well.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt immediate that waits until at most n vector memory operations
// are outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt and
// lgkmcnt left at their maxima, i.e. not waited for)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

typedef float f16v_t __attribute__((ext_vector_type(16)));
constexpr int kKqTok = 528;   // LDS bytes per staged token: 512 of fp16 + pad
constexpr int kKqBs = 40;     // LDS bytes per token of fp16 bsums: 32 + pad

// up to kMaxSegs matrices over the same activations in one launch: segment
// s owns row groups [g0[s], g0[s + 1]) of 128 rows
constexpr int kMaxSegs = 4;
struct KqSegs {
    const uint8_t* w[kMaxSegs];
    float* o[kMaxSegs];
    int d[kMaxSegs];
    int g0[kMaxSegs + 1];
    int n;
};

// K steps (16 products each) per exactly summed chain of a block's S_b
template <bool Q5>
constexpr int kChainSteps = Q5 ? 4 : 8;

// after K step s of a block: at the end of a chain, keep its exact sum
// (Q4_K: the first chain in P; Q5_K: added into the int32 sum SI)
template <bool Q5>
__device__ __forceinline__ void chain_end(int s, const f16v_t& S, f16v_t& P, int (&SI)[16]) {
    constexpr int CS = kChainSteps<Q5>;
    if (s % CS != CS - 1) return;
    if (Q5) {
#pragma unroll
        for (int v = 0; v < 16; v++) SI[v] = (s == CS - 1 ? 0 : SI[v]) + (int)S[v];
    } else if (s == CS - 1) {
        P = S;
    }
}

// output v's S_b as fp32: Q4_K the fp32 sum of two exact chains (the exact
// integer rounded once), Q5_K the int32 sum converted
template <bool Q5>
__device__ __forceinline__ float chain_block_sum(const f16v_t& S, const f16v_t& P, const int (&SI)[16], int v) {
    return Q5 ? (float)SI[v] : P[v] + S[v];
}

// the int32 S_b and M_b of output v = 8 (v >> 2) + (v & 3) of token t0 + ...
template <bool Q5>
__device__ __forceinline__ void store_block_sums(int32_t* So, int32_t* Mo, const f16v_t& S, const f16v_t& P,
                                                 const int (&SI)[16], const f16v_t& M, int row, int d, int t0, int m,
                                                 int nb, int b) {
    if (row >= d) return;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int tok = t0 + 8 * (v >> 2) + (v & 3);
        if (tok >= m) continue;
        const size_t o = ((size_t)tok * d + row) * nb + b;
        So[o] = Q5 ? SI[v] : (int)P[v] + (int)S[v];
        Mo[o] = (int)M[v];
    }
}

// ---- Q4_K / Q5_K on the int8 matrix cores (mm_batch_kq8_kernel) ----------
// Lane (i, kg) of a wave owns weight row 32 w + i and, in every sub-block,
// positions 16 kg .. 16 kg + 15: of the device qs plane it loads words
// 16 kg .. 16 kg + 15 of the block (bytes 16 kg .. 16 kg + 15 of each 32-byte
// chunk c, whose low nibbles are sub-block 2c and high nibbles 2c + 1), so
// word q of chunk c gives positions 16 kg + 4q .. +3 of both sub-blocks.
// The activations are staged per token with position p of sub-block j at
// byte 32 j + p, so lane half kg's A operand is one 16-byte LDS read.
constexpr int kKq8Tok = 272;   // LDS bytes per staged token: 256 codes + pad

// MODE 0: the outputs.  MODE 1 (PB): one block per workgroup (blockIdx.y),
// whose per-block term u (before the token's Q8_K d) is stored instead of
// folded: out gets nb slices of m x d.  MODE 2 (DB): every block's int32 S_b
// and M_b into S = o[0] and M = o[1], each [m][d][nb] (one segment).
template <bool Q5, int NT, int NWV, int MODE = 0>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2))) void mm_batch_kq8_kernel(
    const KqSegs sg, const uint8_t* __restrict__ q8, int nb, int m) {
    constexpr bool PB = MODE == 1, DB = MODE == 2;
    constexpr int NTH = 64 * NWV;
    constexpr int TOK = 32 * NT;
    constexpr int UPT = (TOK * 8 + NTH - 1) / NTH;
    constexpr int BQ = (TOK * 4 + NTH - 1) / NTH;
    __shared__ __align__(16) uint8_t sA[2][TOK * kKq8Tok];
    __shared__ __align__(16) uint8_t sS[2][TOK * kKqBs];
    __shared__ __align__(16) float sD[2][TOK];
    typedef int i4v_t __attribute__((ext_vector_type(4)));
    typedef int i16v_t __attribute__((ext_vector_type(16)));

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 31, kg = lane >> 5;
    int bx, by;
    xcd_tile((m + TOK - 1) / TOK, bx, by);
    int seg = 0;
#pragma unroll
    for (int k = 1; k < kMaxSegs; k++)
        if (k < sg.n && bx >= sg.g0[k]) seg = k;
    const uint8_t* __restrict__ w = sg.w[seg];
    const int d = sg.d[seg];
    float* __restrict__ out = sg.o[seg] + (PB ? (size_t)blockIdx.y * m * d : 0);
    const int b0 = PB ? (int)blockIdx.y : 0, b1 = PB ? b0 + 1 : nb;   // this workgroup's blocks
    const int row = (bx - sg.g0[seg]) * (32 * NWV) + wave * 32 + i;
    const int tokb = by * TOK;
    const size_t nblk = (size_t)d * nb;
    const size_t hdr_off = (Q5 ? 160 : 128) * nblk, qh_off = 128 * nblk;
    const size_t q8row = ((size_t)nb * 292 + 63) & ~(size_t)63;
    const size_t rB = (size_t)min(row, d - 1) * nb;

    struct WRaw {
        uint4 qs[4];
        uint4 qh;
        uint4 hdr;
    };
    struct XRaw {
        uint4 a0[UPT], a1[UPT];
        uint2 bs[BQ];
        float yd;
    };
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)(hdr_off + 16 * nblk), kBufWord3);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)q8, (short)0, (int)(m * q8row), kBufWord3);
    const int vqs = (int)(rB * 128) + 64 * kg, vqh = (int)(qh_off + rB * 32) + 16 * kg, vhdr = (int)(hdr_off + rB * 16);
    int vx[UPT], vbs[BQ];
#pragma unroll
    for (int j = 0; j < UPT; j++) {
        const int u = min(tid + j * NTH, TOK * 8 - 1);
        vx[j] = min(tokb + (u >> 3), m - 1) * (int)q8row + 32 * (u & 7);
    }
#pragma unroll
    for (int j = 0; j < BQ; j++) {
        const int u = min(tid + j * NTH, TOK * 4 - 1);
        vbs[j] = min(tokb + (u >> 2), m - 1) * (int)q8row + (int)q8k_bsums_off(nb) + 8 * (u & 3);
    }
    const int vyd = min(tokb + min(tid, TOK - 1), m - 1) * (int)q8row + (int)q8k_d_off(nb);
    auto load_w = [&](int b, WRaw& r) {
#pragma unroll
        for (int q = 0; q < 4; q++) r.qs[q] = buf_load16(rw, vqs + 16 * q, b * 128);
        if (Q5) r.qh = buf_load16(rw, vqh, b * 32);
        r.hdr = buf_load16(rw, vhdr, b * 16);
    };
    auto load_x = [&](int b, XRaw& r) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            r.a0[j] = buf_load16(rq, vx[j], b * 256);
            r.a1[j] = buf_load16(rq, vx[j] + 16, b * 256);
        }
#pragma unroll
        for (int j = 0; j < BQ; j++) r.bs[j] = buf_load8(rq, vbs[j], b * 32);
        r.yd = __uint_as_float(buf_load4(rq, vyd, b * 4));
    };
    // unit (t, l'): device Q8_K words 8l' + 4h + jj hold sub-block 2jj + h,
    // positions 4l' .. 4l'+3; staged at 32 (2jj + h) + 4l' of the token's row
    auto stage = [&](const XRaw& r, int st) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * NTH, lq = u & 7;
            if (UPT * NTH != TOK * 8 && u >= TOK * 8) continue;
            uint8_t* dst = sA[st] + (u >> 3) * kKq8Tok + 4 * lq;
            const uint32_t wd[8] = {r.a0[j].x, r.a0[j].y, r.a0[j].z, r.a0[j].w,
                                    r.a1[j].x, r.a1[j].y, r.a1[j].z, r.a1[j].w};
#pragma unroll
            for (int k = 0; k < 8; k++) {   // k = 4h + jj
                const int h = k >> 2, jj = k & 3;
                *reinterpret_cast<uint32_t*>(dst + 32 * (2 * jj + h)) = wd[k];
            }
        }
#pragma unroll
        for (int j = 0; j < BQ; j++) {
            const int u = tid + j * NTH;
            if (u < TOK * 4) {
                const h2_t lo = {(_Float16)(int16_t)(r.bs[j].x & 0xffffu), (_Float16)(int16_t)(r.bs[j].x >> 16)};
                const h2_t hi = {(_Float16)(int16_t)(r.bs[j].y & 0xffffu), (_Float16)(int16_t)(r.bs[j].y >> 16)};
                *reinterpret_cast<uint2*>(sS[st] + (u >> 2) * kKqBs + 8 * (u & 3)) = make_uint2(h2_bits(lo), h2_bits(hi));
            }
        }
        if (tid < TOK) sD[st][tid] = r.yd;
    };

    f16v_t acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[nt][v] = 0.0f;
    f16v_t zero;
    i16v_t izero;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        zero[v] = 0.0f;
        izero[v] = 0;
    }

    // one block from stage st: after the barrier (block b's activations are
    // in st, and every wave is done with the other stage), the next block's
    // weight loads; half-way through the products, block b + 1's activations
    // (loaded during block b - 1) go into the other stage and block b + 2's
    // loads start (the block loop runs two blocks per trip so that the sets
    // alternate without copies; loads past the end repeat the last block: no
    // branch, so the compiler's waits for them are exact)
    XRaw xn;
    auto block = [&](int b, int st, const WRaw& wc, WRaw& wnext) {
        lds_barrier();
        if (!PB) load_w(min(b + 1, nb - 1), wnext);
        uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
        unpack_scales(wc.hdr.y, wc.hdr.z, wc.hdr.w, sc_lo, sc_hi, mn_lo, mn_hi);
        int SI[NT][16];
        const uint8_t* at0 = sA[st] + i * kKq8Tok + 16 * kg;
#pragma unroll
        for (int sb = 0; sb < 8; sb++) {
            if (!PB && sb == 4 && b + 1 < b1) {
                stage(xn, st ^ 1);
                load_x(min(b + 2, nb - 1), xn);
            }
            const int c = sb >> 1, h = sb & 1;
            uint32_t cw[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t word = c == 0 ? wc.qs[q].x : c == 1 ? wc.qs[q].y : c == 2 ? wc.qs[q].z : wc.qs[q].w;
                uint32_t v = h ? (word >> 4) & 0x0f0f0f0fu : word & 0x0f0f0f0fu;
                if (Q5) {
                    const uint32_t hw = q == 0 ? wc.qh.x : q == 1 ? wc.qh.y : q == 2 ? wc.qh.z : wc.qh.w;
                    v |= ((hw >> sb) & 0x01010101u) << 4;
                }
                cw[q] = v;
            }
            const i4v_t B = {(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
            const int scv = byte_of(sb < 4 ? sc_lo : sc_hi, sb & 3);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const i4v_t A = *reinterpret_cast<const i4v_t*>(at0 + 32 * nt * kKq8Tok + 32 * sb);
                const i16v_t Z = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, izero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 16; v++) SI[nt][v] = (sb == 0 ? 0 : SI[nt][v]) + __mul24(scv, Z[v]);
            }
        }
        const int msh = 16 * kg;
        const _Float16 m0 = (_Float16)(float)((mn_lo >> msh) & 0xffu), m1 = (_Float16)(float)((mn_lo >> (msh + 8)) & 0xffu);
        const _Float16 m4 = (_Float16)(float)((mn_hi >> msh) & 0xffu), m5 = (_Float16)(float)((mn_hi >> (msh + 8)) & 0xffu);
        const h4_t Bm1 = {m0, m0, m1, m1}, Bm2 = {m4, m4, m5, m5};
        const float dx = hbits_to_f32(wc.hdr.x & 0xffffu), dmx = hbits_to_f32(wc.hdr.x >> 16);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint8_t* bs = sS[st] + (32 * nt + i) * kKqBs + 8 * kg;
            const h4_t A1 = *reinterpret_cast<const h4_t*>(bs), A2 = *reinterpret_cast<const h4_t*>(bs + 16);
            f16v_t M = __builtin_amdgcn_mfma_f32_32x32x8f16(A1, Bm1, zero, 0, 0, 0);
            M = __builtin_amdgcn_mfma_f32_32x32x8f16(A2, Bm2, M, 0, 0, 0);
            if (DB) {
                if (row < d) {
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int tok = tokb + 32 * nt + 8 * (v >> 2) + 4 * kg + (v & 3);
                        if (tok >= m) continue;
                        const size_t o = ((size_t)tok * d + row) * nb + b;
                        reinterpret_cast<int32_t*>(sg.o[0])[o] = SI[nt][v];
                        reinterpret_cast<int32_t*>(sg.o[1])[o] = (int)M[v];
                    }
                }
                continue;
            }
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const float4 yd = *reinterpret_cast<const float4*>(sD[st] + 32 * nt + 8 * a + 4 * kg);
                const float y4[4] = {yd.x, yd.y, yd.z, yd.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int v = 4 * a + c;
                    const float u = __builtin_fmaf(dx, (float)SI[nt][v], -(dmx * M[v]));
                    acc[nt][v] = PB ? u : __builtin_fmaf(y4[c], u, acc[nt][v]);
                }
            }
        }
    };
    WRaw w0, w1;
    load_w(b0, w0);
    load_x(b0, xn);
    stage(xn, 0);
    if (!PB) load_x(min(b0 + 1, nb - 1), xn);
    for (int b = b0; b < b1; b += 2) {
        block(b, 0, w0, w1);
        if (b + 1 < b1) block(b + 1, 1, w1, w0);
    }
    if (!DB && row < d) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int tok = tokb + 32 * nt + 8 * (v >> 2) + 4 * kg + (v & 3);
                if (tok < m) out[(size_t)tok * d + row] = acc[nt][v];
            }
    }
}

template <bool Q5, int NT, int NWV, int MODE = 0>
void launch_mm_batch8(const KqSegs& sg, const uint8_t* q8, int nb, int m) {
    const int gy = (m + 32 * NT - 1) / (32 * NT);
    hipLaunchKernelGGL((mm_batch_kq8_kernel<Q5, NT, NWV, MODE>), dim3(sg.g0[sg.n] * gy), dim3(64 * NWV), 0, g4_stream(),
                       sg, q8, nb, m);
}

// ---- Q4_K / Q5_K through fp16 weight images (mm_batch_img_kernel) --------
// The in-register weight decode of a quantized-tensor kernel (nibbles, Q5_K
// high bits, the scales) is most of its vector instructions and sets its
// pace.  An image does that decode once per matrix, when the model
// is loaded: every weight's sc * q (the 6-bit sub-block scale times the
// 4/5-bit code, an integer <= 63 * 31, exact in fp16) stored as the B operand
// of v_mfma_f32_32x32x16_f16, plus per row and block d, dmin and the mins.
// The block sums are the same integers, chained in exact pieces (kChainSteps:
// Q4_K two chains of 128 products, Q5_K four of 64, each below 2^24 whatever
// order the matrix core adds in), and the fold the same three fp32 steps, so
// the outputs are mm_batch_kq8_kernel's bits; the
// kernel's loop is MFMAs, LDS reads of the activations and the block fold.
// The image does not record its type: the caller names it (Q5_K needs the
// shorter chains).
// K positions inside a block follow the device Q8_K byte order: position
// p = 32l + 16h + 4j + c is element 64j + 32h + 4l + c (sub-block 2j + h),
// so a token's Q8_K bytes are its A operand in place.
//   codes : [rg][nb][16 steps][64 lanes] x 16 B, rg = ceil(d / 32): lane
//           L = i + 32 kg of step s holds row 32 g + i, K positions
//           16 s + 8 kg .. +7 (8 fp16)
//   hdr   : [rg][nb][64 lanes] x 16 B: fp32 d, fp32 dmin, fp16 pairs
//           {m_2kg, m_2kg+1} and {m_4+2kg, m_5+2kg} (the min operands of
//           lane half kg)
// Rows past d are zero.
constexpr int kImgStep = 1024, kImgBlk = 16 * kImgStep, kImgHdr = 1024;

size_t kq_img_bytes(int d, int nb) { return (size_t)((d + 31) / 32) * nb * (kImgBlk + kImgHdr); }

__device__ __forceinline__ uint32_t h16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

// one thread per (row group, block, lane) of the image
template <bool Q5>
__global__ __launch_bounds__(256) void kq_image_kernel(const uint8_t* __restrict__ w, uint8_t* __restrict__ img, int d,
                                                       int nb, int rg) {
    const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (size_t)rg * nb * 64) return;
    const int L = (int)(id & 63), i = L & 31, kg = L >> 5;
    const size_t gb = id >> 6;   // g * nb + b
    const int b = (int)(gb % nb), g = (int)(gb / nb);
    const int row = 32 * g + i;
    uint4* codes = reinterpret_cast<uint4*>(img + gb * kImgBlk + 16 * L);
    uint4* hdo = reinterpret_cast<uint4*>(img + (size_t)rg * nb * kImgBlk + gb * kImgHdr + 16 * L);
    if (row >= d) {
        for (int s = 0; s < 16; s++) codes[s * (kImgStep / 16)] = make_uint4(0, 0, 0, 0);
        *hdo = make_uint4(0, 0, 0, 0);
        return;
    }
    const size_t nblk = (size_t)d * nb, blk = (size_t)row * nb + b;
    const uint4 hdr = *reinterpret_cast<const uint4*>(w + (Q5 ? 160 : 128) * nblk + blk * 16);
    uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
    unpack_scales(hdr.y, hdr.z, hdr.w, sc_lo, sc_hi, mn_lo, mn_hi);
    const uint8_t* qs = w + blk * 128;        // device word 4l + j = GGUF qs word 8j + l
    const uint8_t* qh = w + 128 * nblk + blk * 32;
    for (int s = 0; s < 16; s++) {
        uint32_t hv[4];
        for (int t2 = 0; t2 < 4; t2++) {
            uint32_t pair = 0;
            for (int u = 0; u < 2; u++) {
                const int p = 16 * s + 8 * kg + 2 * t2 + u;
                const int l = p >> 5, h = (p >> 4) & 1, j = (p >> 2) & 3, c = p & 3, sb = 2 * j + h;
                const int byte = qs[16 * l + 4 * j + c];
                int q = h ? byte >> 4 : byte & 15;
                if (Q5) q |= ((qh[4 * l + c] >> sb) & 1) << 4;
                pair |= h16_bits((float)(byte_of(sb < 4 ? sc_lo : sc_hi, sb & 3) * q)) << (16 * u);
            }
            hv[t2] = pair;
        }
        codes[s * (kImgStep / 16)] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
    }
    const uint32_t ma = h16_bits((float)byte_of(mn_lo, 2 * kg)), mb = h16_bits((float)byte_of(mn_lo, 2 * kg + 1));
    const uint32_t mc = h16_bits((float)byte_of(mn_hi, 2 * kg)), md = h16_bits((float)byte_of(mn_hi, 2 * kg + 1));
    *hdo = make_uint4(__float_as_uint(f16_to_f32(hdr.x & 0xffffu)), __float_as_uint(f16_to_f32(hdr.x >> 16)),
                      ma | (mb << 16), mc | (md << 16));
}

// NWV waves of 32 rows (one image row group each) x 32 NT tokens per
// workgroup; segments as in mm_batch_kq8_kernel, in units of 32 NWV rows
// LDS slot (16 bytes) of step s, lane half kg inside a token's row: the two
// halves of a step 128 bytes apart, so that the lanes (i, 0) and (i, 1) of
// one 128-bit read fall in different banks (2 s + kg, the plain order, had
// three times the bank-conflict cycles and took 8 % longer)
__device__ __forceinline__ int img_slot(int s, int kg) { return (s & 7) + 8 * kg + 16 * (s >> 3); }

// MODE 0: the outputs; MODE 2: every block's int32 S_b and M_b, as
// mm_batch_kq8_kernel's MODE 2
template <bool Q5, int NT, int NWV, int MODE = 0>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2))) void mm_batch_img_kernel(
    const KqSegs sg, const uint8_t* __restrict__ q8, int nb, int m) {
    constexpr bool DB = MODE == 2;
    constexpr int CS = kChainSteps<Q5>;
    constexpr int NTH = 64 * NWV;
    constexpr int TOK = 32 * NT;
    constexpr int UPT = (TOK * 8 + NTH - 1) / NTH;   // (token, 32-byte unit) pairs per thread
    constexpr int BQ = (TOK * 4 + NTH - 1) / NTH;    // 8-byte bsums quarters per thread
    __shared__ __align__(16) uint8_t sA[2][TOK * kKqTok];
    __shared__ __align__(16) uint8_t sS[2][TOK * kKqBs];
    __shared__ __align__(16) float sD[2][TOK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 31, kg = lane >> 5;
    int bx, by;
    xcd_tile((m + TOK - 1) / TOK, bx, by);
    int seg = 0;
#pragma unroll
    for (int k = 1; k < kMaxSegs; k++)
        if (k < sg.n && bx >= sg.g0[k]) seg = k;
    const uint8_t* __restrict__ img = sg.w[seg];
    const int d = sg.d[seg];
    float* __restrict__ out = sg.o[seg];
    const int rg = (d + 31) / 32;
    const int gw = (bx - sg.g0[seg]) * NWV + wave;   // this wave's row group
    const int g = min(gw, rg - 1);
    const int row = 32 * gw + i;
    const int tokb = by * TOK;
    const size_t q8row = ((size_t)nb * 292 + 63) & ~(size_t)63;   // q8_row_stride

    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)img, (short)0, (int)((size_t)rg * nb * (kImgBlk + kImgHdr)), kBufWord3);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)q8, (short)0, (int)(m * q8row), kBufWord3);
    const int vw = g * nb * kImgBlk + 16 * lane;
    const int vh = rg * nb * kImgBlk + g * nb * kImgHdr + 16 * lane;
    int vx[UPT], vbs[BQ];
#pragma unroll
    for (int j = 0; j < UPT; j++) {
        const int u = min(tid + j * NTH, TOK * 8 - 1);
        vx[j] = min(tokb + (u >> 3), m - 1) * (int)q8row + 32 * (u & 7);
    }
#pragma unroll
    for (int j = 0; j < BQ; j++) {
        const int u = min(tid + j * NTH, TOK * 4 - 1);
        vbs[j] = min(tokb + (u >> 2), m - 1) * (int)q8row + (int)q8k_bsums_off(nb) + 8 * (u & 3);
    }
    const int vyd = min(tokb + min(tid, TOK - 1), m - 1) * (int)q8row + (int)q8k_d_off(nb);

    struct XRaw {
        uint4 a0[UPT], a1[UPT];
        uint2 bs[BQ];
        float yd;
    };
    auto load_x = [&](int b, XRaw& r) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            r.a0[j] = buf_load16(rq, vx[j], b * 256);
            r.a1[j] = buf_load16(rq, vx[j] + 16, b * 256);
        }
#pragma unroll
        for (int j = 0; j < BQ; j++) r.bs[j] = buf_load8(rq, vbs[j], b * 32);
        r.yd = __uint_as_float(buf_load4(rq, vyd, b * 4));
    };
    // unit (t, l'): Q8_K device bytes 32l' .. 32l'+31 of the block -> fp16 at
    // K positions 32l' .. 32l'+31 of token row t
    auto stage = [&](const XRaw& r, int st) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * NTH;
            if (UPT * NTH != TOK * 8 && u >= TOK * 8) continue;
            uint8_t* dst = sA[st] + (u >> 3) * kKqTok;
            const int s0 = 2 * (u & 7);   // steps s0, s0 + 1
            const uint2 c0 = i8x4_to_h4(r.a0[j].x), c1 = i8x4_to_h4(r.a0[j].y);
            const uint2 c2 = i8x4_to_h4(r.a0[j].z), c3 = i8x4_to_h4(r.a0[j].w);
            const uint2 c4 = i8x4_to_h4(r.a1[j].x), c5 = i8x4_to_h4(r.a1[j].y);
            const uint2 c6 = i8x4_to_h4(r.a1[j].z), c7 = i8x4_to_h4(r.a1[j].w);
            *reinterpret_cast<uint4*>(dst + 16 * img_slot(s0, 0)) = make_uint4(c0.x, c0.y, c1.x, c1.y);
            *reinterpret_cast<uint4*>(dst + 16 * img_slot(s0, 1)) = make_uint4(c2.x, c2.y, c3.x, c3.y);
            *reinterpret_cast<uint4*>(dst + 16 * img_slot(s0 + 1, 0)) = make_uint4(c4.x, c4.y, c5.x, c5.y);
            *reinterpret_cast<uint4*>(dst + 16 * img_slot(s0 + 1, 1)) = make_uint4(c6.x, c6.y, c7.x, c7.y);
        }
#pragma unroll
        for (int j = 0; j < BQ; j++) {
            const int u = tid + j * NTH;
            if (u < TOK * 4) {
                const h2_t lo = {(_Float16)(int16_t)(r.bs[j].x & 0xffffu), (_Float16)(int16_t)(r.bs[j].x >> 16)};
                const h2_t hi = {(_Float16)(int16_t)(r.bs[j].y & 0xffffu), (_Float16)(int16_t)(r.bs[j].y >> 16)};
                *reinterpret_cast<uint2*>(sS[st] + (u >> 2) * kKqBs + 8 * (u & 3)) = make_uint2(h2_bits(lo), h2_bits(hi));
            }
        }
        if (tid < TOK) sD[st][tid] = r.yd;
    };

    f16v_t acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[nt][v] = 0.0f;
    f16v_t zero;
#pragma unroll
    for (int v = 0; v < 16; v++) zero[v] = 0.0f;

    // the weights of block b + 1 are loaded step by step as block b's
    // products consume block b's (W[s] is reloaded right after its MFMAs);
    // loads past the last block repeat it (no branch: the compiler's waits
    // stay exact)
    uint4 W[16], H;
#pragma unroll
    for (int s = 0; s < 16; s++) W[s] = buf_load16(rw, vw, s * kImgStep);
    H = buf_load16(rw, vh, 0);
    XRaw xn;
    load_x(0, xn);
    stage(xn, 0);
    load_x(min(1, nb - 1), xn);
    auto block = [&](int b, int st) {
        lds_barrier();
        const uint4 Hc = H;
        const int bn = min(b + 1, nb - 1);
        H = buf_load16(rw, vh, bn * kImgHdr);
        f16v_t S[NT], P[NT];
        int SI[NT][16];
        const uint8_t* at0 = sA[st] + i * kKqTok;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            if (s == 8 && b + 1 < nb) {
                stage(xn, st ^ 1);
                load_x(min(b + 2, nb - 1), xn);
            }
            const h8_t B = __builtin_bit_cast(h8_t, W[s]);
            const int so = 16 * img_slot(s, kg);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const h8_t A = *reinterpret_cast<const h8_t*>(at0 + 32 * nt * kKqTok + so);
                S[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, B, s % CS == 0 ? zero : S[nt], 0, 0, 0);
                chain_end<Q5>(s, S[nt], P[nt], SI[nt]);
            }
            W[s] = buf_load16(rw, vw, bn * kImgBlk + s * kImgStep);
        }
        const uint32_t ml = (Hc.z & 0xffffu) | (Hc.z << 16), mh = (Hc.z >> 16) | (Hc.z & 0xffff0000u);
        const uint32_t nl = (Hc.w & 0xffffu) | (Hc.w << 16), nh = (Hc.w >> 16) | (Hc.w & 0xffff0000u);
        const h4_t Bm1 = __builtin_bit_cast(h4_t, make_uint2(ml, mh)), Bm2 = __builtin_bit_cast(h4_t, make_uint2(nl, nh));
        const float dx = __uint_as_float(Hc.x), dmx = __uint_as_float(Hc.y);
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint8_t* bs = sS[st] + (32 * nt + i) * kKqBs + 8 * kg;
            const h4_t A1 = *reinterpret_cast<const h4_t*>(bs), A2 = *reinterpret_cast<const h4_t*>(bs + 16);
            f16v_t M = __builtin_amdgcn_mfma_f32_32x32x8f16(A1, Bm1, zero, 0, 0, 0);
            M = __builtin_amdgcn_mfma_f32_32x32x8f16(A2, Bm2, M, 0, 0, 0);
            if (DB) {
                store_block_sums<Q5>(reinterpret_cast<int32_t*>(sg.o[0]), reinterpret_cast<int32_t*>(sg.o[1]), S[nt],
                                     P[nt], SI[nt], M, gw < rg ? row : d, d, tokb + 32 * nt + 4 * kg, m, nb, b);
                continue;
            }
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const float4 yd = *reinterpret_cast<const float4*>(sD[st] + 32 * nt + 8 * a + 4 * kg);
                const float y4[4] = {yd.x, yd.y, yd.z, yd.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int v = 4 * a + c;
                    acc[nt][v] = __builtin_fmaf(
                        y4[c], __builtin_fmaf(dx, chain_block_sum<Q5>(S[nt], P[nt], SI[nt], v), -(dmx * M[v])), acc[nt][v]);
                }
            }
        }
    };
    for (int b = 0; b < nb; b += 2) {
        block(b, 0);
        if (b + 1 < nb) block(b + 1, 1);
    }

    if (!DB && gw < rg && row < d) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int tok = tokb + 32 * nt + 8 * (v >> 2) + 4 * kg + (v & 3);
                if (tok < m) out[(size_t)tok * d + row] = acc[nt][v];
            }
    }
}

template <bool Q5, int NT, int NWV, int MODE = 0>
void launch_mm_batch_img(const KqSegs& sg, const uint8_t* q8, int nb, int m) {
    const int gy = (m + 32 * NT - 1) / (32 * NT);
    hipLaunchKernelGGL((mm_batch_img_kernel<Q5, NT, NWV, MODE>), dim3(sg.g0[sg.n] * gy), dim3(64 * NWV), 0, g4_stream(),
                       sg, q8, nb, m);
}

// The fold of g4_mm_batch_q8_blocks' per-block terms, in block order as the
// GEMM kernel folds them (g = fma(d_tb, u_b, g) from 0), optionally followed
// by gelu(g) * ple (main.c:1989-1993, as gelu_mul_rows_kernel) and the Q8_K
// rows of the result (as quantize_rows_q8k_kernel): one workgroup per token
constexpr int kFoldMaxD = 1024, kFoldMaxBlocks = 64;
__global__ __launch_bounds__(256) void fold_gelu_mul_q8_kernel(const float* __restrict__ u, const uint8_t* __restrict__ q8,
                                                               int nb, const float* __restrict__ ple, int pstride,
                                                               float* __restrict__ out, uint8_t* __restrict__ q8o, int d,
                                                               int m) {
    __shared__ float yd[kFoldMaxBlocks];
    __shared__ __align__(16) float row[kFoldMaxD];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t qrow = ((size_t)nb * 292 + 63) & ~(size_t)63;   // q8_row_stride(nb)
    const float* qd = reinterpret_cast<const float*>(q8 + (size_t)t * qrow + q8k_d_off(nb));
    for (int b = tid; b < nb; b += 256) yd[b] = qd[b];
    __syncthreads();
    for (int r = tid; r < d; r += 256) {
        float g = 0.0f;
        for (int b = 0; b < nb; b++) g = __builtin_fmaf(yd[b], u[((size_t)b * m + t) * d + r], g);
        const float v = ple ? gelu_ref(g) * ple[(size_t)t * pstride + r] : g;
        out[(size_t)t * d + r] = v;
        row[r] = v;
    }
    if (q8o) {
        __syncthreads();
        const int db = d / 256;
        const size_t orow = ((size_t)db * 292 + 63) & ~(size_t)63;   // q8_row_stride(db)
        for (int blk = wave; blk < db; blk += 4) {
            const float4 f = reinterpret_cast<const float4*>(row + blk * 256)[lane];
            const float v4[4] = {f.x, f.y, f.z, f.w};
            quantize_block_wave(v4, lane, q8o + (size_t)t * orow, db, blk);
        }
    }
}


// the shipped tiling: 128 rows x 32 tokens per workgroup (a sweep over 32 and
// 64 tokens, one or two accumulator chains and preloaded A operands at the
// E4B shapes over 511 tokens: 10240x2560 60 us, 2048x2560 18 us, 2560x2048
// 22 us; the 64-token tile needs 211 VGPRs, two waves per SIMD)
constexpr int kKqNT = 1;

// waves (32 rows each) per workgroup: five when four would need more than
// one workgroup per CU and five fit in one (a 2560-row matrix at 511 tokens:
// 320 against 256 workgroups; 2560x2560 23.9 against 26.3 us, O 2560x2048
// 19.1 against 20.8), else four (gate 10240x2560 63.4 against 87.6 us with
// five, 256x2560 16.3 against 21.0; 2048 rows, one round either way, 18.5
// against 23.4; Q|K as two segments of 2048 and 512 rows needs 17 five-wave
// row groups, and six waves measured the same as four, 25.4 us)
int kq_waves(const int* d, int nseg, int m) {
    const long long gy = (m + 32 * kKqNT - 1) / (32 * kKqNT), cus = g4_num_cus();
    auto grid = [&](int nwv) {
        long long g = 0;
        for (int k = 0; k < nseg; k++) g += (d[k] + 32 * nwv - 1) / (32 * nwv) * gy;
        return g;
    };
    return grid(4) > cus && grid(5) <= cus ? 5 : 4;
}

// ---- fp32 activations: Q6_K and bf16 matrices --------------------------
// Y[m x d] = X[m x n] . W[d x n]^T where the reference multiplies fp32
// activations by the dequantized weights (mm_quant_rows for Q6_K,
// gemma4-4b/cpu-blas/main.c:1539-1556 with dequant_q6_k main.c:213-236;
// mm_bf16 main.c:1529-1537).  Each weight is dequantized to the reference's fp32 value
// (Q6_K: (d * sc) * (q - 32) in that order; bf16: the high half of the
// fp32) and multiplied by the fp32 activation on the matrix cores
// (v_mfma_f32_16x16x4_f32: fp32 products, fp32 sums); only the order of
// the sums differs from the per-token dot.
//
// Operands: the 16 tokens of a tile are the A rows, 16 weight rows the B
// columns, so a lane's results are one weight row of four tokens and a
// store writes 16 consecutive rows of a token.  Lane group g (lanes
// 16g..16g+15) supplies K index g of every 16x16x4 step; over one 256-long
// block it walks 64 elements of its row:
//   Q6_K: g = 2h + s -> elements 128h + 32k + 16s + t (k < 4, t < 16), i.e.
//         the 32 ql bytes at 32g, the 16 qh bytes at 16g and the scales
//         8h + s + 2k of the planar block (layout.hip);
//   bf16: elements 64g .. 64g+63.
// The activations of the workgroup's tokens are staged per block in LDS in
// natural order (260 floats per token: conflict-free 16-byte reads).
constexpr int kF32XS = 260;

template <bool BF, int RW, int NT>
__global__ __launch_bounds__(64 * RW) void mm_batch_f32_kernel(const uint8_t* __restrict__ w,
                                                               const float* __restrict__ x, float* __restrict__ out,
                                                               int n, int d, int m) {
    constexpr int NTHR = 64 * RW;
    constexpr int TOK = 16 * NT;
    constexpr int XV = TOK * 64 / NTHR;             // float4 of activations per thread and block
    static_assert(XV * NTHR == TOK * 64, "token tile must divide among the threads");
    __shared__ __align__(16) float sx[TOK * kF32XS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, g = lane >> 4;
    const int row0 = blockIdx.x * (16 * RW) + wave * 16;
    const int tok0 = blockIdx.y * TOK;
    const int nb = n >> 8;
    const size_t rj = (size_t)min(row0 + i, d - 1);  // this lane's weight row
    const Q6KPlanes P = q6k_planes((size_t)d * nb);
    const int h = g >> 1, s = g & 1;

    struct WRaw {
        uint4 v[BF ? 8 : 3];     // bf16: 64 values; Q6_K: ql (2) and qh (1)
        uint2 sc;
        uint32_t dh;
    };
    auto load_w = [&](int b, WRaw& r) {
        if (BF) {
            const uint4* p = reinterpret_cast<const uint4*>(w + (rj * n + (size_t)b * 256 + 64 * g) * 2);
#pragma unroll
            for (int k = 0; k < 8; k++) r.v[k] = p[k];
        } else {
            const size_t blk = rj * nb + b;
            const uint4* ql = reinterpret_cast<const uint4*>(w + P.ql + blk * 128 + 32 * g);
            r.v[0] = ql[0];
            r.v[1] = ql[1];
            r.v[2] = *reinterpret_cast<const uint4*>(w + P.qh + blk * 64 + 16 * g);
            r.sc = *reinterpret_cast<const uint2*>(w + P.sc + blk * 16 + 8 * h);
            r.dh = *reinterpret_cast<const uint16_t*>(w + P.d + blk * 2);
        }
    };
    struct XRaw {
        f4_t v[XV];
    };
    // unit u = tid + j * NTHR: token u >> 6, float4 u & 63 of the block
    auto load_x = [&](int b, XRaw& r) {
#pragma unroll
        for (int j = 0; j < XV; j++) {
            const int u = tid + j * NTHR;
            const int t = min(tok0 + (u >> 6), m - 1);
            r.v[j] = reinterpret_cast<const f4_t*>(x + (size_t)t * n + (size_t)b * 256)[u & 63];
        }
    };
    auto stage = [&](const XRaw& r) {
#pragma unroll
        for (int j = 0; j < XV; j++) {
            const int u = tid + j * NTHR;
            *reinterpret_cast<f4_t*>(sx + (u >> 6) * kF32XS + 4 * (u & 63)) = r.v[j];
        }
    };

    f4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = f4_t{0.f, 0.f, 0.f, 0.f};

    WRaw wn;
    XRaw xn;
    load_w(0, wn);
    load_x(0, xn);
    for (int b = 0; b < nb; b++) {
        lds_barrier();   // the previous block's LDS reads are done
        stage(xn);
        const WRaw wc = wn;
        // the next block (the last one again at the end: an unconditional
        // load keeps the prefetch registers out of scratch memory)
        const int bn = min(b + 1, nb - 1);
        load_w(bn, wn);
        load_x(bn, xn);
        lds_barrier();

        const float* xa = sx + i * kF32XS;
        if (BF) {
#pragma unroll
            for (int t4 = 0; t4 < 16; t4++) {
                const uint32_t lo = t4 & 1 ? wc.v[t4 >> 1].z : wc.v[t4 >> 1].x;
                const uint32_t hi = t4 & 1 ? wc.v[t4 >> 1].w : wc.v[t4 >> 1].y;
                const float wv[4] = {__uint_as_float(lo << 16), __uint_as_float(lo & 0xffff0000u),
                                     __uint_as_float(hi << 16), __uint_as_float(hi & 0xffff0000u)};
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const float4 a = *reinterpret_cast<const float4*>(xa + 16 * t * kF32XS + 64 * g + 4 * t4);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, wv[0], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, wv[1], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, wv[2], acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, wv[3], acc[t], 0, 0, 0);
                }
            }
        } else {
            const float df = hbits_to_f32(wc.dh);
            const uint32_t qlw[8] = {wc.v[0].x, wc.v[0].y, wc.v[0].z, wc.v[0].w,
                                     wc.v[1].x, wc.v[1].y, wc.v[1].z, wc.v[1].w};
            const uint32_t qhw[4] = {wc.v[2].x, wc.v[2].y, wc.v[2].z, wc.v[2].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                // scale of sub-block 8h + s + 2k (bytes s + 2k of this half's 8)
                const int sb = s + 2 * k;
                const float dsc = df * (float)(int8_t)byte_of(sb < 4 ? wc.sc.x : wc.sc.y, sb & 3);
#pragma unroll
                for (int t4 = 0; t4 < 4; t4++) {
                    // elements t = 4t4..4t4+3: ql bytes 16(t>>3) + 8(k&1) + (t&7),
                    // nibble k>>1; qh bytes t, bits 2k..2k+1
                    const uint32_t ql = qlw[4 * (t4 >> 1) + 2 * (k & 1) + (t4 & 1)];
                    const uint32_t q = ((ql >> (4 * (k >> 1))) & 0x0f0f0f0fu) |
                                       (((qhw[t4] >> (2 * k)) & 0x03030303u) << 4);
                    const uint32_t qx = q ^ 0x20202020u;   // 6-bit two's complement of q - 32
                    float wv[4];
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        wv[c] = dsc * (float)(int)__builtin_amdgcn_sbfe(qx, 8 * c, 6);   // the builtin's type is unsigned
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        const float4 a = *reinterpret_cast<const float4*>(xa + 16 * t * kF32XS + 128 * h + 16 * s +
                                                                          32 * k + 4 * t4);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, wv[0], acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, wv[1], acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, wv[2], acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, wv[3], acc[t], 0, 0, 0);
                    }
                }
            }
        }
    }
    // lane (g, i) holds tokens 4g + v of each tile, weight row row0 + i
    const int row = row0 + i;
    if (row < d) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int tok = tok0 + 16 * t + 4 * g + v;
                if (tok < m) out[(size_t)tok * d + row] = acc[t][v];
            }
    }
}

// tilings from a sweep over 2-8 row waves x 1-4 token tiles at the E4B
// shapes and 511 tokens (all bit-identical): Q6_K 64 rows x 16 tokens per
// workgroup (FFN down 310 us against 334 us at 64 x 32; V 26 against 38 us);
// bf16 64 rows x 32 tokens (PLE projection 302 us against 325 us)
constexpr int kF32RW = 4;

template <bool BF>
void launch_mm_batch_f32(const uint8_t* w, const float* x, float* o, int n, int d, int m) {
    constexpr int NT = BF ? 2 : 1;
    const dim3 grid((d + 16 * kF32RW - 1) / (16 * kF32RW), (m + 16 * NT - 1) / (16 * NT));
    hipLaunchKernelGGL((mm_batch_f32_kernel<BF, kF32RW, NT>), grid, dim3(64 * kF32RW), 0, g4_stream(), w, x, o, n, d,
                       m);
}

// ---- Q6_K on fp16 matrix cores: split activations ------------------------
// Row layout of the split activations: n/256 blocks of 1024 bytes, the 256 hi
// terms of the block then its 256 lo terms, each in K-step order: step c
// (0..7), lane group g (0..3), 8 elements, where (c, g, t) is element
//   128h + 32k + 16s + 8 half + t   (g = 2h + s, c = 2k + half)
// of the block, i.e. lane group g's elements of the planar Q6_K block
// (layout.hip) in the order its ql/qh bytes hold them.  After the m rows come
// m floats: 2^s of each row, the factor that undoes the row's scaling.
constexpr int kSplitBlk = 1024;      // bytes per 256-element block of a split row

__device__ __forceinline__ int split_pos(int e) {
    const int h = e >> 7, k = (e >> 5) & 3, s = (e >> 4) & 1, half = (e >> 3) & 1;
    return ((((2 * k + half) << 2) | (2 * h + s)) << 3) | (e & 7);
}

// one workgroup per row: max |x|, then x * 2^-s -> hi + lo (fp16, round to
// nearest even; x * 2^-s - hi is exact in fp32)
__global__ __launch_bounds__(256) void split_rows_f16_kernel(const float* __restrict__ x, uint8_t* __restrict__ xs,
                                                             int n, int m) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float4* xr = reinterpret_cast<const float4*>(x + (size_t)t * n);
    float mx = 0.0f;
    for (int u = tid; u < n / 4; u += 256) {
        const float4 f = xr[u];
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // mx = f * 2^E, f in [0.5, 1): scaled max in [2^14, 2^15)
    int E = 0;
    (void)frexpf(mx, &E);
    const int k = mx > 0.0f && mx <= 3.402823466e38f ? min(max(15 - E, -126), 126) : 0;
    const float sf = ldexpf(1.0f, k);
    uint8_t* row = xs + (size_t)t * n * 4;
    for (int u = tid; u < n / 8; u += 256) {
        const float4 f0 = xr[2 * u], f1 = xr[2 * u + 1];
        const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        h8_t hi, lo;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float sv = v[j] * sf;
            const _Float16 hv = (_Float16)sv;
            hi[j] = hv;
            lo[j] = (_Float16)(sv - (float)hv);
        }
        const int e = 8 * u;
        uint8_t* dst = row + (size_t)(e >> 8) * kSplitBlk + 2 * split_pos(e & 255);
        *reinterpret_cast<h8_t*>(dst) = hi;
        *reinterpret_cast<h8_t*>(dst + 512) = lo;
    }
    if (tid == 0) reinterpret_cast<float*>(xs + (size_t)m * n * 4)[t] = ldexpf(1.0f, -k);
}

// gelu(g) * u of one row (the FFN's GELU gate, main.c:1976-1980) split as
// split_rows_f16_kernel splits a row: one workgroup per row; each thread
// keeps the values of its runs of 8 in registers between the max and the
// split, so the product never goes to memory.  NG: runs of 8 per thread
// (n = 2048 * NG).
template <int NG>
__global__ __launch_bounds__(256) void gelu_mul_split_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                             int ustride, uint8_t* __restrict__ xs, int n, int m) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float4* gr = reinterpret_cast<const float4*>(g + (size_t)t * n);
    const float4* ur = reinterpret_cast<const float4*>(u + (size_t)t * ustride);
    float v[NG][8];
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < NG; k++) {
        const int q = tid + 256 * k;
        const float4 g0 = gr[2 * q], g1 = gr[2 * q + 1], u0 = ur[2 * q], u1 = ur[2 * q + 1];
        const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            v[k][j] = gelu_ref(gg[j]) * uu[j];
            mx = fmaxf(mx, fabsf(v[k][j]));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int E = 0;
    (void)frexpf(mx, &E);
    const int k2 = mx > 0.0f && mx <= 3.402823466e38f ? min(max(15 - E, -126), 126) : 0;
    const float sf = ldexpf(1.0f, k2);
    uint8_t* row = xs + (size_t)t * n * 4;
#pragma unroll
    for (int k = 0; k < NG; k++) {
        h8_t hi, lo;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float sv = v[k][j] * sf;
            const _Float16 hv = (_Float16)sv;
            hi[j] = hv;
            lo[j] = (_Float16)(sv - (float)hv);
        }
        const int e = 8 * (tid + 256 * k);
        uint8_t* dst = row + (size_t)(e >> 8) * kSplitBlk + 2 * split_pos(e & 255);
        *reinterpret_cast<h8_t*>(dst) = hi;
        *reinterpret_cast<h8_t*>(dst + 512) = lo;
    }
    if (tid == 0) reinterpret_cast<float*>(xs + (size_t)m * n * 4)[t] = ldexpf(1.0f, -k2);
}

// Y[m x d] = X . W^T for planar Q6_K W over split activations.  A operand
// (tokens): lane (g, i) holds the hi (or lo) terms (c, g, 0..7) of token
// 16 nt + i; B operand (weights): Wh or Wl of the same elements of row
// 16 rt + i.  Result lane (g, i): tokens 16 nt + 4g + v of
// row 16 rt + i.
constexpr int kXsStride = kSplitBlk + 32;   // LDS bytes per staged token

// 16 bytes per lane from a buffer straight into LDS at lds + 16 * lane (the
// LDS address is wave-uniform: it goes to M0).  A plain device function: in
// a kernel template's own body the builtin keeps the host pass from
// emitting the kernel's launch stub.
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voff, soff, 0, 0);
}

// SP (two stages only): the next block's copies are issued one per product
// step of this block instead of all at its start, and one barrier per block
// suffices
template <int RT, int NT, int NS, int NWV, bool SP = false>
__global__ __launch_bounds__(64 * NWV) void mm_batch_q6s_kernel(
    const uint8_t* __restrict__ w, const uint8_t* __restrict__ xs, float* __restrict__ out, int n, int d, int m) {
    constexpr int TOK = 16 * NT;
    // direct-to-LDS copies per block (one token each): wave w takes tokens
    // w, w + NWV, ... (DPW or DPW + 1 of them)
    constexpr int DPW = TOK / NWV, DPX = (TOK + NWV - 1) / NWV;
    static_assert(DPW >= 1, "every wave copies a token");
    static_assert(!SP || (NS == 2 && DPX <= 8), "spread copies: two stages, at most one copy per product step");
    // NS stages: blocks b + 1 .. b + NS - 1 are on their way while block b is
    // read (the loads take longer than a block's products)
    __shared__ __align__(16) uint8_t sx[NS][TOK * kXsStride];

    // (the wave index read as uniform: the copies' scalar offsets below then
    // need no per-lane loop)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4, h = g >> 1, s = g & 1;
    int bx, by;
    xcd_tile((m + TOK - 1) / TOK, bx, by);
    const int rbase = bx * (16 * RT * NWV) + wave * (16 * RT);
    const int tokb = by * TOK;
    const int nb = n >> 8;
    const size_t nblk = (size_t)d * nb;
    const Q6KPlanes P = q6k_planes(nblk);
    const size_t xrow = (size_t)n * 4;

    // weights through buffer loads: per-lane offsets fixed, the block's
    // offset in a scalar register
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)(P.d + 2 * nblk), kBufWord3);
    int vql[RT], vqh[RT], vsc[RT], vd[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int rB = min(rbase + 16 * rt + i, d - 1) * nb;
        vql[rt] = (int)P.ql + rB * 128 + 32 * g;
        vqh[rt] = (int)P.qh + rB * 64 + 16 * g;
        vsc[rt] = (int)P.sc + rB * 16 + 8 * h;
        vd[rt] = (int)P.d + rB * 2;
    }
    struct WRaw {
        uint4 ql[RT][2];   // lane group g's 32 ql bytes
        uint4 qh[RT];      // its 16 qh bytes
        uint2 sc[RT];      // scales of sub-blocks 8h .. 8h+7
        uint32_t dh[RT];
    };
    auto load_w = [&](int b, WRaw& r) {
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            r.ql[rt][0] = buf_load16(rw, vql[rt], b * 128);
            r.ql[rt][1] = buf_load16(rw, vql[rt] + 16, b * 128);
            r.qh[rt] = buf_load16(rw, vqh[rt], b * 64);
            r.sc[rt] = buf_load8(rw, vsc[rt], b * 16);
            r.dh[rt] = __builtin_amdgcn_raw_buffer_load_b16(rw, vd[rt], b * 2, 0);
        }
    };
    // block b's activations of token tokb + wave + NWV q -> stage row wave + NWV q:
    // one 1 KB copy per wave instruction, 16 bytes per lane (tokens past m
    // repeat the last one; their outputs are not stored)
    // (buffer-to-LDS loads: one lane offset register, the token's row and the
    // block in a scalar offset)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)xs, (short)0, (int)(m * xrow), kBufWord3);
    int xrows[DPX];
#pragma unroll
    for (int q = 0; q < DPX; q++) xrows[q] = min(tokb + wave + NWV * q, m - 1) * (int)xrow;
    auto dma = [&](int b, uint8_t* stage) {
#pragma unroll
        for (int q = 0; q < DPX; q++)
            if (DPX == DPW || wave + NWV * q < TOK)
                buf_load_lds16(rx, stage + (wave + NWV * q) * kXsStride, 16 * lane, xrows[q] + b * kSplitBlk);
    };

    f4_t acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[rt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    const f4_t zero = {0.f, 0.f, 0.f, 0.f};
    const h2_t m1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};

    // one block from stage cur and weight set wc, with block b + NS - 1's
    // weights and activations sent into wn and nxt
    auto block = [&](int b, const uint8_t* cur, uint8_t* nxt, const WRaw& wc, WRaw& wn) {
        const int bn = min(b + NS - 1, nb - 1);
        if (SP) {
            // this wave's copies of block b (issued during block b - 1) and
            // everything before them have landed; after the barrier every
            // wave's have, and every wave is done reading nxt (block b - 1)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            lds_barrier();
            load_w(bn, wn);
        } else {
            lds_barrier();   // block b - 1's reads of nxt are done
            // block b + NS - 1's copies (the last block again after the end:
            // no branch), then a wait that leaves at most the copies of
            // blocks b + 1 .. b + NS - 1 in flight: everything issued before
            // them has landed, block b's copies included.  Counting only the
            // copies keeps the wait correct wherever the compiler places the
            // weight loads (it has moved them past the compute of the block
            // before): weight loads among the most recent operations only
            // make it wait for more
            dma(bn, nxt);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(DPW * (NS - 1)));   // (DPW: the fewest copies a wave issues)
            load_w(bn, wn);
            lds_barrier();   // every wave's copies of block b are in cur
        }

        f4_t S[RT][NT];
        const uint8_t* xa0 = cur + i * kXsStride + 16 * g;
        // activation operands one step ahead of their products
        h8_t Ah[2][NT], Al[2][NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            Ah[0][nt] = *reinterpret_cast<const h8_t*>(xa0 + 16 * nt * kXsStride);
            Al[0][nt] = *reinterpret_cast<const h8_t*>(xa0 + 16 * nt * kXsStride + 512);
        }
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int k = c >> 1, half = c & 1, cb = c & 1;
            if (c + 1 < 8) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const uint8_t* xa = xa0 + 16 * nt * kXsStride + 64 * (c + 1);
                    Ah[cb ^ 1][nt] = *reinterpret_cast<const h8_t*>(xa);
                    Al[cb ^ 1][nt] = *reinterpret_cast<const h8_t*>(xa + 512);
                }
            }
            if (SP && c < DPX && (DPX == DPW || wave + NWV * c < TOK))   // copy c of block bn
                buf_load_lds16(rx, nxt + (wave + NWV * c) * kXsStride, 16 * lane, xrows[c < DPX ? c : 0] + bn * kSplitBlk);
            __builtin_amdgcn_sched_barrier(0);   // the reads stay ahead of this step's products
            h8_t Wa[RT], Wb[RT];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                // codes of elements (c, g, 0..7): ql bytes 16 half + 8 (k & 1) + t,
                // nibble k >> 1; qh bytes 8 half + t, bits 2k .. 2k+1
                const uint4 L = wc.ql[rt][half];
                const uint32_t l0 = (k & 1) ? L.z : L.x, l1 = (k & 1) ? L.w : L.y;
                const uint32_t h0 = half ? wc.qh[rt].z : wc.qh[rt].x, h1 = half ? wc.qh[rt].w : wc.qh[rt].y;
                const uint32_t q0 = ((l0 >> (4 * (k >> 1))) & 0x0f0f0f0fu) | (((h0 >> (2 * k)) & 0x03030303u) << 4);
                const uint32_t q1 = ((l1 >> (4 * (k >> 1))) & 0x0f0f0f0fu) | (((h1 >> (2 * k)) & 0x03030303u) << 4);
                // q - 32 exactly: fp16(1024 + q) - 1056
                const h2_t v0 = bits_h2(__builtin_amdgcn_perm(kMagic, q0, kSelLo)) + m1056;
                const h2_t v1 = bits_h2(__builtin_amdgcn_perm(kMagic, q0, kSelHi)) + m1056;
                const h2_t v2 = bits_h2(__builtin_amdgcn_perm(kMagic, q1, kSelLo)) + m1056;
                const h2_t v3 = bits_h2(__builtin_amdgcn_perm(kMagic, q1, kSelHi)) + m1056;
                // scale of sub-block 8h + 2k + s: byte 2k + s.  w = sc * (q - 32)
                // = Wh + Wl: Wh its fp16 rounding, Wl in {-1, 0, 1} (exact)
                const int sb = 2 * k + s;
                const _Float16 scf = (_Float16)(float)(int)(int8_t)byte_of(sb < 4 ? wc.sc[rt].x : wc.sc[rt].y, sb & 3);
                const h2_t SC = {scf, scf};
                const h2_t w0 = v0 * SC, w1 = v1 * SC, w2 = v2 * SC, w3 = v3 * SC;
                Wa[rt] = __builtin_bit_cast(h8_t, make_uint4(h2_bits(w0), h2_bits(w1), h2_bits(w2), h2_bits(w3)));
                Wb[rt] = __builtin_bit_cast(
                    h8_t, make_uint4(h2_bits(__builtin_elementwise_fma(v0, SC, -w0)), h2_bits(__builtin_elementwise_fma(v1, SC, -w1)),
                                     h2_bits(__builtin_elementwise_fma(v2, SC, -w2)), h2_bits(__builtin_elementwise_fma(v3, SC, -w3))));
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    // Wh xh + Wh xl + Wl xh (Wl xl is below 2^-22 of the term)
                    f4_t t = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah[cb][nt], Wa[rt], c == 0 ? zero : S[rt][nt], 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al[cb][nt], Wa[rt], t, 0, 0, 0);
                    S[rt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah[cb][nt], Wb[rt], t, 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            const float dw = hbits_to_f32(wc.dh[rt]);
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int v = 0; v < 4; v++) acc[rt][nt][v] = __builtin_fmaf(dw, S[rt][nt][v], acc[rt][nt][v]);
        }
    };

    WRaw wr[NS];
#pragma unroll
    for (int k = 0; k < NS - 1; k++) {
        load_w(min(k, nb - 1), wr[k]);
        dma(min(k, nb - 1), sx[k]);
    }
    for (int b = 0; b < nb; b += NS) {
#pragma unroll
        for (int k = 0; k < NS; k++)
            if (b + k < nb) block(b + k, sx[k], sx[(k + NS - 1) % NS], wr[k], wr[(k + NS - 1) % NS]);
    }
    // the copies of the clamped blocks past the end are still in flight:
    // they land in LDS before the workgroup ends
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

    const float* tsc = reinterpret_cast<const float*>(xs + (size_t)m * xrow);
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int tok = tokb + 16 * nt + 4 * g + v;
            if (tok >= m) continue;
            const float ts = tsc[tok];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int row = rbase + 16 * rt + i;
                if (row < d) out[(size_t)tok * d + row] = acc[rt][nt][v] * ts;
            }
        }
}

constexpr int kQ6RT = 1, kQ6NS = 2;

template <int NT, int NWV, bool SP = false>
void launch_mm_batch_q6s(const uint8_t* w, const uint8_t* xs, float* o, int n, int d, int m) {
    const int gx = (d + 16 * kQ6RT * NWV - 1) / (16 * kQ6RT * NWV), gy = (m + 16 * NT - 1) / (16 * NT);
    hipLaunchKernelGGL((mm_batch_q6s_kernel<kQ6RT, NT, kQ6NS, NWV, SP>), dim3(gx * gy), dim3(64 * NWV), 0, g4_stream(), w,
                       xs, o, n, d, m);
}

// Workgroup shapes, measured at 2560 x 10240 (FFN down) on MI355X:
//   * 160 rows (ten waves) x 32 tokens when that grid has at least 3/4 of a
//     workgroup per CU: at 511 tokens exactly one per CU, 131 against 155 us
//     for 64-row workgroups (640 of them: 1.25 rounds of two per CU); 260
//     against 281 us at 1024 tokens, equal at 200;
//   * else 64 rows x 32 tokens, or x 16 when the 32-token grid would not fill
//     one round of resident workgroups (two per CU): V (512 rows) over 511
//     tokens 14.3 against 19.2 us; FFN down at 64 tokens 45 against 92 us for
//     the ten-wave shape.
// Deeper pipelines (activations 2 or 3 blocks ahead) measured slower in
// every shape: the copies' throughput, not their latency, sets the pace;
// issuing them one per product step instead of all at a block's start helps
// the ten-wave shape (128 against 135 us) but not the 64-row one (V 15.1
// against 14.2 us).
void launch_q6s_auto(const uint8_t* w, const uint8_t* xs, float* o, int n, int d, int m) {
    const long long cus = g4_num_cus();
    const long long gy32 = (m + 31) / 32;
    if (d % 160 == 0 && (long long)(d / 160) * gy32 * 4 >= 3 * cus) return launch_mm_batch_q6s<2, 10, true>(w, xs, o, n, d, m);
    const long long wg32 = (long long)((d + 63) / 64) * gy32;
    if (wg32 < 2 * cus) launch_mm_batch_q6s<1, 4>(w, xs, o, n, d, m);
    else launch_mm_batch_q6s<2, 4>(w, xs, o, n, d, m);
}

// m rows of k floats -> m consecutive device Q8_K rows of k/256 blocks
__global__ __launch_bounds__(256) void quantize_rows_q8k_kernel(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                                int nb, int m, size_t stride) {
    const int wb = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
    if (wb >= nb * m) return;   // uniform per wave
    const int t = wb / nb, b = wb - t * nb;
    const float4 f = reinterpret_cast<const float4*>(x + (size_t)t * nb * 256 + (size_t)b * 256)[lane];
    const float v[4] = {f.x, f.y, f.z, f.w};
    quantize_block_wave(v, lane, y + (size_t)t * stride, nb, b);
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// batched Q8_K rows start on 64-byte boundaries (a row is nb * 292 bytes)
size_t q8_row_stride(int nb) { return ((size_t)nb * 292 + 63) & ~(size_t)63; }

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" size_t g4_q8K_row_stride(int k) { return k > 0 && k % 256 == 0 ? q8_row_stride(k / 256) : 0; }

extern "C" int g4_quantize_rows_q8_K(const float* x, void* y, int k, int m) {
    G4_CHECK_ARG(x && y, "g4_quantize_rows_q8_K: null pointer");
    G4_CHECK_ARG(k > 0 && k % 256 == 0, "g4_quantize_rows_q8_K: k=%d is not a positive multiple of 256", k);
    G4_CHECK_ARG(m > 0, "g4_quantize_rows_q8_K: m=%d", m);
    G4_CHECK_ARG(al16(x) && al16(y), "g4_quantize_rows_q8_K: x and y must be 16-byte aligned");
    const int nb = k / 256;
    G4_CHECK_ARG((long long)nb * m < (1LL << 31) / 64, "g4_quantize_rows_q8_K: %d x %d blocks", m, nb);
    const int waves = nb * m;
    hipLaunchKernelGGL(quantize_rows_q8k_kernel, dim3((waves + 3) / 4), dim3(256), 0, g4_stream(), x, (uint8_t*)y, nb, m,
                       q8_row_stride(nb));
    return g4_check_launch("quantize_rows_q8k_kernel");
}

extern "C" int g4_mm_batch_q8_multi(float* const* o, const void* const* w, const int* d, int nseg, const void* q8,
                                    int n, int m, int type) {
    G4_CHECK_ARG(o && w && d && q8, "g4_mm_batch_q8: null pointer");
    G4_CHECK_ARG(nseg >= 1 && nseg <= kMaxSegs, "g4_mm_batch_q8: %d matrices (1..%d)", nseg, kMaxSegs);
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && m > 0, "g4_mm_batch_q8: n=%d m=%d", n, m);
    G4_CHECK_ARG(al16(q8), "g4_mm_batch_q8: q8 must be 16-byte aligned");
    const int nb = n / 256;
    // the kernel addresses both operands with 32-bit buffer offsets
    G4_CHECK_ARG((size_t)m * q8_row_stride(nb) < (1u << 31), "g4_mm_batch_q8: %d Q8_K rows exceed 2 GiB", m);
    if (type != G4_Q4_K && type != G4_Q5_K) return g4_fail(G4_ERR_TYPE, "g4_mm_batch_q8: type %d has no Q8_K batched path", type);
    for (int k = 0; k < nseg; k++) {
        G4_CHECK_ARG(o[k] && w[k], "g4_mm_batch_q8: null pointer");
        G4_CHECK_ARG(al16(o[k]) && al16(w[k]), "g4_mm_batch_q8: o and w must be 16-byte aligned");
        G4_CHECK_ARG(d[k] > 0 && (size_t)d[k] * nb * 176 < (1u << 31), "g4_mm_batch_q8: d=%d", d[k]);
    }
    const int nwv = kq_waves(d, nseg, m), rg = 32 * nwv;   // rows per workgroup
    KqSegs sg{};
    sg.n = nseg;
    long long gx = 0;
    for (int k = 0; k < nseg; k++) {
        sg.w[k] = (const uint8_t*)w[k];
        sg.o[k] = o[k];
        sg.d[k] = d[k];
        sg.g0[k] = (int)gx;
        gx += (d[k] + rg - 1) / rg;
    }
    sg.g0[nseg] = (int)gx;
    G4_CHECK_ARG(gx * ((m + 32 * kKqNT - 1) / (32 * kKqNT)) < (1LL << 31), "g4_mm_batch_q8: %d tokens too many", m);
    if (type == G4_Q4_K) {
        if (nwv == 5) launch_mm_batch8<false, kKqNT, 5>(sg, (const uint8_t*)q8, nb, m);
        else launch_mm_batch8<false, kKqNT, 4>(sg, (const uint8_t*)q8, nb, m);
    } else {
        if (nwv == 5) launch_mm_batch8<true, kKqNT, 5>(sg, (const uint8_t*)q8, nb, m);
        else launch_mm_batch8<true, kKqNT, 4>(sg, (const uint8_t*)q8, nb, m);
    }
    return g4_check_launch("mm_batch_kq8_kernel");
}

extern "C" int g4_mm_batch_q8(float* o, const void* w, const void* q8, int n, int d, int m, int type) {
    return g4_mm_batch_q8_multi(&o, &w, &d, 1, q8, n, m, type);
}

extern "C" int g4_mm_batch_q8_blocks(float* u, const void* w, const void* q8, int n, int d, int m, int type) {
    G4_CHECK_ARG(u && w && q8, "g4_mm_batch_q8_blocks: null pointer");
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && m > 0 && d > 0, "g4_mm_batch_q8_blocks: n=%d d=%d m=%d", n, d, m);
    G4_CHECK_ARG(al16(u) && al16(w) && al16(q8), "g4_mm_batch_q8_blocks: u, w and q8 must be 16-byte aligned");
    const int nb = n / 256;
    G4_CHECK_ARG(nb <= 65535 && (size_t)m * q8_row_stride(nb) < (1u << 31) && (size_t)d * nb * 176 < (1u << 31),
                 "g4_mm_batch_q8_blocks: %d x %d weights or %d rows too large", d, n, m);
    if (type != G4_Q4_K && type != G4_Q5_K) return g4_fail(G4_ERR_TYPE, "g4_mm_batch_q8_blocks: type %d has no Q8_K batched path", type);
    KqSegs sg{};
    sg.n = 1;
    sg.w[0] = (const uint8_t*)w;
    sg.o[0] = u;
    sg.d[0] = d;
    sg.g0[0] = 0;
    sg.g0[1] = (d + 127) / 128;
    G4_CHECK_ARG((long long)sg.g0[1] * ((m + 31) / 32) < (1LL << 31), "g4_mm_batch_q8_blocks: %d tokens too many", m);
    const int gy = (m + 31) / 32;
    if (type == G4_Q4_K)
        hipLaunchKernelGGL((mm_batch_kq8_kernel<false, 1, 4, 1>), dim3(sg.g0[1] * gy, nb), dim3(256), 0, g4_stream(), sg,
                           (const uint8_t*)q8, nb, m);
    else
        hipLaunchKernelGGL((mm_batch_kq8_kernel<true, 1, 4, 1>), dim3(sg.g0[1] * gy, nb), dim3(256), 0, g4_stream(), sg,
                           (const uint8_t*)q8, nb, m);
    return g4_check_launch("mm_batch_kq8_kernel (per block)");
}

extern "C" size_t g4_kq_image_bytes(int n, int d) {
    return n > 0 && n % 256 == 0 && d > 0 ? kq_img_bytes(d, n / 256) : 0;
}

extern "C" int g4_kq_image(void* img, const void* w, int n, int d, int type) {
    G4_CHECK_ARG(img && w, "g4_kq_image: null pointer");
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && d > 0, "g4_kq_image: n=%d d=%d", n, d);
    G4_CHECK_ARG(al16(img) && al16(w), "g4_kq_image: img and w must be 16-byte aligned");
    if (type != G4_Q4_K && type != G4_Q5_K) return g4_fail(G4_ERR_TYPE, "g4_kq_image: type %d has no image", type);
    const int nb = n / 256, rg = (d + 31) / 32;
    G4_CHECK_ARG(kq_img_bytes(d, nb) < (1u << 31), "g4_kq_image: the image of %d x %d weights exceeds 2 GiB", d, n);
    const size_t threads = (size_t)rg * nb * 64;
    if (type == G4_Q4_K)
        hipLaunchKernelGGL(kq_image_kernel<false>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g4_stream(),
                           (const uint8_t*)w, (uint8_t*)img, d, nb, rg);
    else
        hipLaunchKernelGGL(kq_image_kernel<true>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, g4_stream(),
                           (const uint8_t*)w, (uint8_t*)img, d, nb, rg);
    return g4_check_launch("kq_image_kernel");
}

// tile: tokens per workgroup 32 nt, waves (32-row groups) nwv; 0 picks
static int mm_batch_img_tiled(float* const* o, const void* const* img, const int* d, int nseg, const void* q8, int n,
                              int m, int type, int nt, int nwv) {
    G4_CHECK_ARG(o && img && d && q8, "g4_mm_batch_img: null pointer");
    if (type != G4_Q4_K && type != G4_Q5_K) return g4_fail(G4_ERR_TYPE, "g4_mm_batch_img: type %d has no image", type);
    G4_CHECK_ARG(nseg >= 1 && nseg <= kMaxSegs, "g4_mm_batch_img: %d matrices (1..%d)", nseg, kMaxSegs);
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && m > 0, "g4_mm_batch_img: n=%d m=%d", n, m);
    G4_CHECK_ARG(al16(q8), "g4_mm_batch_img: q8 must be 16-byte aligned");
    const int nb = n / 256;
    G4_CHECK_ARG((size_t)m * q8_row_stride(nb) < (1u << 31), "g4_mm_batch_img: %d Q8_K rows exceed 2 GiB", m);
    for (int k = 0; k < nseg; k++) {
        G4_CHECK_ARG(o[k] && img[k], "g4_mm_batch_img: null pointer");
        G4_CHECK_ARG(al16(o[k]) && al16(img[k]), "g4_mm_batch_img: o and img must be 16-byte aligned");
        G4_CHECK_ARG(d[k] > 0 && kq_img_bytes(d[k], nb) < (1u << 31), "g4_mm_batch_img: d=%d", d[k]);
    }
    if (nt == 0 || nwv == 0) {
        // 64-token tiles when they give every CU a workgroup (eight-wave ones
        // from eight per CU), else 32-token tiles of 128 or 64 rows (511
        // tokens: 2x10240 rows 81.8 us with 64 x 128 tiles against 102.5 with
        // 32 x 128; 2560 x 2048 14.5 us with 32 x 128 against 19.5)
        auto wgs = [&](int t, int w) {
            long long g = 0;
            for (int k = 0; k < nseg; k++) g += (long long)((d[k] + 32 * w - 1) / (32 * w)) * ((m + 32 * t - 1) / (32 * t));
            return g;
        };
        // (Q5_K's four chains per block do not fit 64-token tiles in registers)
        const long long cus = g4_num_cus();
        const bool q5 = type == G4_Q5_K;
        if (!q5 && wgs(2, 4) >= 8 * cus) nt = 2, nwv = 8;
        else if (!q5 && wgs(2, 4) >= cus) nt = 2, nwv = 4;
        else if (wgs(1, 4) >= cus) nt = 1, nwv = 4;
        else nt = 1, nwv = 2;
    }
    G4_CHECK_ARG((nt == 1 && (nwv == 2 || nwv == 4 || nwv == 8)) || (nt == 2 && (nwv == 4 || nwv == 8)),
                 "g4_mm_batch_img: tile %d x %d", nt, nwv);
    const int rgw = 32 * nwv;   // rows per workgroup
    KqSegs sg{};
    sg.n = nseg;
    long long gx = 0;
    for (int k = 0; k < nseg; k++) {
        sg.w[k] = (const uint8_t*)img[k];
        sg.o[k] = o[k];
        sg.d[k] = d[k];
        sg.g0[k] = (int)gx;
        gx += (d[k] + rgw - 1) / rgw;
    }
    sg.g0[nseg] = (int)gx;
    G4_CHECK_ARG(gx * ((m + 32 * nt - 1) / (32 * nt)) < (1LL << 31), "g4_mm_batch_img: %d tokens too many", m);
    const uint8_t* q = (const uint8_t*)q8;
    const int key = 10 * nt + nwv;
    if (type == G4_Q4_K) {
        switch (key) {
        case 12: launch_mm_batch_img<false, 1, 2>(sg, q, nb, m); break;
        case 14: launch_mm_batch_img<false, 1, 4>(sg, q, nb, m); break;
        case 18: launch_mm_batch_img<false, 1, 8>(sg, q, nb, m); break;
        case 24: launch_mm_batch_img<false, 2, 4>(sg, q, nb, m); break;
        default: launch_mm_batch_img<false, 2, 8>(sg, q, nb, m); break;
        }
    } else {
        switch (key) {
        case 12: launch_mm_batch_img<true, 1, 2>(sg, q, nb, m); break;
        case 14: launch_mm_batch_img<true, 1, 4>(sg, q, nb, m); break;
        case 18: launch_mm_batch_img<true, 1, 8>(sg, q, nb, m); break;
        case 24: launch_mm_batch_img<true, 2, 4>(sg, q, nb, m); break;
        default: launch_mm_batch_img<true, 2, 8>(sg, q, nb, m); break;
        }
    }
    return g4_check_launch("mm_batch_img_kernel");
}

extern "C" int g4_mm_batch_img_multi(float* const* o, const void* const* img, const int* d, int nseg, const void* q8,
                                     int n, int m, int type) {
    return mm_batch_img_tiled(o, img, d, nseg, q8, n, m, type, 0, 0);
}

extern "C" int g4_mm_batch_img(float* o, const void* img, const void* q8, int n, int d, int m, int type) {
    return mm_batch_img_tiled(&o, &img, &d, 1, q8, n, m, type, 0, 0);
}

// the same with the tile given (tokens 32 nt, rows 32 nwv): shape sweeps
extern "C" int g4_mm_batch_img_tile(float* o, const void* img, const void* q8, int n, int d, int m, int type, int nt,
                                    int nwv) {
    return mm_batch_img_tiled(&o, &img, &d, 1, q8, n, m, type, nt, nwv);
}

// every block's int32 S_b and M_b as the batched kernels form them: S and M
// are [m][d][n/256]; image 0: the quantized tensor w (mm_batch_kq8_kernel),
// 1: its fp16 image (mm_batch_img_kernel, one-wave row groups of 32 tokens)
extern "C" int g4_debug_batch_block_sums(const void* w, int image, int n, int d, int m, int type, const void* q8,
                                         int32_t* S, int32_t* M) {
    G4_CHECK_ARG(w && q8 && S && M, "g4_debug_batch_block_sums: null pointer");
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && d > 0 && m > 0, "g4_debug_batch_block_sums: n=%d d=%d m=%d", n, d, m);
    G4_CHECK_ARG(al16(w) && al16(q8), "g4_debug_batch_block_sums: w and q8 must be 16-byte aligned");
    if (type != G4_Q4_K && type != G4_Q5_K)
        return g4_fail(G4_ERR_TYPE, "g4_debug_batch_block_sums: type %d has no Q8_K batched path", type);
    const int nb = n / 256;
    G4_CHECK_ARG((size_t)m * q8_row_stride(nb) < (1u << 31) && (size_t)d * nb * 176 < (1u << 31) &&
                     kq_img_bytes(d, nb) < (1u << 31),
                 "g4_debug_batch_block_sums: %d x %d weights or %d rows too large", d, n, m);
    KqSegs sg{};
    sg.n = 1;
    sg.w[0] = (const uint8_t*)w;
    sg.o[0] = reinterpret_cast<float*>(S);
    sg.o[1] = reinterpret_cast<float*>(M);   // read only by the block-sum mode
    sg.d[0] = d;
    sg.g0[0] = 0;
    const uint8_t* q = (const uint8_t*)q8;
    if (!image) {
        sg.g0[1] = (d + 127) / 128;
        if (type == G4_Q4_K) launch_mm_batch8<false, 1, 4, 2>(sg, q, nb, m);
        else launch_mm_batch8<true, 1, 4, 2>(sg, q, nb, m);
        return g4_check_launch("mm_batch_kq8_kernel (block sums)");
    }
    sg.g0[1] = (d + 127) / 128;
    if (type == G4_Q4_K) launch_mm_batch_img<false, 1, 4, 2>(sg, q, nb, m);
    else launch_mm_batch_img<true, 1, 4, 2>(sg, q, nb, m);
    return g4_check_launch("mm_batch_img_kernel (block sums)");
}

extern "C" int g4_fold_gelu_mul_q8(const float* u, const void* q8, int n, const float* ple, int pstride, float* out,
                                   void* q8o, int d, int m) {
    G4_CHECK_ARG(u && q8 && out && n > 0 && n % 256 == 0 && n / 256 <= kFoldMaxBlocks, "g4_fold_gelu_mul_q8: bad u, q8, out or n=%d", n);
    G4_CHECK_ARG(d > 0 && d <= kFoldMaxD && m > 0 && (!ple || pstride >= d), "g4_fold_gelu_mul_q8: d=%d m=%d", d, m);
    G4_CHECK_ARG(!q8o || d % 256 == 0, "g4_fold_gelu_mul_q8: Q8_K rows need d a multiple of 256 (d=%d)", d);
    hipLaunchKernelGGL(fold_gelu_mul_q8_kernel, dim3(m), dim3(256), 0, g4_stream(), u, (const uint8_t*)q8, n / 256, ple,
                       pstride, out, (uint8_t*)q8o, d, m);
    return g4_check_launch("fold_gelu_mul_q8_kernel");
}

extern "C" int g4_mm_batch(float* o, const float* x, const void* w, int n, int d, int m, int type, void* q8) {
    G4_CHECK_ARG(o && x && w && m > 0, "g4_mm_batch: bad arguments");
    if ((type == G4_Q6_K || type == G4_BF16) && n > 0 && n % 256 == 0 && d > 0 && al16(x) && al16(w)) {
        G4_CHECK_ARG((m + 15) / 16 <= 65535, "g4_mm_batch: m=%d too large", m);
        if (type == G4_Q6_K) launch_mm_batch_f32<false>((const uint8_t*)w, x, o, n, d, m);
        else launch_mm_batch_f32<true>((const uint8_t*)w, x, o, n, d, m);
        return g4_check_launch("mm_batch_f32_kernel");
    }
    if (type == G4_Q4_K || type == G4_Q5_K) {
        G4_CHECK_ARG(q8, "g4_mm_batch: null q8 workspace");
        int rc = g4_quantize_rows_q8_K(x, q8, n, m);
        if (rc) return rc;
        return g4_mm_batch_q8(o, w, q8, n, d, m, type);
    }
    // the other types take the per-token path (one GEMV launch per token)
    for (int t = 0; t < m; t++) {
        int rc = g4_mm(o + (size_t)t * d, x + (size_t)t * n, w, n, d, type, q8, 0);
        if (rc) return rc;
    }
    return G4_OK;
}

extern "C" size_t g4_split_rows_bytes(int n, int m) {
    return n > 0 && n % 256 == 0 && m > 0 ? (size_t)m * n * 4 + (size_t)m * 4 : 0;
}

extern "C" int g4_split_rows_f16(const float* x, void* xs, int n, int m) {
    G4_CHECK_ARG(x && xs, "g4_split_rows_f16: null pointer");
    G4_CHECK_ARG(n > 0 && n % 256 == 0, "g4_split_rows_f16: n=%d is not a positive multiple of 256", n);
    G4_CHECK_ARG(m > 0, "g4_split_rows_f16: m=%d", m);
    G4_CHECK_ARG(al16(x) && al16(xs), "g4_split_rows_f16: x and xs must be 16-byte aligned");
    hipLaunchKernelGGL(split_rows_f16_kernel, dim3(m), dim3(256), 0, g4_stream(), x, (uint8_t*)xs, n, m);
    return g4_check_launch("split_rows_f16_kernel");
}

extern "C" int g4_gelu_mul_split_rows(const float* g, const float* u, int ustride, void* xs, int n, int m) {
    G4_CHECK_ARG(g && u && xs, "g4_gelu_mul_split_rows: null pointer");
    G4_CHECK_ARG(n == 2048 || n == 4096 || n == 8192 || n == 10240 || n == 12288 || n == 16384,
                 "g4_gelu_mul_split_rows: n=%d (2048 * k, k in 1, 2, 4, 5, 6, 8)", n);
    G4_CHECK_ARG(m > 0 && ustride >= n && ustride % 4 == 0, "g4_gelu_mul_split_rows: m=%d ustride=%d", m, ustride);
    G4_CHECK_ARG(al16(g) && al16(u) && al16(xs), "g4_gelu_mul_split_rows: g, u and xs must be 16-byte aligned");
    const dim3 grid(m), blk(256);
    uint8_t* x = (uint8_t*)xs;
    switch (n / 2048) {
    case 1: hipLaunchKernelGGL(gelu_mul_split_kernel<1>, grid, blk, 0, g4_stream(), g, u, ustride, x, n, m); break;
    case 2: hipLaunchKernelGGL(gelu_mul_split_kernel<2>, grid, blk, 0, g4_stream(), g, u, ustride, x, n, m); break;
    case 4: hipLaunchKernelGGL(gelu_mul_split_kernel<4>, grid, blk, 0, g4_stream(), g, u, ustride, x, n, m); break;
    case 5: hipLaunchKernelGGL(gelu_mul_split_kernel<5>, grid, blk, 0, g4_stream(), g, u, ustride, x, n, m); break;
    case 6: hipLaunchKernelGGL(gelu_mul_split_kernel<6>, grid, blk, 0, g4_stream(), g, u, ustride, x, n, m); break;
    default: hipLaunchKernelGGL(gelu_mul_split_kernel<8>, grid, blk, 0, g4_stream(), g, u, ustride, x, n, m); break;
    }
    return g4_check_launch("gelu_mul_split_kernel");
}

extern "C" int g4_mm_batch_split(float* o, const void* w, const void* xs, int n, int d, int m, int type) {
    G4_CHECK_ARG(o && w && xs, "g4_mm_batch_split: null pointer");
    // the kernel addresses both operands with 32-bit buffer offsets
    G4_CHECK_ARG((size_t)m * n * 4 < (1u << 31) && (size_t)d * (n / 256) * 210 < (1u << 31),
                 "g4_mm_batch_split: %d x %d weights or %d rows exceed 2 GiB", d, n, m);
    G4_CHECK_ARG(al16(w) && al16(xs), "g4_mm_batch_split: w and xs must be 16-byte aligned");
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && d > 0 && m > 0, "g4_mm_batch_split: n=%d d=%d m=%d", n, d, m);
    // (the largest grid of the workgroup shapes: 64 rows x 16 tokens)
    G4_CHECK_ARG((long long)((d + 63) / 64) * ((m + 15) / 16) < (1LL << 31), "g4_mm_batch_split: %d x %d outputs too many",
                 m, d);
    if (type != G4_Q6_K) return g4_fail(G4_ERR_TYPE, "g4_mm_batch_split: type %d has no split-activation path", type);
    launch_q6s_auto((const uint8_t*)w, (const uint8_t*)xs, o, n, d, m);
    return g4_check_launch("mm_batch_q6s_kernel");
}
