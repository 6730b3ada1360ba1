// prefill.hip -- many tokens through one K-quant matrix at once (prefill):
// Y[m x d] = Q8_K(X[m x n]) . W[d x n]^T on the gfx950 matrix cores, with
// every output bit-identical to the per-token GEMV (gemv.hip) and hence to
// the reference's AVX2 dot, vec_dot_q4_K_q8_K / vec_dot_q5_K_q8_K
// (gemma4-4b/cpu-blas/main.c:476-529, 531-593).  The reference has no
// batched path: generate() calls forward() once per prompt token
// (main.c:2366-2384), i.e. quantize_row_q8_K + mm_quant_dot_rows per token.
//
// Exactness.  The AVX2 dot keeps, per block, eight int32 lanes
//   sumi[k] = sum_j sc_j * sum_{e<4} q[32j + 4k + e] * q8[32j + 4k + e]
// (j = sub-block, k = lane), plus four min lanes (Q4_K)
//   prod[p] = m_2p * (bs_4p + bs_4p+1) + m_2p+1 * (bs_4p+2 + bs_4p+3)
// or their sum (Q5_K), and folds them into fp32 accumulators with the
// block's d = y.d * fp16(x.d) and dmin = -y.d * fp16(x.dmin).  Here the
// lane-k sums are matrix-core products over a 32-long K axis that gathers
// positions 4k..4k+3 of all eight sub-blocks, with the sub-block scale
// folded into the weight (sc * q <= 63 * 31 = 1953) and the activation as
// fp16 (|q8| <= 128): every product and every partial sum is an integer
// below 2^24 in magnitude, so the fp32 accumulation inside the matrix core
// is exact whatever its order, and equals the int32 lane sum.  The min
// lanes are 16-long products of m_j with the 16-element bsums (|bs| <=
// 2032, exact in fp16).  The fp32 steps after that (d*sumi FMA per lane and
// block in block order, the fixed horizontal-add tree) are the reference's.
//
// Work split.  A 256-thread workgroup owns 64 weight rows x 32 tokens:
// four row waves of 16 rows, each with two 16x16 output tiles (32 tokens).
// Per block the workgroup stages the 32 tokens' activations into LDS as
// fp16, already in the lane-k order; each wave
// builds its weight operand (codes * scale as fp16) in registers from the
// planar Q4_K/Q5_K bytes.  The next block's bytes are loaded into
// registers while the current block is computed.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int kPfTokStride = 528;    // LDS bytes per staged token (512 + pad)
constexpr int kPfBsStride = 32;      // LDS bytes per token of fp16 bsums

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

// four codes c (one per byte, < 256) -> four fp16 c * s, exactly:
// fma(1024 + c, s, -1024 s) is c * s (an integer < 2048) before rounding
__device__ __forceinline__ uint2 codes_to_h4(uint32_t c, h2_t s, h2_t ns) {
    const h2_t lo = __builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(kMagic, c, kSelLo)), s, ns);
    const h2_t hi = __builtin_elementwise_fma(bits_h2(__builtin_amdgcn_perm(kMagic, c, kSelHi)), s, ns);
    return make_uint2(h2_bits(lo), h2_bits(hi));
}

__device__ __forceinline__ float hbits_to_f32(uint32_t h) {
    _Float16 v;
    const uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// RW row waves x TW token waves; each wave owns 16 rows x NT 16-token tiles.
// At least WPE waves per SIMD caps the VGPRs at 512 / WPE: at 256 or fewer the
// compiler writes the matrix-core results straight to VGPRs instead of going
// through accumulation registers (a v_accvgpr_read per result element).
template <bool Q5, int RW, int TW, int NT, int WPE = 2>
__global__ __launch_bounds__(64 * RW * TW) __attribute__((amdgpu_waves_per_eu(WPE))) void mm_batch_kq_kernel(const uint8_t* __restrict__ w,
                                                                    const uint8_t* __restrict__ q8,
                                                                    float* __restrict__ out, int nb, int d, int m) {
    constexpr int NTHR = 64 * RW * TW;
    constexpr int TOK = 16 * NT * TW;                      // tokens per workgroup
    constexpr int UNITS = TOK * 8;                          // (token, lane-k) staging units
    constexpr int UPT = (UNITS + NTHR - 1) / NTHR;          // units per thread
    constexpr int BQ = (TOK * 4 + NTHR - 1) / NTHR;         // bsums quarters per thread
    __shared__ __align__(16) uint8_t sB[TOK * kPfTokStride];
    __shared__ __align__(16) uint8_t sS[TOK * kPfBsStride];
    __shared__ float sD[TOK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, g = lane >> 4;               // operand row / column, K group
    const int rw = wave % RW, tw = wave / RW;              // row wave, token wave
    const int row0 = blockIdx.x * (16 * RW) + rw * 16;
    const int tokb = blockIdx.y * TOK;
    const int tw0 = tw * 16 * NT;                          // first token of this wave (in the workgroup)
    const size_t nblk = (size_t)d * nb;
    const size_t hdr_off = (Q5 ? 160 : 128) * nblk, qh_off = 128 * nblk;
    const size_t q8row = ((size_t)nb * 292 + 63) & ~(size_t)63;   // q8_row_stride

    // weight operand row of this lane, and the four output rows 4g+v
    const size_t rA = (size_t)min(row0 + i, d - 1) * nb;
    size_t rD[4];
#pragma unroll
    for (int v = 0; v < 4; v++) rD[v] = (size_t)min(row0 + 4 * g + v, d - 1) * nb;

    struct WRaw {
        uint32_t qs[8];
        uint32_t qh[8];
        uint4 hdr;
        uint32_t dh[4];
    };
    struct XRaw {
        uint4 a0[UPT], a1[UPT];
        uint2 bs[BQ];
        float yd;
    };
    auto load_w = [&](int b, WRaw& r) {
        const uint8_t* qa = w + (rA + b) * 128 + 4 * g;
#pragma unroll
        for (int k = 0; k < 8; k++) r.qs[k] = *reinterpret_cast<const uint32_t*>(qa + 16 * k);
        if (Q5) {
            const uint8_t* ha = w + qh_off + (rA + b) * 32;
#pragma unroll
            for (int k = 0; k < 8; k++) r.qh[k] = *reinterpret_cast<const uint32_t*>(ha + 4 * k);
        }
        r.hdr = *reinterpret_cast<const uint4*>(w + hdr_off + (rA + b) * 16);
#pragma unroll
        for (int v = 0; v < 4; v++) r.dh[v] = *reinterpret_cast<const uint32_t*>(w + hdr_off + (rD[v] + b) * 16);
    };
    // unit u = tid + j*NTHR: token u >> 3, lane-k u & 7 (its 32 device bytes)
    auto load_x = [&](int b, XRaw& r) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * NTHR;
            r.a0[j] = make_uint4(0u, 0u, 0u, 0u);
            r.a1[j] = r.a0[j];
            if (UNITS % NTHR == 0 || u < UNITS) {
                const uint8_t* p = q8 + (size_t)min(tokb + (u >> 3), m - 1) * q8row + (size_t)b * 256 + 32 * (u & 7);
                r.a0[j] = *reinterpret_cast<const uint4*>(p);
                r.a1[j] = *reinterpret_cast<const uint4*>(p + 16);
            }
        }
#pragma unroll
        for (int j = 0; j < BQ; j++) {
            const int u = tid + j * NTHR;
            r.bs[j] = make_uint2(0u, 0u);
            if (u < TOK * 4)
                r.bs[j] = *reinterpret_cast<const uint2*>(q8 + (size_t)min(tokb + (u >> 2), m - 1) * q8row +
                                                          q8k_bsums_off(nb) + (size_t)b * 32 + 8 * (u & 3));
        }
        r.yd = 0.0f;
        if (tid < TOK) r.yd = reinterpret_cast<const float*>(q8 + (size_t)min(tokb + tid, m - 1) * q8row +
                                                             q8k_d_off(nb))[b];
    };
    // activations of one block -> LDS: token t, lane k: the K group g entry
    // is 8 halves = device words g of a0 (sub-block 2g) and of a1 (sub-block
    // 2g+1), i.e. q8 elements 64g+4k+e and 64g+32+4k+e
    auto stage = [&](const XRaw& r) {
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = tid + j * NTHR;
            if (UNITS % NTHR == 0 || u < UNITS) {
                const bool ok = tokb + (u >> 3) < m;
                uint8_t* dst = sB + (u >> 3) * kPfTokStride + 64 * (u & 7);
                const uint32_t a0[4] = {r.a0[j].x, r.a0[j].y, r.a0[j].z, r.a0[j].w};
                const uint32_t a1[4] = {r.a1[j].x, r.a1[j].y, r.a1[j].z, r.a1[j].w};
#pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    uint4 h = make_uint4(0u, 0u, 0u, 0u);
                    if (ok) {
                        const uint2 l = i8x4_to_h4(a0[gg]), hh = i8x4_to_h4(a1[gg]);
                        h = make_uint4(l.x, l.y, hh.x, hh.y);
                    }
                    *reinterpret_cast<uint4*>(dst + 16 * gg) = h;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < BQ; j++) {
            const int u = tid + j * NTHR;
            if (u < TOK * 4) {
                uint2 h = make_uint2(0u, 0u);
                if (tokb + (u >> 2) < m) {
                    const h2_t lo = {(_Float16)(int16_t)(r.bs[j].x & 0xffffu), (_Float16)(int16_t)(r.bs[j].x >> 16)};
                    const h2_t hi = {(_Float16)(int16_t)(r.bs[j].y & 0xffffu), (_Float16)(int16_t)(r.bs[j].y >> 16)};
                    h = make_uint2(h2_bits(lo), h2_bits(hi));
                }
                *reinterpret_cast<uint2*>(sS + (u >> 2) * kPfBsStride + 8 * (u & 3)) = h;
            }
        }
        if (tid < TOK) sD[tid] = tokb + tid < m ? r.yd : 0.0f;
    };

    f4_t acc[NT][8];
    f4_t accm[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
        for (int k = 0; k < 8; k++) acc[t][k] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < 4; p++) accm[t][p] = f4_t{0.f, 0.f, 0.f, 0.f};
    }
    const f4_t zero = {0.f, 0.f, 0.f, 0.f};

    WRaw wn;
    XRaw xn;
    load_w(0, wn);
    load_x(0, xn);
    for (int b = 0; b < nb; b++) {
        __syncthreads();   // the previous block's LDS reads are done
        stage(xn);
        const WRaw wc = wn;
        if (b + 1 < nb) {
            load_w(b + 1, wn);
            load_x(b + 1, xn);
        }
        __syncthreads();

        // scales of this lane's operand row: sub-blocks 2g, 2g+1
        uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
        unpack_scales(wc.hdr.y, wc.hdr.z, wc.hdr.w, sc_lo, sc_hi, mn_lo, mn_hi);
        const int sh = 16 * (g & 1);
        const uint32_t scw = g < 2 ? sc_lo : sc_hi, mnw = g < 2 ? mn_lo : mn_hi;
        const _Float16 sa = (_Float16)(float)((scw >> sh) & 0xffu), sb = (_Float16)(float)((scw >> (sh + 8)) & 0xffu);
        const _Float16 ma = (_Float16)(float)((mnw >> sh) & 0xffu), mb = (_Float16)(float)((mnw >> (sh + 8)) & 0xffu);
        const h2_t SA = {sa, sa}, SB = {sb, sb};
        const h2_t NA = {(_Float16)(-1024.0f) * sa, (_Float16)(-1024.0f) * sa};
        const h2_t NB = {(_Float16)(-1024.0f) * sb, (_Float16)(-1024.0f) * sb};

        // fp32 scales of the four output rows x the token tiles
        float dd[NT][4], dm[NT][4];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const float yd = sD[tw0 + 16 * t + i];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                dd[t][v] = yd * hbits_to_f32(wc.dh[v] & 0xffffu);
                dm[t][v] = -yd * hbits_to_f32(wc.dh[v] >> 16);
            }
        }
        const uint8_t* bt0 = sB + (tw0 + i) * kPfTokStride + 16 * g;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t lo = wc.qs[k] & 0x0f0f0f0fu, hi = (wc.qs[k] >> 4) & 0x0f0f0f0fu;
            if (Q5) {
                lo |= ((wc.qh[k] >> (2 * g)) & 0x01010101u) << 4;
                hi |= ((wc.qh[k] >> (2 * g + 1)) & 0x01010101u) << 4;
            }
            const uint2 al = codes_to_h4(lo, SA, NA), ah = codes_to_h4(hi, SB, NB);
            const h8_t A = __builtin_bit_cast(h8_t, make_uint4(al.x, al.y, ah.x, ah.y));
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const h8_t B = *reinterpret_cast<const h8_t*>(bt0 + 16 * t * kPfTokStride + 64 * k);
                const f4_t D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) acc[t][k][v] = __builtin_fmaf(dd[t][v], D[v], acc[t][k][v]);
            }
        }
        // min lanes: lane group g carries bsums 4g..4g+3 (sub-blocks 2g, 2g+1)
        const _Float16 z = (_Float16)0.0f;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const h4_t Bm = *reinterpret_cast<const h4_t*>(sS + (tw0 + 16 * t + i) * kPfBsStride + 8 * g);
            if (Q5) {
                const h4_t Am = {ma, ma, mb, mb};
                const f4_t P = __builtin_amdgcn_mfma_f32_16x16x16f16(Am, Bm, zero, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float tm = dm[t][v] * P[v];
                    accm[t][0][v] = accm[t][0][v] + tm;
                }
            } else {
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const h4_t Am = g == p ? h4_t{ma, ma, mb, mb} : h4_t{z, z, z, z};
                    const f4_t P = __builtin_amdgcn_mfma_f32_16x16x16f16(Am, Bm, zero, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++) accm[t][p][v] = __builtin_fmaf(dm[t][v], P[v], accm[t][p][v]);
                }
            }
        }
    }

    // the reference's horizontal adds (hsum_float_8, then the min lanes)
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int tok = tokb + tw0 + 16 * t + i;
        float r[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float h = ((acc[t][4][v] + acc[t][0][v]) + (acc[t][6][v] + acc[t][2][v])) +
                            ((acc[t][5][v] + acc[t][1][v]) + (acc[t][7][v] + acc[t][3][v]));
            if (Q5) {
                r[v] = h + accm[t][0][v];
            } else {
                const float hm = (accm[t][0][v] + accm[t][2][v]) + (accm[t][1][v] + accm[t][3][v]);
                r[v] = h + hm;
            }
        }
        if (tok < m) {
            const int rowo = row0 + 4 * g;
            float* o = out + (size_t)tok * d + rowo;
            if (rowo + 3 < d && ((d & 3) == 0)) {
                *reinterpret_cast<float4*>(o) = make_float4(r[0], r[1], r[2], r[3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (rowo + v < d) o[v] = r[v];
            }
        }
    }
}

// the shipped tiling (fastest of a sweep over 1..8 row waves, 1..4 token
// waves, 1..4 tiles at E4B shapes and 512 tokens): 4 row waves x 1 token
// wave x 2 tiles = 64 rows x 32 tokens per 256-thread workgroup
constexpr int kRW = 4, kTW = 1, kNT = 2;
constexpr int kPfToks = 16 * kNT * kTW;

template <bool Q5, int RW, int TW, int NT, int WPE = 2>
void launch_mm_batch(const uint8_t* w, const uint8_t* q8, float* o, int nb, int d, int m) {
    const dim3 grid((d + 16 * RW - 1) / (16 * RW), (m + 16 * NT * TW - 1) / (16 * NT * TW));
    hipLaunchKernelGGL((mm_batch_kq_kernel<Q5, RW, TW, NT, WPE>), grid, dim3(64 * RW * TW), 0, g4_stream(), w, q8, o,
                       nb, d, m);
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
        __syncthreads();   // the previous block's LDS reads are done
        stage(xn);
        const WRaw wc = wn;
        // the next block (the last one again at the end: an unconditional
        // load keeps the prefetch registers out of scratch memory)
        const int bn = min(b + 1, nb - 1);
        load_w(bn, wn);
        load_x(bn, xn);
        __syncthreads();

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

extern "C" int g4_mm_batch_q8(float* o, const void* w, const void* q8, int n, int d, int m, int type) {
    G4_CHECK_ARG(o && w && q8, "g4_mm_batch_q8: null pointer");
    G4_CHECK_ARG(al16(o), "g4_mm_batch_q8: o must be 16-byte aligned");
    G4_CHECK_ARG(al16(w) && al16(q8), "g4_mm_batch_q8: w and q8 must be 16-byte aligned");
    G4_CHECK_ARG(n > 0 && n % 256 == 0 && d > 0 && m > 0, "g4_mm_batch_q8: n=%d d=%d m=%d", n, d, m);
    G4_CHECK_ARG(m <= 65535 * kPfToks, "g4_mm_batch_q8: m=%d too large", m);
    const int nb = n / 256;
    if (type == G4_Q4_K) {
        launch_mm_batch<false, kRW, kTW, kNT>((const uint8_t*)w, (const uint8_t*)q8, o, nb, d, m);
    } else if (type == G4_Q5_K) {
        launch_mm_batch<true, kRW, kTW, kNT>((const uint8_t*)w, (const uint8_t*)q8, o, nb, d, m);
    } else {
        return g4_fail(G4_ERR_TYPE, "g4_mm_batch_q8: type %d has no Q8_K batched path", type);
    }
    return g4_check_launch("mm_batch_kq_kernel");
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
