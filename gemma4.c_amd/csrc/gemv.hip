// gemv.hip -- K-quant GEMV kernels for gfx950 (decode, batch 1).
//
// o[d] = W[d x n] . x   (W row-major, ne[0] = n; gemma4-4b/cpu-blas/main.c:1669)
//
// Q4_K / Q5_K x Q8_K (mm_quant_dot_rows): one row per 8-lane group, bit-exact
// with the reference's AVX2 dot (see gemv_q45_rows_kernel).
// Q6_K x fp32 (mm_quant_rows): row slices per 8-lane group with x in LDS,
// fp32 tolerance (see gemv_q6k_rows_kernel).
// Q6_K x Q8_K (integer, no reference counterpart) and BF16 x fp32: 256-thread
// workgroups of 32 row tasks.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

constexpr int kWG = 256;      // threads per workgroup
constexpr int kGroups = 32;   // 8-lane groups per workgroup

__device__ __forceinline__ uint32_t word_of(const uint4& v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
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
    const int row0 = (blockIdx.x * 4 + wave) * RPW;
    uint4 v[RPW][CPL];
    bf16_rows_load<RPW, CPL>(w, n, d, row0, lane, v);
    for (int k = tid; k < n / 4; k += kWG) reinterpret_cast<float4*>(xs)[k] = reinterpret_cast<const float4*>(x)[k];
    __syncthreads();
    float res[RPW];
    bf16_rows_dot<RPW, CPL>(v, xs, n / 8, lane, res);
#pragma unroll
    for (int r = 0; r < RPW; r++)
        if (lane == 0 && row0 + r < d) out[row0 + r] = res[r];
}

// ------------------------------------------------------------------------
// Q4_K / Q5_K x Q8_K (the decode path)
// ------------------------------------------------------------------------
// A row is owned by SPLIT 8-lane groups.  Lane l of a group takes bytes
// 4l..4l+3 of every 32-byte qs chunk of a block (the AVX2 lane partition,
// main.c:500-523) and computes that block's exact integer sums (sumi: the
// scaled nibble dots, prod: the min products) and its fp32 scales
// D = y.d * d and DM = -y.d * dmin.  Group g takes blocks g*NH .. g*NH+NH-1;
// the other groups' values are gathered by lane shuffles into group 0, which
// runs the reference's fp32 accumulation over the blocks in order (eight FMA
// lanes plus four min lanes for Q4_K, one scalar min lane for Q5_K) and its
// fixed horizontal-add tree -- bit-identical to main.c:476-529 / 531-593.
// Splitting the integer work over two groups doubles the waves in flight;
// 64-thread workgroups carry 8/SPLIT rows.  fp16 d/dmin are converted by
// the hardware (exact, subnormals included).
__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
    _Float16 v;
    const uint16_t b = (uint16_t)h;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// QIN (single-block rows only): the workgroup quantizes the fp32 input xin
// itself (the one Q8_K block, exactly as quantize_row_q8_K) into LDS, and
// workgroup 0 also stores it to q8 -- the reference's mm() side effect.
// aux (nullable, NMAT == 1): epilogue out = gelu(r) * aux[row]
// (main.c:1989-1993).
// a second tensor stacked under the first (same type and n, own output),
// and (prologue kernels) a Q6_K tensor taking the fp32 normed vector the
// prologue leaves in LDS, as mm_quant_rows does (main.c:1539-1556)
struct Stack2 {
    const uint8_t* w;
    float* out;
    int d;
    const uint8_t* w6;
    float* out6;
    int d6;
};
// attention merge prologue (PRO 2): the G chunk partials (o[hd], max, sum)
// of each head (head_dim 256 or 512: hb = hd / 256 Q8_K blocks per head) as
// attn_chunk_kernel leaves them; out / q8: the merged vector and its Q8_K
// (workgroup 0, each optional)
struct MergeArgs {
    const float* part;
    float* out;
    uint8_t* q8;
    int G;
    int hb;
};
constexpr int kMergeMaxG = G4_MERGE_MAX_CHUNKS;   // chunks per head the merge prologue holds in registers

// Q6_K rows per prologue workgroup of wg threads: wg/8 lane groups, ks6 per row
constexpr int q6_pro_rows(int wg, int ks6) { return wg / 8 / ks6; }

// Q6_K rows of a prologue kernel's workgroup vb: WG threads, q6_pro_rows(WG,
// KS6) rows x KS6 slices, x = the fp32 normed vector (the prologue's nv, staged
// here in pbuf); same lane mapping and arithmetic as gemv_q6k_rows_kernel
// (below).  The weight loads are issued before the prologue's arithmetic.
template <int NB, int WG, int KS6>
__device__ __forceinline__ void q6k_prologue_rows(const Stack2& st, int vb, const ResidualArgs& ra, const Res4& r4,
                                                  float* pbuf, float (*red)[16]) {
    constexpr int QB = (NB + KS6 - 1) / KS6;
    constexpr int R6 = q6_pro_rows(WG, KS6);
    const int tid = threadIdx.x, L = tid & 7, g = tid >> 3, h = L >> 2, u = L & 3;
    const int rr6 = g % R6, ks = g / R6;
    const int row_ = vb * R6 + rr6, row = min(row_, st.d6 - 1);
    const Q6KPlanes P = q6k_planes((size_t)st.d6 * NB);
    uint4 qlv[QB];
    uint2 qhv[QB], scv[QB];
    uint32_t dv[QB];
#pragma unroll
    for (int i = 0; i < QB; i++) {
        const size_t blk = (size_t)row * NB + min(ks + i * KS6, NB - 1);
        qlv[i] = *reinterpret_cast<const uint4*>(st.w6 + P.ql + blk * 128 + 16 * L);
        qhv[i] = *reinterpret_cast<const uint2*>(st.w6 + P.qh + blk * 64 + 8 * L);
        scv[i] = *reinterpret_cast<const uint2*>(st.w6 + P.sc + blk * 16 + 8 * h);
        dv[i] = *reinterpret_cast<const uint16_t*>(st.w6 + P.d + blk * 2);
    }
    float q[4], nv[4];
    residual4_finish(ra, r4, red, false, 0, q, nv);
    reinterpret_cast<float4*>(pbuf)[tid] = make_float4(nv[0], nv[1], nv[2], nv[3]);
    // sums of the runs of 8 of x: this thread's 4 and its neighbour's
    float* x8 = pbuf + NB * 256 + ((NB * 292 + 15) & ~15) / 4;
    const float s4 = (nv[0] + nv[1]) + (nv[2] + nv[3]);
    const float o4 = __shfl_xor(s4, 1, 64);
    if ((tid & 1) == 0) x8[tid >> 1] = s4 + o4;
    lds_sync();
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < QB; i++) {
        const int b = ks + i * KS6;
        if (b < NB) {
            const uint4 ql = qlv[i];
            const uint2 qh = qhv[i], sc = scv[i];
            const float df = half_bits_to_f32(dv[i]);
            const float* xb = pbuf + b * 256 + 128 * h + 8 * u;
            const float* sb8 = x8 + b * 32 + 16 * h + u;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const uint32_t qa = (kk & 1) ? ql.z : ql.x;
                const uint32_t qb = (kk & 1) ? ql.w : ql.y;
                const uint32_t la = kk < 2 ? (qa & 0x0f0f0f0fu) : ((qa >> 4) & 0x0f0f0f0fu);
                const uint32_t lb = kk < 2 ? (qb & 0x0f0f0f0fu) : ((qb >> 4) & 0x0f0f0f0fu);
                const uint32_t ca = la | (((qh.x >> (2 * kk)) & 0x03030303u) << 4);
                const uint32_t cb = lb | (((qh.y >> (2 * kk)) & 0x03030303u) << 4);
                const float4 x0 = *reinterpret_cast<const float4*>(xb + 32 * kk);
                const float4 x1 = *reinterpret_cast<const float4*>(xb + 32 * kk + 4);
                float dot = x0.x * (float)(ca & 0xff);
                dot = __builtin_fmaf(x0.y, (float)((ca >> 8) & 0xff), dot);
                dot = __builtin_fmaf(x0.z, (float)((ca >> 16) & 0xff), dot);
                dot = __builtin_fmaf(x0.w, (float)(ca >> 24), dot);
                dot = __builtin_fmaf(x1.x, (float)(cb & 0xff), dot);
                dot = __builtin_fmaf(x1.y, (float)((cb >> 8) & 0xff), dot);
                dot = __builtin_fmaf(x1.z, (float)((cb >> 16) & 0xff), dot);
                dot = __builtin_fmaf(x1.w, (float)(cb >> 24), dot);
                dot = __builtin_fmaf(-32.0f, sb8[4 * kk], dot);
                const int sbi = (u >> 1) + 2 * kk;
                const int8_t s8 = (int8_t)byte_of(sbi < 4 ? sc.x : sc.y, sbi & 3);
                acc = __builtin_fmaf(df * (float)s8, dot, acc);
            }
        }
    }
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    acc += __shfl_xor(acc, 4, 64);
    float* part = x8 + NB * 32;
    if (L == 0) part[g] = acc;
    lds_sync();
    if (tid < R6) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < KS6; j++) sum += part[j * R6 + tid];
        if (vb * R6 + tid < st.d6) st.out6[vb * R6 + tid] = sum;
    }
    (void)row_;
}

// PRO 1: residual prologue (ra, st); PRO 2: attention merge prologue (mg).
// LG: the lane groups of a row hand their block values to group 0 through
// LDS (one write and one read per block) instead of lane shuffles.
//
// The body runs as workgroup bid with thread index tid (a workgroup of WG
// threads); q8s: 292 bytes of LDS for the QIN path's Q8_K block; xload(t):
// the QIN input float4 of lane t (XL: read after the weight loads are
// issued instead of before); put(o, row, v) stores an output.
template <bool Q5, int NMAT, bool DBG, int NB, int SPLIT, bool QIN, int WG, int PRO, bool LG, int KS6, bool XL,
          typename XIn, typename Put>
__device__ __forceinline__ void q45_rows_body(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                              const uint8_t* q8, float* __restrict__ out, int nb_rt, int d,
                                              int32_t* __restrict__ dbgS, int32_t* __restrict__ dbgM,
                                              uint8_t* __restrict__ q8_store, const float* __restrict__ aux,
                                              const ResidualArgs& ra, const Stack2& st, const MergeArgs& mg, int bid,
                                              int tid, uint8_t* q8s, XIn&& xload, Put&& put) {
    static_assert(!QIN || (WG == 64 && NB == 1), "the single-block input path runs one wave over one block");
    static_assert(!PRO || (WG == 64 * NB && NB > 0 && !DBG), "the prologue needs one wave per block");
    static_assert(PRO != 2 || NMAT == 1, "the merge prologue feeds one matrix");
    constexpr int GL = 8 * SPLIT;                               // lanes per row
    constexpr int NH = NB > 0 ? (NB + SPLIT - 1) / SPLIT : 1;   // blocks per group (unrolled case)
    const int nb = NB > 0 ? NB : nb_rt;
    const int l = tid & 7, k = l & 3, grp = SPLIT > 1 ? (tid >> 3) & (SPLIT - 1) : 0;
    const int row_ = bid * (WG / GL) + tid / GL;
    // with the prologue (or the input quantized in the wave) every thread
    // stays for its barriers; rows past the end compute the last row and do
    // not store.  Rows d.. d+st.d-1 (PRO only) belong to the stacked second
    // tensor.
    const int dtot = d + (PRO == 1 ? st.d : 0);
    const int row = (PRO || QIN) ? min(row_, dtot - 1) : row_;
    const bool sec = PRO == 1 && row >= d;
    const int dl = sec ? st.d : d, rl = sec ? row - d : row;
    const uint8_t* const wa = sec ? st.w : w0;
    float* const outp = sec ? st.out : out;
    if (!PRO && !QIN && row >= d) return;   // whole rows (groups of GL lanes) leave together
    const uint32_t nblk = (uint32_t)dl * (uint32_t)nb;
    const uint32_t hdr_off = (Q5 ? 160u : 128u) * nblk;          // q4k_planes / q5k_planes
    const uint32_t qh_off = 128u * nblk;
    const uint32_t rb = (uint32_t)rl * (uint32_t)nb;             // first block of the row
    // the epilogue's multiplier, loaded now (without one: this row of the
    // output, which only this group writes, read and not used)
    const float aux_v = (aux ? aux : outp)[rl];
    const uint8_t* a_qs = q8 + 32 * l;
    const uint8_t* a_bs = q8 + q8k_bsums_off(nb) + 8 * k;
    const float* a_d = reinterpret_cast<const float*>(q8 + q8k_d_off(nb));

    // raw operands of one block (both matrices share the activation block)
    struct Raw {
        uint4 a0, a1, wq[NMAT], hd[NMAT];
        uint2 bsw;
        uint32_t qh[NMAT];
        float yd;
    };
    auto load_a = [&](int b, Raw& r) {
        r.a0 = *reinterpret_cast<const uint4*>(a_qs + b * 256);
        r.a1 = *reinterpret_cast<const uint4*>(a_qs + b * 256 + 16);
        r.bsw = *reinterpret_cast<const uint2*>(a_bs + b * 32);
        r.yd = a_d[b];
    };
    auto load_w = [&](int b, Raw& r) {
        const uint32_t blk = rb + (uint32_t)b;
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            const uint8_t* base = m ? w1 : wa;
            r.wq[m] = *reinterpret_cast<const uint4*>(base + blk * 128u + 16 * l);
            r.hd[m] = *reinterpret_cast<const uint4*>(base + hdr_off + blk * 16u);
            r.qh[m] = Q5 ? *reinterpret_cast<const uint32_t*>(base + qh_off + blk * 32u + 4 * l) : 0u;
        }
    };
    auto load = [&](int b, Raw& r) {
        load_a(b, r);
        load_w(b, r);
    };
    // one block's integer sums and fp32 scales for matrix m
    auto block = [&](int m, int b, const Raw& r, int32_t& S, int32_t& P, float& D, float& DM) {
        const int bs_lo = (int)(int16_t)(r.bsw.x & 0xffffu) + (int)(int16_t)(r.bsw.x >> 16);
        const int bs_hi = (int)(int16_t)(r.bsw.y & 0xffffu) + (int)(int16_t)(r.bsw.y >> 16);
        const uint4 wq = r.wq[m], hd = r.hd[m];
        const uint32_t qh = r.qh[m];
        uint32_t sc_lo, sc_hi, mn_lo, mn_hi;
        unpack_scales(hd.y, hd.z, hd.w, sc_lo, sc_hi, mn_lo, mn_hi);
        int32_t sumi = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t qw = word_of(wq, j);
            uint32_t lo = qw & 0x0f0f0f0fu, hi = (qw >> 4) & 0x0f0f0f0fu;
            if (Q5) {
                lo |= ((qh >> (2 * j)) & 0x01010101u) << 4;
                hi |= ((qh >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            const int dl = __builtin_amdgcn_sdot4((int)lo, (int)word_of(r.a0, j), 0, false);
            const int dh = __builtin_amdgcn_sdot4((int)hi, (int)word_of(r.a1, j), 0, false);
            const uint32_t scw = j < 2 ? sc_lo : sc_hi;
            // |dl|, |dh| <= 4*31*127 and scales <= 63: exact in 24-bit products
            sumi += __mul24(byte_of(scw, 2 * (j & 1)), dl) + __mul24(byte_of(scw, 2 * (j & 1) + 1), dh);
        }
        const uint32_t mnw = k < 2 ? mn_lo : mn_hi;
        S = sumi;
        P = __mul24(byte_of(mnw, 2 * (k & 1)), bs_lo) + __mul24(byte_of(mnw, 2 * (k & 1) + 1), bs_hi);
        D = r.yd * half_bits_to_f32(hd.x & 0xffffu);
        DM = -r.yd * half_bits_to_f32(hd.x >> 16);
        if (Q5) {
            // the four min products summed exactly, on every lane of the group
            int32_t pm = l < 4 ? P : 0;
            pm += __shfl_xor(pm, 1, 64);
            pm += __shfl_xor(pm, 2, 64);
            P = __shfl(pm, tid & ~7, 64);
        }
        if (DBG) {
            int32_t sS = sumi, sM = l < 4 ? P : 0;
            if (Q5) sM = l == 0 ? P : 0;
            sS += __shfl_xor(sS, 1, 64); sS += __shfl_xor(sS, 2, 64); sS += __shfl_xor(sS, 4, 64);
            sM += __shfl_xor(sM, 1, 64); sM += __shfl_xor(sM, 2, 64); sM += __shfl_xor(sM, 4, 64);
            if (l == 0) { dbgS[rb + (uint32_t)b] = sS; dbgM[rb + (uint32_t)b] = sM; }
        }
    };

    float acc[NMAT], accm[NMAT], summs[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) { acc[m] = 0.0f; accm[m] = 0.0f; summs[m] = 0.0f; }
    // the reference's per-block fp32 step
    auto step = [&](int m, int32_t S, int32_t P, float D, float DM) {
        acc[m] = __builtin_fmaf(D, (float)S, acc[m]);
        if (Q5) {
            const float tm = DM * (float)P;
            summs[m] = summs[m] + tm;
        } else if (l < 4) {
            accm[m] = __builtin_fmaf(DM, (float)P, accm[m]);
        }
    };

    if (NB > 0) {
        // every load of this group's blocks first, then the integer work
        Raw raw[NH];
        if constexpr (PRO == 2) {
            // the attention output is merged here: wave v takes block v of
            // the vector (head v / hb, its dims 256 (v mod hb) + 4L .. +3 on
            // lane L), issuing every chunk's partial (m, l) and o loads and
            // then its weight loads before anything waits; the merge is
            // attn_merge_kernel's arithmetic in its order (max of the chunk
            // maxima, f_g = exp(m_g - M) for chunks with weight, the wave-sum
            // of l_g f_g, o = sum_g o_g f_g from g = 0, o / L), so the vector,
            // its Q8_K (wave v: block v into LDS) and the outputs are the
            // separate merge + GEMV's bits
            const int lane = tid & 63, v = tid >> 6;
            const int G = mg.G, hb = mg.hb;
            const int h = hb == 1 ? v : v >> 1, half = v - h * hb;
            const int RS = 256 * hb + 2;   // partial row stride (floats)
            const float* ph = mg.part + (size_t)h * G * RS;
            const float2 ml = *reinterpret_cast<const float2*>(ph + (size_t)min(lane, G - 1) * RS + 256 * hb);
            float2 oa[kMergeMaxG], ob[kMergeMaxG];
#pragma unroll
            for (int u = 0; u < kMergeMaxG; u++) {
                const float* pr = ph + (size_t)min(u, G - 1) * RS + 256 * half + 4 * lane;
                oa[u] = *reinterpret_cast<const float2*>(pr);
                ob[u] = *reinterpret_cast<const float2*>(pr + 2);
            }
#pragma unroll
            for (int i = 0; i < NH; i++) load_w(min(grp * NH + i, nb - 1), raw[i]);
            __builtin_amdgcn_sched_barrier(0);   // every load issued before the merge waits
            const float mgv = lane < G ? ml.x : -INFINITY;
            const float lgv = lane < G ? ml.y : 0.0f;
            const float M = wave_max(mgv);
            const float f = lane < G && lgv > 0.0f ? expf(mgv - M) : 0.0f;
            const float L = wave_sum(lane < G ? 0.0f + lgv * f : 0.0f);
            float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            // chunk 0 always counts (G >= 1) and the chunks past G are
            // selected away rather than skipped: under a branch the compiler
            // moved chunk 0's loads into it and waited there for every load
            // issued before (the weights)
#pragma unroll
            for (int u = 0; u < kMergeMaxG; u++) {
                const float fu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), u));
                const bool on = u == 0 || u < G;
                o[0] = on ? __builtin_fmaf(oa[u].x, fu, o[0]) : o[0];
                o[1] = on ? __builtin_fmaf(oa[u].y, fu, o[1]) : o[1];
                o[2] = on ? __builtin_fmaf(ob[u].x, fu, o[2]) : o[2];
                o[3] = on ? __builtin_fmaf(ob[u].y, fu, o[3]) : o[3];
            }
            float r[4];
#pragma unroll
            for (int c = 0; c < 4; c++) r[c] = L > 0.0f ? o[c] / L : 0.0f;
            extern __shared__ __align__(16) float pbuf[];
            uint8_t* q8l = reinterpret_cast<uint8_t*>(pbuf);
            quantize_block_wave(r, lane, q8l, NB, v);
            if (bid == 0) {
                if (mg.out) reinterpret_cast<float4*>(mg.out)[tid] = make_float4(r[0], r[1], r[2], r[3]);
                if (mg.q8) quantize_block_wave(r, lane, mg.q8, NB, v);
            }
            lds_sync();
            const uint8_t* a_qs_l = q8l + 32 * l;
            const uint8_t* a_bs_l = q8l + q8k_bsums_off(NB) + 8 * k;
            const float* a_d_l = reinterpret_cast<const float*>(q8l + q8k_d_off(NB));
#pragma unroll
            for (int i = 0; i < NH; i++) {
                const int b = grp * NH + i;
                if (b < nb) {
                    raw[i].a0 = *reinterpret_cast<const uint4*>(a_qs_l + b * 256);
                    raw[i].a1 = *reinterpret_cast<const uint4*>(a_qs_l + b * 256 + 16);
                    raw[i].bsw = *reinterpret_cast<const uint2*>(a_bs_l + b * 32);
                    raw[i].yd = a_d_l[b];
                }
            }
        } else if constexpr (PRO == 1) {
            // the activations are produced here: residual step, norm and Q8_K
            // by the whole workgroup (one float4 of each vector per thread,
            // wave w quantizes block w into LDS; workgroup 0 also stores
            // x_out, xb2 and q8), then read from LDS.  The step's small loads
            // go first, the weight loads behind them, so the norm's arithmetic
            // waits only for the former.  Workgroups past the K-quant rows
            // take the Q6_K tensor (st.w6) on the fp32 normed vector.
            constexpr int rpw = WG / GL;
            const int qk_wgs = (dtot + rpw - 1) / rpw;
            const bool vwg = st.w6 != nullptr && bid >= qk_wgs;
            Res4 r4;
            residual4_load(ra, r4, 0);
            if (!vwg) {
                // every group loads NH blocks (past the row's end: its last
                // block again, not used), so the number of loads behind the
                // step's own is fixed and the norm waits only for the latter
#pragma unroll
                for (int i = 0; i < NH; i++) load_w(min(grp * NH + i, nb - 1), raw[i]);
            }
            extern __shared__ __align__(16) float pbuf[];   // NB*256 floats, the Q8_K blocks, [Q6_K: run sums]
            __shared__ float red[2][16];
            uint8_t* q8l = reinterpret_cast<uint8_t*>(pbuf + NB * 256);
            if (vwg) {
                q6k_prologue_rows<NB, WG, KS6>(st, bid - qk_wgs, ra, r4, pbuf, red);
                return;
            }
            float qv[4], nv[4];
            residual4_finish(ra, r4, red, bid == 0, 0, qv, nv);
            quantize_block_wave(qv, tid & 63, q8l, NB, tid >> 6);
            if (bid == 0 && ra.q8) quantize_block_wave(qv, tid & 63, ra.q8, NB, tid >> 6);
            lds_sync();
            const uint8_t* a_qs_l = q8l + 32 * l;
            const uint8_t* a_bs_l = q8l + q8k_bsums_off(NB) + 8 * k;
            const float* a_d_l = reinterpret_cast<const float*>(q8l + q8k_d_off(NB));
#pragma unroll
            for (int i = 0; i < NH; i++) {
                const int b = grp * NH + i;
                if (b < nb) {
                    raw[i].a0 = *reinterpret_cast<const uint4*>(a_qs_l + b * 256);
                    raw[i].a1 = *reinterpret_cast<const uint4*>(a_qs_l + b * 256 + 16);
                    raw[i].bsw = *reinterpret_cast<const uint2*>(a_bs_l + b * 32);
                    raw[i].yd = a_d_l[b];
                }
            }
        } else if constexpr (QIN) {
            // the inputs, then the weight block, then the wave quantizes the
            // 256 inputs into LDS (workgroup 0 also stores them) while the
            // weights are in flight (the load counter retires in order: the
            // quantize waits only for what was issued before the weights)
            float4 f;
            if constexpr (!XL) f = xload(tid);
            load_w(0, raw[0]);
            if constexpr (XL) f = xload(tid);
            const float v[4] = {f.x, f.y, f.z, f.w};
            quantize_block_wave(v, tid, q8s, 1, 0);
            if (bid == 0 && q8_store) quantize_block_wave(v, tid, q8_store, 1, 0);
            __syncthreads();
            raw[0].a0 = *reinterpret_cast<const uint4*>(q8s + 32 * l);
            raw[0].a1 = *reinterpret_cast<const uint4*>(q8s + 32 * l + 16);
            raw[0].bsw = *reinterpret_cast<const uint2*>(q8s + q8k_bsums_off(1) + 8 * k);
            raw[0].yd = reinterpret_cast<const float*>(q8s + q8k_d_off(1))[0];
        } else {
#pragma unroll
            for (int i = 0; i < NH; i++) load(min(grp * NH + i, nb - 1), raw[i]);
        }
        int32_t S[NMAT][NH], P[NMAT][NH];
        float D[NMAT][NH], DM[NMAT][NH];
#pragma unroll
        for (int i = 0; i < NH; i++) {
            const int b = grp * NH + i;
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                S[m][i] = 0; P[m][i] = 0; D[m][i] = 0.0f; DM[m][i] = 0.0f;
                if (b < nb) block(m, b, raw[i], S[m][i], P[m][i], D[m][i], DM[m][i]);
            }
        }
        if (DBG) return;
        if constexpr (LG && SPLIT > 1 && NB > 0) {
            // a row's SPLIT groups lie in one wave (GL divides 64), whose LDS
            // operations complete in order: no barrier between the writes
            // and group 0's reads, which run the fp32 steps in block order
            constexpr int RW = WG / GL;
            static_assert(64 % GL == 0, "a row's lane groups must share a wave");
            __shared__ uint4 gth[RW][NMAT][NB][8];
            const int rw = tid / GL;
#pragma unroll
            for (int i = 0; i < NH; i++) {
                const int b = grp * NH + i;
                if (b < NB) {
#pragma unroll
                    for (int m = 0; m < NMAT; m++)
                        gth[rw][m][b][l] = make_uint4((uint32_t)S[m][i], (uint32_t)P[m][i], __float_as_uint(D[m][i]),
                                                      __float_as_uint(DM[m][i]));
                }
            }
            if (grp == 0) {
#pragma unroll
                for (int b = 0; b < NB; b++) {
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        const uint4 e = gth[rw][m][b][l];
                        step(m, (int32_t)e.x, (int32_t)e.y, __uint_as_float(e.z), __uint_as_float(e.w));
                    }
                }
            }
        } else {
#pragma unroll
        for (int gs = 0; gs < SPLIT; gs++) {
#pragma unroll
            for (int i = 0; i < NH; i++) {
                if (gs * NH + i < nb) {
#pragma unroll
                    for (int m = 0; m < NMAT; m++) {
                        int32_t So = S[m][i], Po = P[m][i];
                        float Do = D[m][i], DMo = DM[m][i];
                        if (gs > 0) {   // group gs's values, seen from group 0 (lane ^ 8*gs)
                            So = __shfl_xor(So, 8 * gs, 64);
                            Po = __shfl_xor(Po, 8 * gs, 64);
                            Do = __shfl_xor(Do, 8 * gs, 64);
                            DMo = __shfl_xor(DMo, 8 * gs, 64);
                        }
                        step(m, So, Po, Do, DMo);
                    }
                }
            }
        }
        }
    } else {
        for (int b = 0; b < nb; b++) {
            Raw r;
            load(b, r);
#pragma unroll
            for (int m = 0; m < NMAT; m++) {
                int32_t S, P;
                float D, DM;
                block(m, b, r, S, P, D, DM);
                if (!DBG) step(m, S, P, D, DM);
            }
        }
        if (DBG) return;
    }
    float r[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const float t1 = acc[m] + __shfl_xor(acc[m], 4, 64);
        const float t2 = t1 + __shfl_xor(t1, 2, 64);
        const float h = t2 + __shfl_xor(t2, 1, 64);
        if (Q5) {
            r[m] = h + summs[m];
        } else {
            const float v1 = accm[m] + __shfl_xor(accm[m], 2, 64);
            const float hm = v1 + __shfl_xor(v1, 1, 64);
            r[m] = h + hm;
        }
    }
    if (l == 0 && grp == 0 && row_ < dtot) {
        if (NMAT == 2) put(outp, rl, gelu_ref(r[0]) * r[NMAT - 1]);
        else put(outp, rl, aux ? gelu_ref(r[0]) * aux_v : r[0]);
    }
}

template <bool Q5, int NMAT, bool DBG, int NB, int SPLIT, bool QIN, int WG = 64, int PRO = 0, bool LG = false,
          int KS6 = SPLIT>
__global__ __launch_bounds__(WG) void gemv_q45_rows_kernel(const uint8_t* __restrict__ w0,
                                                           const uint8_t* __restrict__ w1,
                                                           const uint8_t* q8, float* __restrict__ out,
                                                           int nb_rt, int d, int32_t* __restrict__ dbgS,
                                                           int32_t* __restrict__ dbgM, const float* __restrict__ xin,
                                                           uint8_t* __restrict__ q8_store,
                                                           const float* __restrict__ aux, const ResidualArgs ra,
                                                           const Stack2 st, const MergeArgs mg) {
    __shared__ __align__(16) uint8_t q8s[QIN ? 292 : 16];
    q45_rows_body<Q5, NMAT, DBG, NB, SPLIT, QIN, WG, PRO, LG, KS6, false>(
        w0, w1, q8, out, nb_rt, d, dbgS, dbgM, q8_store, aux, ra, st, mg, blockIdx.x, threadIdx.x, q8s,
        [&](int t) { return reinterpret_cast<const float4*>(xin)[t]; },
        [](float* o, int row, float v) { o[row] = v; });
}

// ------------------------------------------------------------------------
// The PLE gate and projection of a decode layer in one launch
// (main.c:1982-1994)
// ------------------------------------------------------------------------
// Workgroups [0, P) are g4_mm_residual_q8's PLE-gate workgroups (the
// residual step of the FFN output, Q8_K of x', gelu(gate . q8) * ple: the
// same bits), each storing its values as (value, sequence) pairs, one 64-bit
// device-scope store per value.  Workgroups [P, P + C) run the projection,
// one wave per 8 rows as the single-block-input GEMV does (mm() quantizing
// the 256 gate values: the same bits); each wave issues its weight block and
// then polls the pairs until all 256 carry this call's sequence number.  A
// pair is written and read whole, so no flag, fence or store
// acknowledgement is waited for; the sequence number (*seq, which the caller
// changes between calls on one buffer) keeps an earlier call's values from
// counting.  The gate workgroups have the lowest ids and are dispatched
// first; a poll gives up after kPleSpins rounds and sets the error word.
constexpr int kPleNB = 10;                 // n / 256: one wave per Q8_K block
constexpr int kPleGateRows = 64 * kPleNB / 32;   // gate rows per workgroup (32 lanes a row)
constexpr int kPleProjRows = 8 * kPleNB;   // projection rows per workgroup (8 a wave)
constexpr uint32_t kPleSpins = 1u << 20;

__host__ __device__ inline size_t ple_pair_words(int pd) { return ((size_t)pd + 1) & ~(size_t)1; }

template <bool Q5G, bool Q5P>
__global__ __launch_bounds__(64 * kPleNB) void ple_fused_kernel(const uint8_t* __restrict__ wg,
                                                              const uint8_t* __restrict__ wp, float* __restrict__ y,
                                                              int pd, int dp, const float* __restrict__ mul,
                                                              const ResidualArgs ra, unsigned long long* pairs,
                                                              const uint32_t* seq) {
    const int P = (pd + kPleGateRows - 1) / kPleGateRows;
    const uint32_t sq = *seq;
    if ((int)blockIdx.x < P) {
        q45_rows_body<Q5G, 1, false, kPleNB, 4, false, 64 * kPleNB, 1, true, 4, false>(
            wg, nullptr, nullptr, nullptr, kPleNB, pd, nullptr, nullptr, nullptr, mul, ra, Stack2{}, MergeArgs{},
            blockIdx.x, threadIdx.x, nullptr, [](int) { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); },
            [&](float*, int row, float v) {
                __hip_atomic_store(pairs + row, ((unsigned long long)sq << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            });
        return;
    }
    __shared__ __align__(16) uint8_t q8s[kPleNB][292];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint32_t* err = reinterpret_cast<uint32_t*>(pairs + ple_pair_words(pd));
    q45_rows_body<Q5P, 1, false, 1, 1, true, 64, 0, false, 1, true>(
        wp, nullptr, nullptr, y, 1, dp, nullptr, nullptr, nullptr, nullptr, ResidualArgs{}, Stack2{}, MergeArgs{},
        ((int)blockIdx.x - P) * kPleNB + wave, lane, q8s[wave],
        [&](int t) {
            // wave 0 polls (lane t: values 4t .. 4t+3, the float4 the
            // single-block path quantizes; pd = 256, checked by the launcher)
            // and hands the values to the other waves through LDS
            __shared__ __align__(16) float gv[256];
            if (wave == 0) {
                unsigned long long a[4];
                for (uint32_t spins = 0;; spins++) {
                    bool ok = true;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        a[j] = __hip_atomic_load(pairs + 4 * t + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        ok = ok && (uint32_t)(a[j] >> 32) == sq;
                    }
                    if (__all(ok)) break;
                    if (spins >= kPleSpins) {
                        if (t == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                reinterpret_cast<float4*>(gv)[t] = make_float4(__uint_as_float((uint32_t)a[0]), __uint_as_float((uint32_t)a[1]),
                                                              __uint_as_float((uint32_t)a[2]), __uint_as_float((uint32_t)a[3]));
            }
            lds_sync();
            return reinterpret_cast<const float4*>(gv)[t];
        },
        [](float* o, int row, float v) { o[row] = v; });
}

// ------------------------------------------------------------------------
// Q4_K / Q5_K x Q8_K, streaming form (rows of 8, 10 or 16 blocks)
// ------------------------------------------------------------------------
// One wave per workgroup; an 8-lane group owns one row of one matrix and
// runs all NB blocks of it in order, so no lane shuffles are needed between
// blocks.  With two matrices (gate|up) lanes 0..31 take four gate rows and
// lanes 32..63 the same four up rows; with one matrix the wave has eight
// rows.  The wave issues, in this order, its loads of the Q8_K vector
// (staged in LDS: every group needs the whole vector) and then, per block,
// each lane's 16 weight bytes and its row's 16-byte header (the 8 lanes of a
// group read the same header: one request), so the weight stream is in
// flight before anything waits.  Per block the lane's integer sums are
// those of gemv_q45_rows_kernel, formed with fewer instructions: each pair
// of nibble dots (dl, dh) is packed as two int16 (|dl|, |dh| <= 4*31*127)
// and multiplied by its two sub-block scales in one v_dot2, and the min
// lane's product m_a*(bs0+bs1) + m_b*(bs2+bs3) is two v_dot2 over the raw
// int16 bsums.  The fp32 steps and the horizontal adds are the reference's
// (main.c:476-529, 531-593), so outputs are bit-identical to the rows
// kernel.
typedef short s2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ int dot2_i16(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2_t, a), __builtin_bit_cast(s2_t, b), c, false);
}

// PRO: a workgroup of NB such waves (64 NB threads, n = 256 NB) whose Q8_K
// vector is made by the workgroup itself: the residual step, norm and Q8_K
// of ResidualArgs with one float4 of each vector per thread and block w
// quantized by wave w (its loads issued first, then every wave's header and
// weight loads, so the norm's arithmetic runs while the weights stream in),
// into LDS; workgroup 0 also stores the residual stream, xb2 and the Q8_K
// when asked.
constexpr int kStreamProLead = 2;   // weight blocks per lane issued before the prologue

template <bool Q5, int NB, int NMAT, bool PRO = false>
__global__ __launch_bounds__(PRO ? 64 * NB : 64) void gemv_q45_stream_kernel(const uint8_t* __restrict__ w0,
                                                                         const uint8_t* __restrict__ w1,
                                                                         const uint8_t* __restrict__ q8,
                                                                         float* __restrict__ out, int d,
                                                                         const float* __restrict__ aux,
                                                                         const ResidualArgs ra) {
    constexpr int RPW = 8 / NMAT;                 // rows per wave
    constexpr int NWV = PRO ? NB : 1;             // waves per workgroup
    constexpr int Q8B = NB * 292;                 // device Q8_K bytes
    constexpr int Q8C = Q8B / 16, Q8T = (Q8B - Q8C * 16) / 4;
    constexpr int QPL = PRO ? 0 : (Q8C + 63) / 64;
    __shared__ __align__(16) uint8_t sq[Q8B + 16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l = lane & 7, k = l & 3;
    const int grp = (lane >> 3) & (RPW - 1);
    const int m = NMAT == 2 ? lane >> 5 : 0;
    const int r0 = (blockIdx.x * NWV + wv) * RPW;
    const int row = min(r0 + grp, d - 1);
    const uint32_t nblk = (uint32_t)d * NB;
    const uint32_t hdr_off = (Q5 ? 160u : 128u) * nblk, qh_off = 128u * nblk;   // q4k_planes / q5k_planes

    [[maybe_unused]] Res4 r4;
    if constexpr (PRO) residual4_load(ra, r4, 0);
    // the Q8_K vector is staged in LDS (the same for every wave)
    uint4 qv[QPL > 0 ? QPL : 1];
    uint32_t tv = 0u;
#pragma unroll
    for (int j = 0; j < QPL; j++) {
        const int c = lane + 64 * j;
        qv[j] = make_uint4(0u, 0u, 0u, 0u);
        if (c < Q8C) qv[j] = reinterpret_cast<const uint4*>(q8)[c];
    }
    if (!PRO && lane < Q8T) tv = reinterpret_cast<const uint32_t*>(q8 + Q8C * 16)[lane];
    // each lane loads its row's block headers with its weights (the 8 lanes
    // of a group read the same 16 bytes: one request).  Staged through LDS
    // instead, the header loads under a lane condition compiled to a branch
    // whose result copy waited for every load before it (vmcnt(0)), so the
    // weight loads started only after the staging loads had returned
    const uint8_t* const wm = m ? w1 : w0;
    const uint32_t rb = (uint32_t)row * NB;
    uint4 wq[NB], hd[NB];
    uint32_t qh[NB];
    auto load_blocks = [&](int b0, int b1) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b < b0 || b >= b1) continue;
            wq[b] = *reinterpret_cast<const uint4*>(wm + (rb + b) * 128u + 16 * l);
            hd[b] = *reinterpret_cast<const uint4*>(wm + hdr_off + (rb + b) * 16u);
            qh[b] = Q5 ? *reinterpret_cast<const uint32_t*>(wm + qh_off + (rb + b) * 32u + 4 * l) : 0u;
        }
    };
    // With the prologue only the first kStreamProLead blocks are issued
    // before it and the rest after it.  The whole matrix in flight at once
    // (every workgroup's loads issued within the first microsecond) holds the
    // prologue's own small loads behind it in the memory queues: gate|up
    // with the residual step (2 x 10240 x 2560, cold caches) has its
    // prologue done 6.1 us after a workgroup's entry with all ten blocks
    // issued first, 3.9 us with two; the launch takes 11.5 against 13.5 us.
    constexpr int NB0 = PRO ? (kStreamProLead < NB ? kStreamProLead : NB) : NB;
    load_blocks(0, NB0);
    __builtin_amdgcn_sched_barrier(0);   // all loads issued before the LDS stores wait for the first ones
    if constexpr (PRO) {
        // one float4 of each vector per thread, wave w quantizes block w
        __shared__ float red[2][16];
        float qv[4], nv[4];
        residual4_finish(ra, r4, red, blockIdx.x == 0, 0, qv, nv);
        quantize_block_wave(qv, lane, sq, NB, wv);
        if (blockIdx.x == 0 && ra.q8) quantize_block_wave(qv, lane, ra.q8, NB, wv);
    } else {
#pragma unroll
        for (int j = 0; j < QPL; j++) {
            const int c = lane + 64 * j;
            if (c < Q8C) reinterpret_cast<uint4*>(sq)[c] = qv[j];
        }
        if (lane < Q8T) reinterpret_cast<uint32_t*>(sq + Q8C * 16)[lane] = tv;
    }
    // (with the prologue an LDS-only barrier: __syncthreads() would also wait
    // for every weight load, so no block's dot could start before the last
    // one had landed)
    if constexpr (PRO) lds_sync();
    else __syncthreads();
    load_blocks(NB0, NB);

    // byte selectors of the two mins (m_2k, m_2k+1 of min lane k), as int16 pairs
    const uint32_t selA = (k & 1) ? 0x0c020c02u : 0x0c000c00u;
    const uint32_t selB = (k & 1) ? 0x0c030c03u : 0x0c010c01u;
    // min lanes 0, 1 use mins 0..3, lanes 2, 3 mins 4..7; a mask rather than
    // a conditional, which the compiler turns into a branch per block and
    // then hoists every block's LDS reads above it (198 VGPRs instead of 74)
    const uint32_t kmask = k < 2 ? 0xffffffffu : 0u;
    float acc = 0.0f, accm = 0.0f, summs = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const uint8_t* a_qs = sq + 32 * l + b * 256;
        const uint4 a0 = *reinterpret_cast<const uint4*>(a_qs);
        const uint4 a1 = *reinterpret_cast<const uint4*>(a_qs + 16);
        const uint2 bsw = *reinterpret_cast<const uint2*>(sq + q8k_bsums_off(NB) + b * 32 + 8 * k);
        const float yd = reinterpret_cast<const float*>(sq + q8k_d_off(NB))[b];
        // the 6-bit scales (sub-blocks 0..3, 4..7) and this min lane's two mins
        const uint32_t sc_lo = hd[b].y & 0x3f3f3f3fu;
        const uint32_t sc_hi = (hd[b].w & 0x0f0f0f0fu) | (((hd[b].y >> 6) & 0x03030303u) << 4);
        const uint32_t mn_lo = hd[b].z & 0x3f3f3f3fu;
        const uint32_t mn_hi = ((hd[b].w >> 4) & 0x0f0f0f0fu) | (((hd[b].z >> 6) & 0x03030303u) << 4);
        const uint32_t mnw = (mn_lo & kmask) | (mn_hi & ~kmask);
        int32_t sumi = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t qw = word_of(wq[b], j);
            uint32_t lo = qw & 0x0f0f0f0fu, hi = (qw >> 4) & 0x0f0f0f0fu;
            if (Q5) {
                lo |= ((qh[b] >> (2 * j)) & 0x01010101u) << 4;
                hi |= ((qh[b] >> (2 * j + 1)) & 0x01010101u) << 4;
            }
            const int dl = __builtin_amdgcn_sdot4((int)lo, (int)word_of(a0, j), 0, false);
            const int dh = __builtin_amdgcn_sdot4((int)hi, (int)word_of(a1, j), 0, false);
            const uint32_t pk = __builtin_amdgcn_perm((uint32_t)dh, (uint32_t)dl, 0x05040100u);
            const uint32_t scp = __builtin_amdgcn_perm(0u, j < 2 ? sc_lo : sc_hi, (j & 1) ? 0x0c030c02u : 0x0c010c00u);
            sumi = dot2_i16(pk, scp, sumi);
        }
        int32_t P = dot2_i16(bsw.x, __builtin_amdgcn_perm(0u, mnw, selA),
                             dot2_i16(bsw.y, __builtin_amdgcn_perm(0u, mnw, selB), 0));
        const float D = yd * half_bits_to_f32(hd[b].x & 0xffffu);
        const float DM = -yd * half_bits_to_f32(hd[b].x >> 16);
        if (Q5) {
            // the four min products summed exactly, on every lane of the group
            int32_t pm = l < 4 ? P : 0;
            pm += __shfl_xor(pm, 1, 64);
            pm += __shfl_xor(pm, 2, 64);
            P = __shfl(pm, lane & ~7, 64);
        }
        acc = __builtin_fmaf(D, (float)sumi, acc);
        if (Q5) {
            const float tm = DM * (float)P;
            summs = summs + tm;
        } else if (l < 4) {
            accm = __builtin_fmaf(DM, (float)P, accm);
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
    const int ro = r0 + grp;
    if (NMAT == 2) {
        const float up = __shfl_xor(r, 32, 64);
        if (l == 0 && m == 0 && ro < d) out[ro] = gelu_ref(r) * up;
    } else if (l == 0 && ro < d) {
        out[ro] = aux ? gelu_ref(r) * aux[ro] : r;
    }
}

// ------------------------------------------------------------------------
// Q6_K x fp32 (mm_quant_rows semantics), one row slice per 8-lane group
// ------------------------------------------------------------------------
// A 256-thread workgroup stages x in LDS once and sweeps row groups of
// 32/KS rows; each row is split over KS groups (ks takes blocks ks, ks+KS,
// ...) whose partial sums are added in LDS.  Lane L = 4h+u of a group owns
// the 32 weights 128h + 32k + 8u + e (k < 4, e < 8) of each block: their
// 6-bit codes q are assembled four at a time into bytes, converted to float
// and multiplied by x; a run of 8 contributes sum x*q - 32 * sum x (the run
// sums of x are computed once per workgroup) scaled once by d*sc (the
// reference scales every weight, (d*sc)*(q-32); results agree to fp32
// tolerance, not bit for bit).
// The weights stream in batches of QB blocks per lane through two register
// sets: batch j + 1 (the next blocks of the row, or the first of the next
// row group) is in flight while batch j is multiplied, and every load is
// issued unconditionally on clamped indices, so the waits count exactly and
// never drain the next batch.  The first two batches are issued before x is
// staged.  AM: also the first-index maximum of the outputs (as stored, after
// the soft-cap) over this workgroup's rows as an argmax key in part[block].
constexpr int kQ6XsBlk = 256 + 8;   // LDS floats per block of x in gemv_q6k_rows_kernel

template <int KS, bool SOFTCAP, bool AM = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void gemv_q6k_rows_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                            float* __restrict__ out, int nb, int d, float cap,
                                                            unsigned long long* __restrict__ part_am) {
    // LDS: x (n floats, 4 floats of padding after every 128: a block's two
    // halves, read by lanes h = 0 and 1 of a group at once, then fall in
    // different banks), the sums of its runs of 8 (n/8 floats), [32] partials
    extern __shared__ __align__(16) float xs[];
    __shared__ unsigned long long red[4];
    constexpr int RPW = 32 / KS;
    constexpr int QB = 5;                  // blocks per load batch
    const int tid = threadIdx.x, L = tid & 7, g = tid >> 3, h = L >> 2, u = L & 3;
    const int rr = g % RPW, ks = g / RPW;
    const size_t nblk = (size_t)d * nb;
    const Q6KPlanes P = q6k_planes(nblk);
    float* x8 = xs + nb * kQ6XsBlk;
    float* part = x8 + nb * 32;
    const float inv = SOFTCAP ? 1.0f / cap : 0.0f;
    const int ngroups = (d + RPW - 1) / RPW;
    const int nbt = ((nb + KS - 1) / KS + QB - 1) / QB;   // batches per row slice
    const int nit = blockIdx.x < ngroups ? (ngroups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int nsteps = nit * nbt;

    struct Batch {
        uint4 ql[QB];
        uint2 qh[QB], sc[QB];
        uint32_t dv[QB];
    };
    // step j: batch j % nbt of this workgroup's row group j / nbt (past the
    // last step: the last one again; blocks past the row: its last block)
    auto load = [&](int j, Batch& bt) {
        j = min(j, nsteps - 1);
        const int it = j / nbt, b0 = ks + (j - it * nbt) * QB * KS;
        const int row = min(((int)blockIdx.x + it * (int)gridDim.x) * RPW + rr, d - 1);
#pragma unroll
        for (int i = 0; i < QB; i++) {
            const size_t blk = (size_t)row * nb + min(b0 + i * KS, nb - 1);
            bt.ql[i] = *reinterpret_cast<const uint4*>(w + P.ql + blk * 128 + 16 * L);
            bt.qh[i] = *reinterpret_cast<const uint2*>(w + P.qh + blk * 64 + 8 * L);
            bt.sc[i] = *reinterpret_cast<const uint2*>(w + P.sc + blk * 16 + 8 * h);
            bt.dv[i] = *reinterpret_cast<const uint16_t*>(w + P.d + blk * 2);
        }
    };
    // x (kQ6Xpt float4 per thread, the rest in a loop) and then the first
    // two batches are in flight before anything waits: a load-then-store
    // loop would wait for every earlier load on each of its iterations
    constexpr int kQ6Xpt = 4;
    const int n4 = nb * 64;                // float4 of x; a multiple of 64, so a wave's lanes agree
    float4 xv[kQ6Xpt];
#pragma unroll
    for (int j = 0; j < kQ6Xpt; j++) {
        const int i = tid + 256 * j;
        xv[j] = i < n4 ? reinterpret_cast<const float4*>(x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    Batch ba, bb;
    if (nsteps > 0) {
        load(0, ba);
        load(1, bb);
    }
    // i covers elements 4i..4i+3; pairs of float4 make one run of 8
    auto stage = [&](int i, const float4& v) {
        reinterpret_cast<float4*>(xs)[i + (i >> 5)] = v;
        const float s4 = (v.x + v.y) + (v.z + v.w);
        const float o4 = __shfl_xor(s4, 1, 64);
        if ((i & 1) == 0) x8[i >> 1] = s4 + o4;
    };
#pragma unroll
    for (int j = 0; j < kQ6Xpt; j++) {
        const int i = tid + 256 * j;
        if (i < n4) stage(i, xv[j]);
    }
    for (int i = tid + 256 * kQ6Xpt; i < n4; i += 256) stage(i, reinterpret_cast<const float4*>(x)[i]);
    if (KS > 1 || n4 > 256 * kQ6Xpt) {
        __syncthreads();
    } else {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // LDS only: the batches stay in flight
    }

    unsigned long long best = 0;           // argmax key of this thread's rows
    float acc = 0.0f;
    auto compute = [&](const Batch& bt, int j) {
        const int it = j / nbt, jb = j - it * nbt, b0 = ks + jb * QB * KS;
        const int rg = (int)blockIdx.x + it * (int)gridDim.x;
        const int row = rg * RPW + rr;
        if (jb == 0) acc = 0.0f;
#pragma unroll
        for (int i = 0; i < QB; i++) {
            const int b = b0 + i * KS;
            if (b < nb) {
                const uint4 ql = bt.ql[i];
                const uint2 qh = bt.qh[i], sc = bt.sc[i];
                const float df = half_bits_to_f32(bt.dv[i]);
                const float* xb = xs + b * kQ6XsBlk + (128 + 4) * h + 8 * u;
                const float* sb8 = x8 + b * 32 + 16 * h + u;
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const uint32_t qa = (kk & 1) ? ql.z : ql.x;      // codes e = 0..3
                    const uint32_t qb = (kk & 1) ? ql.w : ql.y;      // codes e = 4..7
                    const uint32_t la = kk < 2 ? (qa & 0x0f0f0f0fu) : ((qa >> 4) & 0x0f0f0f0fu);
                    const uint32_t lb = kk < 2 ? (qb & 0x0f0f0f0fu) : ((qb >> 4) & 0x0f0f0f0fu);
                    const uint32_t ca = la | (((qh.x >> (2 * kk)) & 0x03030303u) << 4);   // q in [0, 63]
                    const uint32_t cb = lb | (((qh.y >> (2 * kk)) & 0x03030303u) << 4);
                    const float4 x0 = *reinterpret_cast<const float4*>(xb + 32 * kk);
                    const float4 x1 = *reinterpret_cast<const float4*>(xb + 32 * kk + 4);
                    // sum_e x_e (q_e - 32) = sum_e x_e q_e - 32 * sum_e x_e
                    float dot = x0.x * (float)(ca & 0xff);
                    dot = __builtin_fmaf(x0.y, (float)((ca >> 8) & 0xff), dot);
                    dot = __builtin_fmaf(x0.z, (float)((ca >> 16) & 0xff), dot);
                    dot = __builtin_fmaf(x0.w, (float)(ca >> 24), dot);
                    dot = __builtin_fmaf(x1.x, (float)(cb & 0xff), dot);
                    dot = __builtin_fmaf(x1.y, (float)((cb >> 8) & 0xff), dot);
                    dot = __builtin_fmaf(x1.z, (float)((cb >> 16) & 0xff), dot);
                    dot = __builtin_fmaf(x1.w, (float)(cb >> 24), dot);
                    dot = __builtin_fmaf(-32.0f, sb8[4 * kk], dot);
                    const int sbi = (u >> 1) + 2 * kk;
                    const int8_t s8 = (int8_t)byte_of(sbi < 4 ? sc.x : sc.y, sbi & 3);
                    acc = __builtin_fmaf(df * (float)s8, dot, acc);
                }
            }
        }
        if (jb != nbt - 1) return;
        // the row slice is done: sum over the group's 8 lanes (and the KS
        // slices), store, and keep the argmax key
        float a = acc;
        a += __shfl_xor(a, 1, 64);
        a += __shfl_xor(a, 2, 64);
        a += __shfl_xor(a, 4, 64);
        if (KS > 1) {
            if (L == 0) part[g] = a;
            __syncthreads();
            if (tid < RPW) {
                float s = 0.0f;
#pragma unroll
                for (int q = 0; q < KS; q++) s += part[q * RPW + tid];
                const int r = rg * RPW + tid;
                if (r < d) {
                    const float v = SOFTCAP ? cap * tanhf(s * inv) : s;
                    out[r] = v;
                    if (AM) {
                        const unsigned long long k = argmax_key(v, r);
                        best = k > best ? k : best;
                    }
                }
            }
            __syncthreads();
        } else if (L == 0 && row < d) {
            const float v = SOFTCAP ? cap * tanhf(a * inv) : a;
            out[row] = v;
            if (AM) {
                const unsigned long long k = argmax_key(v, row);
                best = k > best ? k : best;
            }
        }
    };
    // steps in pairs over the two register sets (loads past the end repeat
    // the last step: no branch separates a load from its use)
    for (int j = 0; j < nsteps; j += 2) {
        compute(ba, j);
        load(j + 2, ba);
        if (j + 1 < nsteps) compute(bb, j + 1);
        load(j + 3, bb);
    }
    if (AM) {
        best = block_max_u64(best, red);
        if (tid == 0) part_am[blockIdx.x] = best;
    }
}

}  // namespace g4

using namespace g4;

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------
// Q6_K x fp32, one K slice per 8-lane group (rows of up to 64 blocks)
// ------------------------------------------------------------------------
// Group g of a workgroup of 8*nb threads owns block g of every row, so the
// 32 elements of x its lanes use (lane L = 4h+u: 128h + 32k + 8u + e, the
// mapping of gemv_q6k_rows_kernel) and their run sums stay in registers:
// no staging of x through LDS and no LDS reads in the loop.  A workgroup
// runs R consecutive rows and issues every weight load of them before it
// waits (42 KB per workgroup at the FFN-down shape, two workgroups per CU;
// a sweep of R = 3..10 there: 5 fastest, 7.6 us against 8.9 us at 10).  Per row the group's partial dot is summed over its 8 lanes, and the
// nb block partials of each row are added once through LDS.  Same
// arithmetic per block as gemv_q6k_rows_kernel; the blocks are summed as a
// tree (fp32 tolerance of the reference's sequential sum).
namespace g4 {

constexpr int kQ6SliceRows = 5;       // 512 workgroups at the FFN-down shape: two per CU
constexpr int kQ6SliceMaxNb = 64;

template <int R>
__global__ __launch_bounds__(8 * kQ6SliceMaxNb) void gemv_q6k_kslice_kernel(const uint8_t* __restrict__ w,
                                                                          const float* __restrict__ x,
                                                                          float* __restrict__ out, int nb, int d) {
    __shared__ float part[R][kQ6SliceMaxNb];
    const int tid = threadIdx.x, L = tid & 7, g = tid >> 3, h = L >> 2, u = L & 3;
    const int r0 = blockIdx.x * R;
    const Q6KPlanes P = q6k_planes((size_t)d * nb);
    // x of this lane first (runs k = 0..3 of 8 elements at g*256 + 128h +
    // 32k + 8u), then every weight load of the R rows, all issued before
    // anything waits: the load counter retires in order, so the run sums
    // wait only for x and row r only for rows 0..r
    float4 xa[4], xb[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4* xp = reinterpret_cast<const float4*>(x + (size_t)g * 256 + 128 * h + 32 * k + 8 * u);
        xa[k] = xp[0];
        xb[k] = xp[1];
    }
    uint4 ql[R];
    uint2 qh[R], sc[R];
    uint32_t dv[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const size_t blk = (size_t)min(r0 + r, d - 1) * nb + g;
        ql[r] = *reinterpret_cast<const uint4*>(w + P.ql + blk * 128 + 16 * L);
        qh[r] = *reinterpret_cast<const uint2*>(w + P.qh + blk * 64 + 8 * L);
        sc[r] = *reinterpret_cast<const uint2*>(w + P.sc + blk * 16 + 8 * h);
        dv[r] = *reinterpret_cast<const uint16_t*>(w + P.d + blk * 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    float s8[4];
#pragma unroll
    for (int k = 0; k < 4; k++) s8[k] = ((xa[k].x + xa[k].y) + (xa[k].z + xa[k].w)) + ((xb[k].x + xb[k].y) + (xb[k].z + xb[k].w));
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float df = half_bits_to_f32(dv[r]);
        float acc = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const uint32_t qa = (kk & 1) ? ql[r].z : ql[r].x;      // codes e = 0..3
            const uint32_t qb = (kk & 1) ? ql[r].w : ql[r].y;      // codes e = 4..7
            const uint32_t la = kk < 2 ? (qa & 0x0f0f0f0fu) : ((qa >> 4) & 0x0f0f0f0fu);
            const uint32_t lb = kk < 2 ? (qb & 0x0f0f0f0fu) : ((qb >> 4) & 0x0f0f0f0fu);
            const uint32_t ca = la | (((qh[r].x >> (2 * kk)) & 0x03030303u) << 4);   // q in [0, 63]
            const uint32_t cb = lb | (((qh[r].y >> (2 * kk)) & 0x03030303u) << 4);
            // sum_e x_e (q_e - 32) = sum_e x_e q_e - 32 * sum_e x_e
            float dot = xa[kk].x * (float)(ca & 0xff);
            dot = __builtin_fmaf(xa[kk].y, (float)((ca >> 8) & 0xff), dot);
            dot = __builtin_fmaf(xa[kk].z, (float)((ca >> 16) & 0xff), dot);
            dot = __builtin_fmaf(xa[kk].w, (float)(ca >> 24), dot);
            dot = __builtin_fmaf(xb[kk].x, (float)(cb & 0xff), dot);
            dot = __builtin_fmaf(xb[kk].y, (float)((cb >> 8) & 0xff), dot);
            dot = __builtin_fmaf(xb[kk].z, (float)((cb >> 16) & 0xff), dot);
            dot = __builtin_fmaf(xb[kk].w, (float)(cb >> 24), dot);
            dot = __builtin_fmaf(-32.0f, s8[kk], dot);
            const int sbi = (u >> 1) + 2 * kk;
            const int8_t s8i = (int8_t)byte_of(sbi < 4 ? sc[r].x : sc[r].y, sbi & 3);
            acc = __builtin_fmaf(df * (float)s8i, dot, acc);
        }
        // the group's 8 lanes (quad xor 1, 2, then the two quads)
        acc += dpp_f<kDppXor1>(acc);
        acc += dpp_f<kDppXor2>(acc);
        acc += dpp_f<kDppHalfMirror>(acc);
        if (L == 0) part[r][g] = acc;
    }
    __syncthreads();
    // row r: 8 lanes add nb/8 block partials each, then the 8 lanes
    for (int t = tid; t < R * 8; t += blockDim.x) {
        const int r = t >> 3, j = t & 7;
        float s = 0.0f;
        for (int b = j; b < nb; b += 8) s += part[r][b];
        s += dpp_f<kDppXor1>(s);
        s += dpp_f<kDppXor2>(s);
        s += dpp_f<kDppHalfMirror>(s);
        if (j == 0 && r0 + r < d) out[r0 + r] = s;
    }
}

// ------------------------------------------------------------------------
// Q6_K x fp32 with x held in registers (the LM head: many rows of NB blocks)
// ------------------------------------------------------------------------
// A workgroup of 8*NB*kXrRpi threads.  Thread t takes row slot r = t/(8 NB)
// of every pass and slot (b, L) = ((t mod 8NB)/8, t mod 8) of every row it
// visits: the 32 weights 128h + 32k + 8u + e of block b (L = 4h+u, the lane
// mapping of gemv_q6k_rows_kernel), so the 32 elements of x it multiplies
// and their four run sums stay in registers for the whole launch (no LDS
// reads of x, which gemv_q6k_rows_kernel pays once per weight).  A pass
// covers kXrRpi rows; eight passes make a batch of 8*kXrRpi rows whose
// block partials (each summed over its 8 lanes) go to LDS; after a barrier
// one thread per row in one wave (a different wave each batch) add each row's NB
// partials, apply the soft-cap, store and (AM) keep the argmax key.  Batches are dealt to the workgroups round
// robin (d a multiple of the batch); each thread keeps kXrPf
// passes of weight loads in flight (past the last pass: the last one again,
// so no load sits under a branch).
// Same per-block arithmetic as gemv_q6k_rows_kernel (fp32 tolerance of the
// reference's sequential sums).
constexpr int kXrRpi = 8, kXrPf = 4, kXrRow = 12;

template <int NB, bool SOFTCAP, bool AM>
__global__ __launch_bounds__(8 * NB * kXrRpi) void gemv_q6k_xreg_kernel(const uint8_t* __restrict__ w,
                                                                       const float* __restrict__ x,
                                                                       float* __restrict__ out, int d, float cap,
                                                                       unsigned long long* __restrict__ part_am) {
    constexpr int NT = 8 * NB * kXrRpi;
    constexpr int BR = 8 * kXrRpi;   // rows per batch
    static_assert(NB <= kXrRow && NT % 64 == 0 && BR <= 64, "a row's partials fit one LDS row; whole waves");
    static_assert(8 % kXrPf == 0, "the step loop covers whole batches (8 passes)");
    __shared__ __align__(16) float part[2][BR][kXrRow];
    __shared__ unsigned long long red[NT / 64];
    const int t = threadIdx.x, r = t / (8 * NB), s = t - r * (8 * NB), b = s >> 3, L = s & 7, h = L >> 2, u = L & 3;
    const int nbatch = d / BR;
    const int mine = (int)blockIdx.x < nbatch ? (nbatch - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int nsteps = 8 * mine;
    unsigned long long best = 0;   // argmax key of this thread's rows
    if (nsteps > 0) {
        const Q6KPlanes P = q6k_planes((size_t)d * NB);
        // x of this thread (runs k = 0..3 of 8 elements at b*256 + 128h + 32k + 8u)
        float4 xa[4], xb[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4* xp = reinterpret_cast<const float4*>(x + b * 256 + 128 * h + 32 * k + 8 * u);
            xa[k] = xp[0];
            xb[k] = xp[1];
        }
        struct Wt {
            uint4 ql;
            uint2 qh, sc;
            uint32_t dv;
        };
        // a pass's first block (uniform) plus this thread's offsets: the rows
        // are whole batches (d a multiple of BR), so no row is clamped
        const uint32_t rb = (uint32_t)(r * NB + b);
        const uint32_t o_ql = rb * 128u + 16u * L, o_qh = rb * 64u + 8u * L, o_sc = rb * 16u + 8u * h, o_d = rb * 2u;
        auto load = [&](int j, Wt& q) {
            j = min(j, nsteps - 1);
            const size_t pb = ((size_t)((int)blockIdx.x + (j >> 3) * (int)gridDim.x) * BR + (j & 7) * kXrRpi) * NB;
            q.ql = *reinterpret_cast<const uint4*>(w + P.ql + pb * 128 + o_ql);
            q.qh = *reinterpret_cast<const uint2*>(w + P.qh + pb * 64 + o_qh);
            q.sc = *reinterpret_cast<const uint2*>(w + P.sc + pb * 16 + o_sc);
            q.dv = *reinterpret_cast<const uint16_t*>(w + P.d + pb * 2 + o_d);
        };
        Wt ring[kXrPf];
#pragma unroll
        for (int p = 0; p < kXrPf; p++) load(p, ring[p]);
        float s8[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            s8[k] = ((xa[k].x + xa[k].y) + (xa[k].z + xa[k].w)) + ((xb[k].x + xb[k].y) + (xb[k].z + xb[k].w));
        const float inv = SOFTCAP ? 1.0f / cap : 0.0f;
        for (int j0 = 0; j0 < nsteps; j0 += kXrPf) {
#pragma unroll
            for (int p = 0; p < kXrPf; p++) {
                const int j = j0 + p;
                const Wt& q = ring[p];
                const float df = half_bits_to_f32(q.dv);
                float acc = 0.0f;
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    const uint32_t qa = (kk & 1) ? q.ql.z : q.ql.x;   // codes e = 0..3
                    const uint32_t qb = (kk & 1) ? q.ql.w : q.ql.y;   // codes e = 4..7
                    const uint32_t la = kk < 2 ? (qa & 0x0f0f0f0fu) : ((qa >> 4) & 0x0f0f0f0fu);
                    const uint32_t lb = kk < 2 ? (qb & 0x0f0f0f0fu) : ((qb >> 4) & 0x0f0f0f0fu);
                    const uint32_t ca = la | (((q.qh.x >> (2 * kk)) & 0x03030303u) << 4);   // q in [0, 63]
                    const uint32_t cb = lb | (((q.qh.y >> (2 * kk)) & 0x03030303u) << 4);
                    // sum_e x_e (q_e - 32) = sum_e x_e q_e - 32 * sum_e x_e
                    float dot = xa[kk].x * (float)(ca & 0xff);
                    dot = __builtin_fmaf(xa[kk].y, (float)((ca >> 8) & 0xff), dot);
                    dot = __builtin_fmaf(xa[kk].z, (float)((ca >> 16) & 0xff), dot);
                    dot = __builtin_fmaf(xa[kk].w, (float)(ca >> 24), dot);
                    dot = __builtin_fmaf(xb[kk].x, (float)(cb & 0xff), dot);
                    dot = __builtin_fmaf(xb[kk].y, (float)((cb >> 8) & 0xff), dot);
                    dot = __builtin_fmaf(xb[kk].z, (float)((cb >> 16) & 0xff), dot);
                    dot = __builtin_fmaf(xb[kk].w, (float)(cb >> 24), dot);
                    dot = __builtin_fmaf(-32.0f, s8[kk], dot);
                    // scale of sub-block (u >> 1) + 2kk: word kk >> 1, byte (u >> 1) + 2 (kk & 1)
                    const int8_t s8i = (int8_t)byte_of(kk < 2 ? q.sc.x : q.sc.y, (u >> 1) + 2 * (kk & 1));
                    acc = __builtin_fmaf(df * (float)s8i, dot, acc);
                }
                // the slot's next pass, into the registers just read (a load
                // into other registers would be copied back across the loop
                // edge, which waits for it)
                load(j + kXrPf, ring[p]);
                // the block's 8 lanes (quad xor 1, 2, then the two quads)
                acc += dpp_f<kDppXor1>(acc);
                acc += dpp_f<kDppXor2>(acc);
                acc += dpp_f<kDppHalfMirror>(acc);
                float(*pb)[kXrRow] = part[(j >> 3) & 1];
                if (L == 0) pb[(j & 7) * kXrRpi + r][b] = acc;
                if ((j & 7) == 7) {
                    // the batch's rows: every partial is in LDS.  Lanes 0..BR-1
                    // of one wave add them, the wave taking turns by batch so
                    // that no wave falls behind the others at the barriers
                    lds_sync();
                    const int tr = t - 64 * ((j >> 3) % (NT / 64));
                    if (tr >= 0 && tr < BR) {
                        const float* pr = pb[tr];
                        float v[NB];
#pragma unroll
                        for (int i = 0; i < NB; i++) v[i] = pr[i];
#pragma unroll
                        for (int m = 1; m < NB; m <<= 1)
#pragma unroll
                            for (int i = 0; i + m < NB; i += 2 * m) v[i] += v[i + m];
                        const int row = ((int)blockIdx.x + (j >> 3) * (int)gridDim.x) * BR + tr;
                        const float o = SOFTCAP ? cap * tanhf(v[0] * inv) : v[0];
                        out[row] = o;
                        if (AM) {
                            const unsigned long long key = argmax_key(o, row);
                            best = key > best ? key : best;
                        }
                    }
                }
            }
        }
    }
    if (AM) {
        best = block_max_u64(best, red);
        if (t == 0) part_am[blockIdx.x] = best;
    }
}

}  // namespace g4

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

template <bool Q5, int NMAT, bool DBG, int NB, int SPLIT, bool QIN = false>
void launch_q45_nb(const void* w0, const void* w1, const void* q8, float* o, int nb, int d, int32_t* S, int32_t* M,
                   const float* xin = nullptr, void* q8_store = nullptr, const float* aux = nullptr) {
    constexpr int rows_per_wg = 8 / SPLIT;
    hipLaunchKernelGGL((gemv_q45_rows_kernel<Q5, NMAT, DBG, NB, SPLIT, QIN>), dim3((d + rows_per_wg - 1) / rows_per_wg),
                       dim3(64), 0, g4_stream(), (const uint8_t*)w0, (const uint8_t*)w1, (const uint8_t*)q8, o, nb, d,
                       S, M, xin, (uint8_t*)q8_store, aux, ResidualArgs{}, Stack2{}, MergeArgs{});
}

// residual step + norm + Q8_K as the prologue of every workgroup (64 NB
// threads: one wave per Q8_K block, each wave 8/SPLIT rows)
template <bool Q5, int NMAT, int NB, int SPLIT, bool LG = false, int KS6 = SPLIT>
void launch_q45_pro_s(const void* w, const void* w2, float* o, int d, const float* aux, const ResidualArgs& ra,
                      const Stack2& st) {
    constexpr int WG = 64 * NB;
    constexpr int rows_per_wg = WG / (8 * SPLIT);
    const int rows = d + st.d;
    // x, Q8_K, and for a Q6_K tensor the run sums of x and the partials
    const size_t lds = (size_t)NB * 256 * 4 + (((size_t)NB * 292 + 15) & ~(size_t)15) + (size_t)NB * 32 * 4 +
                       (size_t)WG / 8 * 4;
    const int r6 = q6_pro_rows(WG, KS6);
    const int wgs = (rows + rows_per_wg - 1) / rows_per_wg + (st.w6 ? (st.d6 + r6 - 1) / r6 : 0);
    hipLaunchKernelGGL((gemv_q45_rows_kernel<Q5, NMAT, false, NB, SPLIT, false, WG, 1, LG, KS6>),
                       dim3(wgs), dim3(WG), lds, g4_stream(), (const uint8_t*)w,
                       (const uint8_t*)w2, nullptr, o, NB, d, nullptr, nullptr, nullptr, nullptr, aux, ra, st,
                       MergeArgs{});
}

// attention merge + Q8_K as the prologue of every workgroup (64 NB threads:
// wave v merges block v of the vector), then the GEMV with 32 lanes per row
// (the lane groups' block values gathered through LDS)
template <bool Q5, int NB>
void launch_q45_merge(const void* w, float* o, int d, const MergeArgs& mg) {
    constexpr int WG = 64 * NB, SPLIT = 4;
    constexpr int rows_per_wg = WG / (8 * SPLIT);
    const size_t lds = ((size_t)NB * 292 + 15) & ~(size_t)15;
    hipLaunchKernelGGL((gemv_q45_rows_kernel<Q5, 1, false, NB, SPLIT, false, WG, 2, true>),
                       dim3((d + rows_per_wg - 1) / rows_per_wg), dim3(WG), lds, g4_stream(), (const uint8_t*)w,
                       nullptr, nullptr, o, NB, d, nullptr, nullptr, nullptr, nullptr, nullptr, ResidualArgs{},
                       Stack2{}, mg);
}

// residual step + norm + Q8_K as the prologue of every workgroup (64 NB
// threads: one wave per Q8_K block); a row takes 32 lanes (64 with two
// matrices), i.e. 2 NB (NB) rows per workgroup.  At the E4B shape (n = 2560):
// Q|K|V 7.2 us and the PLE gate 5.9 us per launch, against 9.0 / 7.1 us with
// 16 lanes per row (four times fewer workgroups, each CU's SIMDs holding 2.5
// waves of the work) and 8.0 / 6.4 us for the 256-thread form before it;
// 64 lanes per row measured the same as 32 for the PLE gate and 8.4 us for
// Q|K|V.  With 32 lanes per row the four lane groups hand their block values
// to group 0 through LDS: decode step 2.214 against 2.227 ms with lane
// shuffles (64 lanes per row: 2.257 with LDS, 2.281 with shuffles).
template <bool Q5, int NMAT, int NB>
void launch_q45_pro(const void* w, const void* w2, float* o, int d, const float* aux, const ResidualArgs& ra,
                    const Stack2& st) {
    if constexpr (NMAT == 2 || NB > 10) {
        launch_q45_pro_s<Q5, NMAT, NB, 8>(w, w2, o, d, aux, ra, st);
    } else {
        // 16 lanes per K-quant row where 32 would need more workgroups than
        // there are CUs: a ten-wave workgroup fills a CU's wave slots, so the
        // excess ran as a second round of prologues (the global layers'
        // Q|K|V, 4096 + 1024 + 1024 rows: 308 workgroups, 11.5 us; 180 with
        // the Q6_K V rows still on four slices each)
        constexpr int WG = 64 * NB;
        // one matrix alone (the Q projection of the shared-KV layers, 2048
        // rows: 205 workgroups instead of 103) takes 64 lanes a row where
        // that grid fits the CUs: decode step 2.0315 against 2.0354 ms (mean
        // of four A/B pairs on one box)
        if (!w2 && !st.w && !st.w6 && (d + WG / 64 - 1) / (WG / 64) <= g4_num_cus()) {
            launch_q45_pro_s<Q5, NMAT, NB, 8, true>(w, w2, o, d, aux, ra, st);
            return;
        }
        const int wgs4 = (d + st.d + WG / 32 - 1) / (WG / 32) +
                         (st.w6 ? (st.d6 + q6_pro_rows(WG, 4) - 1) / q6_pro_rows(WG, 4) : 0);
        if (wgs4 > g4_num_cus()) launch_q45_pro_s<Q5, NMAT, NB, 2, true, 4>(w, w2, o, d, aux, ra, st);
        else launch_q45_pro_s<Q5, NMAT, NB, 4, true>(w, w2, o, d, aux, ra, st);
    }
}

template <bool Q5, int NB>
void launch_q45_pro_nm(const void* w, const void* w2, float* o, int d, const float* aux, const ResidualArgs& ra,
                       const Stack2& st) {
    if (w2 && !st.w && !st.w6) {
        // gate|up: the streaming kernel, NB waves of 4 rows x {gate, up}
        hipLaunchKernelGGL((gemv_q45_stream_kernel<Q5, NB, 2, true>), dim3((d + 4 * NB - 1) / (4 * NB)), dim3(64 * NB), 0,
                           g4_stream(), (const uint8_t*)w, (const uint8_t*)w2, nullptr, o, d, nullptr, ra);
    } else if (w2) {
        launch_q45_pro<Q5, 2, NB>(w, w2, o, d, nullptr, ra, st);
    } else {
        launch_q45_pro<Q5, 1, NB>(w, nullptr, o, d, aux, ra, st);
    }
}

// rows of nb blocks; the split of a row over lane groups grows with the work
// per lane (the fused gate|up pair does twice the integer work per block)
template <bool Q5, int NMAT, bool DBG>
int launch_q45(const void* w0, const void* w1, const void* q8, float* o, int nb, int d, int32_t* S, int32_t* M,
               const float* aux = nullptr) {
    constexpr int SP = NMAT == 2 ? 4 : 2;
    if (!DBG && (nb == 8 || nb == 10 || nb == 16)) {
        const dim3 grid((d + 8 / NMAT - 1) / (8 / NMAT));
        const uint8_t* a = (const uint8_t*)w0;
        const uint8_t* b = (const uint8_t*)w1;
        const ResidualArgs none{};
        if (nb == 8) hipLaunchKernelGGL((gemv_q45_stream_kernel<Q5, 8, NMAT>), grid, dim3(64), 0, g4_stream(), a, b, (const uint8_t*)q8, o, d, aux, none);
        else if (nb == 10) hipLaunchKernelGGL((gemv_q45_stream_kernel<Q5, 10, NMAT>), grid, dim3(64), 0, g4_stream(), a, b, (const uint8_t*)q8, o, d, aux, none);
        else hipLaunchKernelGGL((gemv_q45_stream_kernel<Q5, 16, NMAT>), grid, dim3(64), 0, g4_stream(), a, b, (const uint8_t*)q8, o, d, aux, none);
        return g4_check_launch("gemv_q45_stream_kernel");
    }
    switch (nb) {   // unrolled for the row lengths of the model (256, 2048, 2560, 4096)
    case 1: launch_q45_nb<Q5, NMAT, DBG, 1, 1>(w0, w1, q8, o, nb, d, S, M, nullptr, nullptr, aux); break;
    case 8: launch_q45_nb<Q5, NMAT, DBG, 8, SP>(w0, w1, q8, o, nb, d, S, M, nullptr, nullptr, aux); break;
    case 10: launch_q45_nb<Q5, NMAT, DBG, 10, SP>(w0, w1, q8, o, nb, d, S, M, nullptr, nullptr, aux); break;
    case 16: launch_q45_nb<Q5, NMAT, DBG, 16, SP>(w0, w1, q8, o, nb, d, S, M, nullptr, nullptr, aux); break;
    default: launch_q45_nb<Q5, NMAT, DBG, 0, 1>(w0, w1, q8, o, nb, d, S, M, nullptr, nullptr, aux); break;
    }
    return g4_check_launch("gemv_q45_rows_kernel");
}

// rows per workgroup pass = 32/KS; pick the smallest split that still gives
// at least two workgroups per CU
template <bool SOFTCAP, int KS>
void launch_q6_ks(const void* w, const float* x, float* o, int nb, int d, float cap) {
    const int ngroups = (d + 32 / KS - 1) / (32 / KS);
    int grid = 4 * g4_num_cus();
    if (grid > ngroups) grid = ngroups;
    const size_t lds = (size_t)nb * kQ6XsBlk * 4 + (size_t)nb * 128 + 32 * 4;
    hipLaunchKernelGGL((gemv_q6k_rows_kernel<KS, SOFTCAP>), dim3(grid), dim3(256), lds, g4_stream(),
                       (const uint8_t*)w, x, o, nb, d, cap, nullptr);
}

// the register-x kernel for rows of 10 blocks (the LM head at hidden 2560)
// once there are enough rows for two workgroups per CU; returns the grid,
// 0 when it does not apply
constexpr int kXrWgPerCu = 1;
template <bool SOFTCAP, bool AM>
int launch_q6_xreg(const void* w, const float* x, float* o, int nb, int d, float cap, unsigned long long* part) {
    const int nbatch = d / (8 * kXrRpi);
    const int grid = kXrWgPerCu * g4_num_cus();
    if (nb != 10 || d % (8 * kXrRpi) || nbatch < grid) return 0;
    hipLaunchKernelGGL((gemv_q6k_xreg_kernel<10, SOFTCAP, AM>), dim3(grid), dim3(8 * 10 * kXrRpi), 0, g4_stream(),
                       (const uint8_t*)w, x, o, d, cap, part);
    return grid;
}

template <bool SOFTCAP>
int launch_q6_f32(const void* w, const float* x, float* o, int nb, int d, float cap) {
    if (launch_q6_xreg<SOFTCAP, false>(w, x, o, nb, d, cap, nullptr)) return g4_check_launch("gemv_q6k_xreg_kernel");
    if (!SOFTCAP && nb <= kQ6SliceMaxNb && nb % 8 == 0) {
        hipLaunchKernelGGL((gemv_q6k_kslice_kernel<kQ6SliceRows>), dim3((d + kQ6SliceRows - 1) / kQ6SliceRows),
                           dim3(8 * nb), 0, g4_stream(), (const uint8_t*)w, x, o, nb, d);
        return g4_check_launch("gemv_q6k_kslice_kernel");
    }
    const int target = 2 * g4_num_cus();
    if ((d + 31) / 32 >= target) launch_q6_ks<SOFTCAP, 1>(w, x, o, nb, d, cap);
    else if ((d + 15) / 16 >= target) launch_q6_ks<SOFTCAP, 2>(w, x, o, nb, d, cap);
    else if ((d + 7) / 8 >= target) launch_q6_ks<SOFTCAP, 4>(w, x, o, nb, d, cap);
    else launch_q6_ks<SOFTCAP, 8>(w, x, o, nb, d, cap);
    return g4_check_launch("gemv_q6k_rows_kernel");
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

bool aligned16(const void* p);

// ---- dense weights of any row length (F32, F16, BF16) -----------------------
// mm_f32 (main.c:1494-1517, cblas_sgemv over row bands), mm_f16 (1519-1527),
// mm_bf16 (1529-1537): o[i] = sum_j x[j] * w[i][j] in fp32.  One wave per
// row, x staged in LDS, the row streamed in 16-byte chunks (8 halves or 4
// floats), eight chunks per lane in flight; the wave's partial sums are
// added by a butterfly (a tree, not the reference's sequential order).
template <int T>   // 0: bf16, 1: f16, 2: f32
__global__ __launch_bounds__(kWG) void gemv_dense_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                         float* __restrict__ out, int n, int d) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    constexpr int EPC = T == 2 ? 4 : 8;   // elements per 16-byte chunk
    constexpr int ES = T == 2 ? 4 : 2;    // element bytes
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nch = n / EPC;
    const int row = blockIdx.x * (kWG / 64) + wave;
    for (int k = tid; k < n / 4; k += kWG) reinterpret_cast<float4*>(xs)[k] = reinterpret_cast<const float4*>(x)[k];
    __syncthreads();
    if (row >= d) return;
    const uint4* wr = reinterpret_cast<const uint4*>(w + (size_t)row * n * ES);
    float acc = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 64 * 8) {
        uint4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int ch = c0 + lane + 64 * j;
            v[j] = ch < nch ? wr[ch] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int ch = c0 + lane + 64 * j;
            if (ch >= nch) continue;
            const uint32_t u[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            if (T == 2) {
                const float4 xa = reinterpret_cast<const float4*>(xs)[ch];
                acc = __builtin_fmaf(xa.x, __uint_as_float(u[0]), acc);
                acc = __builtin_fmaf(xa.y, __uint_as_float(u[1]), acc);
                acc = __builtin_fmaf(xa.z, __uint_as_float(u[2]), acc);
                acc = __builtin_fmaf(xa.w, __uint_as_float(u[3]), acc);
            } else {
                const float4 xa = reinterpret_cast<const float4*>(xs)[2 * ch];
                const float4 xb = reinterpret_cast<const float4*>(xs)[2 * ch + 1];
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t hbits = (u[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                    acc = __builtin_fmaf(xv[e], T == 0 ? bf16_to_f32(hbits) : f16_to_f32(hbits), acc);
                }
            }
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) out[row] = acc;
}

// mm_quant_rows (main.c:1539-1556) for Q4_K / Q5_K, the path of the
// reference's --f32-matmul switch (main.c:1680-1683): every weight
// dequantized to its fp32 value (dequant_q4_k / dequant_q5_k, main.c:172-211)
// and multiplied by the fp32 activation.  One wave per row, x in LDS.
__global__ __launch_bounds__(kWG) void gemv_kq_f32_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                          float* __restrict__ out, int type, int nb, int d) {
    extern __shared__ __align__(16) uint8_t smem[];
    float* xs = reinterpret_cast<float*>(smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n = nb * 256;
    const int row = blockIdx.x * (kWG / 64) + wave;
    for (int k = tid; k < n / 4; k += kWG) reinterpret_cast<float4*>(xs)[k] = reinterpret_cast<const float4*>(x)[k];
    __syncthreads();
    if (row >= d) return;
    const size_t nblk = (size_t)d * nb;
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const size_t blk = (size_t)row * nb + b;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = lane + 64 * k;
            acc = __builtin_fmaf(xs[b * 256 + e], dequant_elem(w, type, nblk, blk, e), acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) out[row] = acc;
}

int launch_dense(int T, const char* who, float* o, const float* x, const void* w, int n, int d) {
    if (!o || !x || !w) return g4_fail(G4_ERR_ARG, "%s: null pointer", who);
    if (!aligned16(w) || !aligned16(x)) return g4_fail(G4_ERR_ARG, "%s: w and x must be 16-byte aligned", who);
    const int mult = T == 2 ? 4 : 8;
    if (n <= 0 || d <= 0 || n % mult || n > 16384)
        return g4_fail(G4_ERR_ARG, "%s: n=%d unsupported (multiple of %d, <= 16384), d=%d", who, n, mult, d);
    const dim3 grid((d + kWG / 64 - 1) / (kWG / 64));
    const size_t lds = (size_t)n * 4;
    const uint8_t* wp = (const uint8_t*)w;
    if (T == 0) hipLaunchKernelGGL(gemv_dense_kernel<0>, grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    else if (T == 1) hipLaunchKernelGGL(gemv_dense_kernel<1>, grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    else hipLaunchKernelGGL(gemv_dense_kernel<2>, grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    return g4_check_launch("gemv_dense_kernel");
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
    if (type == G4_Q4_K || type == G4_Q5_K) {
        hipLaunchKernelGGL(gemv_kq_f32_kernel, dim3((d + kWG / 64 - 1) / (kWG / 64)), dim3(kWG), (size_t)n * 4,
                           g4_stream(), (const uint8_t*)w, x, o, type, n / 256, d);
        return g4_check_launch("gemv_kq_f32_kernel");
    }
    if (type != G4_Q6_K) return g4_fail(G4_ERR_TYPE, "g4_mm_quant_rows: type %d not supported", type);
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

// rows kernel with the argmax keys: returns the grid (number of keys)
template <bool SOFTCAP, int KS>
int launch_q6_am(const void* w, const float* x, float* o, int nb, int d, float cap, unsigned long long* part) {
    const int ngroups = (d + 32 / KS - 1) / (32 / KS);
    int grid = 4 * g4_num_cus();
    if (grid > ngroups) grid = ngroups;
    const size_t lds = (size_t)nb * kQ6XsBlk * 4 + (size_t)nb * 128 + 32 * 4;
    hipLaunchKernelGGL((gemv_q6k_rows_kernel<KS, SOFTCAP, true>), dim3(grid), dim3(256), lds, g4_stream(),
                       (const uint8_t*)w, x, o, nb, d, cap, part);
    return grid;
}

template <bool SOFTCAP>
int launch_q6_am_ks(const void* w, const float* x, float* o, int nb, int d, float cap, unsigned long long* part) {
    if (const int g = launch_q6_xreg<SOFTCAP, true>(w, x, o, nb, d, cap, part)) return g;
    const int target = 2 * g4_num_cus();
    if ((d + 31) / 32 >= target) return launch_q6_am<SOFTCAP, 1>(w, x, o, nb, d, cap, part);
    if ((d + 15) / 16 >= target) return launch_q6_am<SOFTCAP, 2>(w, x, o, nb, d, cap, part);
    if ((d + 7) / 8 >= target) return launch_q6_am<SOFTCAP, 4>(w, x, o, nb, d, cap, part);
    return launch_q6_am<SOFTCAP, 8>(w, x, o, nb, d, cap, part);
}

extern "C" size_t g4_mm_argmax_part_bytes(int d) {
    const size_t a = (size_t)4 * g4_num_cus(), b = g4_argmax_part_bytes(d > 0 ? d : 1) / 8;
    return 8 * (a > b ? a : b);
}

// mm_argmax_row (main.c:1570-1667) and the greedy choice after logits_tied
// (main.c:1780-1796, 2045-2049): the first index of the largest output of
// W . x, of cap * tanh(W . x / cap) when cap > 0.  Q6_K: one launch of the
// LM-head rows kernel that also reduces each workgroup's rows to an argmax
// key, then the final pass; the outputs (d floats) go to logits either way
// (1 MB at the vocabulary of Gemma 4, small beside the 551 MB of weights).
// The other types: g4_mm into logits, the soft-cap, g4_argmax.
extern "C" int g4_mm_argmax_row(const float* x, const void* w, int n, int d, int type, void* q8, float cap,
                                float* logits, void* part, int* out, int* dtok, int* dpos) {
    G4_CHECK_ARG(x && w && part && n > 0 && d > 0, "g4_mm_argmax_row: bad arguments");
    if (type == G4_Q6_K) {
        if (n % 256) return g4_fail(G4_ERR_ARG, "g4_mm_argmax_row: n=%d is not a multiple of 256", n);
        G4_CHECK_ARG(aligned16(w) && aligned16(x), "g4_mm_argmax_row: w and x must be 16-byte aligned");
        float* o = logits;
        G4_CHECK_ARG(o != nullptr, "g4_mm_argmax_row: the logits buffer (d floats) is required");
        unsigned long long* pk = (unsigned long long*)part;
        const int np = cap > 0.0f ? launch_q6_am_ks<true>(w, x, o, n / 256, d, cap, pk)
                                  : launch_q6_am_ks<false>(w, x, o, n / 256, d, 0.0f, pk);
        int rc = g4_check_launch("gemv_q6k_rows_kernel (argmax)");
        if (rc) return rc;
        return g4_argmax_final(part, np, out, dtok, dpos);
    }
    G4_CHECK_ARG(logits, "g4_mm_argmax_row: type %d needs the logits buffer (d floats)", type);
    int rc = g4_mm(logits, x, w, n, d, type, q8, 0);
    if (rc) return rc;
    if (cap > 0.0f && (rc = g4_softcap(logits, d, cap))) return rc;
    return g4_argmax(logits, d, out, part, dtok, dpos);
}

extern "C" int g4_mm_bf16(float* o, const float* x, const void* w, int n, int d) {
    if (!o || !x || !w) return g4_fail(G4_ERR_ARG, "g4_mm_bf16: null pointer");
    if (!aligned16(w) || !aligned16(x)) return g4_fail(G4_ERR_ARG, "g4_mm_bf16: w and x must be 16-byte aligned");
    if (n > 4096) return launch_dense(0, "g4_mm_bf16", o, x, w, n, d);
    if (n <= 0 || d <= 0 || n % 8) return g4_fail(G4_ERR_ARG, "g4_mm_bf16: n=%d unsupported (multiple of 8)", n);
    const int cpl = (n / 8 + 63) / 64;
    const size_t lds = (size_t)n * 4;
    const dim3 grid((d + 7) / 8);
    const uint16_t* wp = (const uint16_t*)w;
    if (cpl <= 4) hipLaunchKernelGGL((gemv_bf16_kernel<2, 4>), grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    else hipLaunchKernelGGL((gemv_bf16_kernel<2, 8>), grid, dim3(kWG), lds, g4_stream(), wp, x, o, n, d);
    return g4_check_launch("gemv_bf16_kernel");
}

// mm_f16 (main.c:1519-1527)
extern "C" int g4_mm_f16(float* o, const float* x, const void* w, int n, int d) {
    return launch_dense(1, "g4_mm_f16", o, x, w, n, d);
}

// mm_f32 (main.c:1494-1517)
extern "C" int g4_mm_f32(float* o, const float* x, const void* w, int n, int d) {
    return launch_dense(2, "g4_mm_f32", o, x, w, n, d);
}

extern "C" int g4_mm(float* o, const float* x, const void* w, int n, int d, int type, void* q8, int q8_ready) {
    switch (type) {
    case G4_F32: return g4_mm_f32(o, x, w, n, d);
    case G4_F16: return g4_mm_f16(o, x, w, n, d);
    case G4_Q4_K:
    case G4_Q5_K: {
        if (n % 256) return g4_fail(G4_ERR_ARG, "mm: n=%d not multiple of QK_K", n);
        if (!q8_ready && n == 256) {
            // one Q8_K block: every workgroup quantizes x itself (no separate launch)
            int rc = check_gemv("mm", o, w, x, n, d);
            if (rc) return rc;
            G4_CHECK_ARG(q8, "mm: null q8");
            if (type == G4_Q4_K) launch_q45_nb<false, 1, false, 1, 1, true>(w, nullptr, nullptr, o, 1, d, nullptr, nullptr, x, q8);
            else launch_q45_nb<true, 1, false, 1, 1, true>(w, nullptr, nullptr, o, 1, d, nullptr, nullptr, x, q8);
            return g4_check_launch("gemv_q45_rows_kernel");
        }
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

extern "C" int g4_mm_quant_dot_rows_gelu_mul(float* o, const void* w, int n, int d, int type, const void* q8,
                                             const float* mul) {
    int rc = check_gemv("g4_mm_quant_dot_rows_gelu_mul", o, w, q8, n, d);
    if (rc) return rc;
    if (!mul) return g4_fail(G4_ERR_ARG, "g4_mm_quant_dot_rows_gelu_mul: null mul");
    const int nb = n / 256;
    if (type == G4_Q4_K) return launch_q45<false, 1, false>(w, nullptr, q8, o, nb, d, nullptr, nullptr, mul);
    if (type == G4_Q5_K) return launch_q45<true, 1, false>(w, nullptr, q8, o, nb, d, nullptr, nullptr, mul);
    return g4_fail(G4_ERR_TYPE, "g4_mm_quant_dot_rows_gelu_mul: type %d not supported", type);
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

static int mm_residual(const char* who, float* o, const void* w, const void* w2, int n, int d, int type,
                       const float* mul, const Stack2& st, const float* x, float* x_out, const float* y,
                       const float* w_post, const float* oscale, const float* w_next, float* xb2, void* q8, int qsrc,
                       float eps) {
    int rc = check_gemv(who, o, w, x, n, d);
    if (rc) return rc;
    G4_CHECK_ARG(!w2 || (aligned16(w2) && !mul), "%s: bad w2 (16-byte aligned, no mul)", who);
    G4_CHECK_ARG(!y || w_post, "%s: y without w_post", who);
    G4_CHECK_ARG(qsrc == 1 || w_next, "%s: quantizing the normed vector needs w_next", who);
    G4_CHECK_ARG(!(y && x_out == x), "%s: x_out must not alias x when y is given", who);
    G4_CHECK_ARG(!(y && xb2 == y), "%s: xb2 must not alias y", who);
    G4_CHECK_ARG(!q8 || aligned16(q8), "%s: q8 must be 16-byte aligned", who);
    // the prologue reads and writes the vectors as float4
    G4_CHECK_ARG(aligned16(x) && (!x_out || aligned16(x_out)) && (!y || (aligned16(y) && aligned16(w_post))) &&
                     (!w_next || aligned16(w_next)) && (!xb2 || aligned16(xb2)),
                 "%s: x, x_out, y, w_post, w_next and xb2 must be 16-byte aligned", who);
    ResidualArgs ra{x, x_out, y, w_post, oscale, w_next, xb2, (uint8_t*)q8, qsrc, n, eps};
    const int nb = n / 256;
    const bool q5 = type == G4_Q5_K;
    if (type != G4_Q4_K && !q5) return g4_fail(G4_ERR_TYPE, "%s: type %d not supported", who, type);
    switch (nb) {
    case 8: q5 ? launch_q45_pro_nm<true, 8>(w, w2, o, d, mul, ra, st) : launch_q45_pro_nm<false, 8>(w, w2, o, d, mul, ra, st); break;
    case 10: q5 ? launch_q45_pro_nm<true, 10>(w, w2, o, d, mul, ra, st) : launch_q45_pro_nm<false, 10>(w, w2, o, d, mul, ra, st); break;
    case 16: q5 ? launch_q45_pro_nm<true, 16>(w, w2, o, d, mul, ra, st) : launch_q45_pro_nm<false, 16>(w, w2, o, d, mul, ra, st); break;
    default: return g4_fail(G4_ERR_ARG, "%s: n=%d (2048, 2560 or 4096)", who, n);
    }
    return g4_check_launch("gemv_q45_rows_kernel<prologue>");
}

// g4_residual_norm (with the residual stream read from x and written to
// x_out) followed by mm_quant_dot_rows on its Q8_K, in one launch: every
// workgroup computes the norm and the Q8_K itself (into LDS) while its weight
// loads are in flight; workgroup 0 stores x_out, xb2 and q8.  With w2 the
// GEMV is the fused gate|up pair: o = gelu(W.x) * (W2.x).
extern "C" int g4_mm_residual_q8(float* o, const void* w, const void* w2, int n, int d, int type, const float* mul,
                                 const float* x, float* x_out, const float* y, const float* w_post,
                                 const float* oscale, const float* w_next, float* xb2, void* q8, int qsrc, float eps) {
    return mm_residual("g4_mm_residual_q8", o, w, w2, n, d, type, mul, Stack2{}, x, x_out, y, w_post, oscale, w_next,
                       xb2, q8, qsrc, eps);
}

// The same with a second, independent GEMV of the same type and n on the
// same Q8_K in the same launch (e.g. the Q and K projections): o1 = W1.q8
// (d1 rows), o2 = W2.q8 (d2 rows).
extern "C" int g4_mm_residual_q8_pair(float* o1, const void* w1, int d1, float* o2, const void* w2, int d2, int n,
                                      int type, const float* x, float* x_out, const float* y, const float* w_post,
                                      const float* oscale, const float* w_next, float* xb2, void* q8, int qsrc,
                                      float eps) {
    G4_CHECK_ARG(o2 && w2 && aligned16(w2) && d2 > 0, "g4_mm_residual_q8_pair: bad second tensor");
    return mm_residual("g4_mm_residual_q8_pair", o1, w1, nullptr, n, d1, type, nullptr,
                       Stack2{(const uint8_t*)w2, o2, d2, nullptr, nullptr, 0}, x, x_out, y, w_post, oscale, w_next,
                       xb2, q8, qsrc, eps);
}

// ... and a third, Q6_K GEMV on the fp32 normed vector (mm_quant_rows,
// main.c:1539-1556): the Q, K and V projections of a layer in one launch.
extern "C" int g4_mm_residual_q8_qkv(float* o1, const void* w1, int d1, float* o2, const void* w2, int d2, float* o3,
                                     const void* w3, int d3, int type3, int n, int type, const float* x, float* x_out,
                                     const float* y, const float* w_post, const float* oscale, const float* w_next,
                                     float* xb2, void* q8, float eps) {
    G4_CHECK_ARG(o2 && w2 && aligned16(w2) && d2 > 0, "g4_mm_residual_q8_qkv: bad second tensor");
    G4_CHECK_ARG(o3 && w3 && aligned16(w3) && d3 > 0, "g4_mm_residual_q8_qkv: bad third tensor");
    if (type3 != G4_Q6_K) return g4_fail(G4_ERR_TYPE, "g4_mm_residual_q8_qkv: third tensor type %d (Q6_K only)", type3);
    return mm_residual("g4_mm_residual_q8_qkv", o1, w1, nullptr, n, d1, type, nullptr,
                       Stack2{(const uint8_t*)w2, o2, d2, (const uint8_t*)w3, o3, d3}, x, x_out, y, w_post, oscale,
                       w_next, xb2, q8, 0, eps);
}

// The attention output projection with the merge of the decode attention's
// chunk partials as its prologue (n = n_heads * 256)
extern "C" int g4_mm_attn_merge(float* o, const void* w, int n, int d, int type, const float* part, int G, int n_heads,
                                int hd, float* q_out, void* q8) {
    int rc = check_gemv("g4_mm_attn_merge", o, w, part, n, d);
    if (rc) return rc;
    G4_CHECK_ARG((hd == 256 || hd == 512) && n_heads > 0 && n == n_heads * hd,
                 "g4_mm_attn_merge: head_dim %d, %d heads, n=%d", hd, n_heads, n);
    G4_CHECK_ARG(G >= 1 && G <= kMergeMaxG, "g4_mm_attn_merge: %d chunks (1..%d)", G, kMergeMaxG);
    G4_CHECK_ARG(!q_out || aligned16(q_out), "g4_mm_attn_merge: q_out must be 16-byte aligned");
    G4_CHECK_ARG(!q8 || aligned16(q8), "g4_mm_attn_merge: q8 must be 16-byte aligned");
    const MergeArgs mg{part, q_out, (uint8_t*)q8, G, hd / 256};
    const bool q5 = type == G4_Q5_K;
    if (type != G4_Q4_K && !q5) return g4_fail(G4_ERR_TYPE, "g4_mm_attn_merge: type %d not supported", type);
    switch (n / 256) {
    case 8: q5 ? launch_q45_merge<true, 8>(w, o, d, mg) : launch_q45_merge<false, 8>(w, o, d, mg); break;
    case 16: q5 ? launch_q45_merge<true, 16>(w, o, d, mg) : launch_q45_merge<false, 16>(w, o, d, mg); break;
    default: return g4_fail(G4_ERR_ARG, "g4_mm_attn_merge: %d heads of %d (n = 2048 or 4096)", n_heads, hd);
    }
    return g4_check_launch("gemv_q45_rows_kernel<merge>");
}

// The PLE gate and projection of a decode layer in one launch (see
// ple_fused_kernel): pairs holds g4_ple_pairs_bytes(pd) bytes, zeroed before
// the first call.
extern "C" size_t g4_ple_pairs_bytes(int pd) { return pd > 0 ? ple_pair_words(pd) * 8 + 16 : 0; }

extern "C" int g4_mm_ple_gate_proj(float* y, const void* w_proj, int type_proj, int d_proj, const void* w_gate,
                                   int type_gate, int n, int pd, const float* mul, const float* x, float* x_out,
                                   const float* y_in, const float* w_post, float eps, void* pairs,
                                   const uint32_t* seq) {
    const char* who = "g4_mm_ple_gate_proj";
    G4_CHECK_ARG(y && w_proj && w_gate && mul && x && x_out && y_in && w_post && pairs && seq, "%s: null pointer", who);
    G4_CHECK_ARG(n == 256 * kPleNB && pd == 256 && d_proj > 0, "%s: n=%d pd=%d d_proj=%d (n = %d, pd = 256)", who, n,
                 pd, d_proj, 256 * kPleNB);
    G4_CHECK((type_gate == G4_Q4_K || type_gate == G4_Q5_K) && (type_proj == G4_Q4_K || type_proj == G4_Q5_K),
             G4_ERR_TYPE, "%s: types %d / %d not supported", who, type_gate, type_proj);
    G4_CHECK_ARG(aligned16(w_proj) && aligned16(w_gate) && aligned16(x) && aligned16(x_out) && aligned16(y_in) &&
                     aligned16(w_post) && aligned16(pairs),
                 "%s: weights, x, x_out, y_in, w_post and pairs must be 16-byte aligned", who);
    G4_CHECK_ARG(x_out != x && (const float*)y != x && y != x_out && (const float*)y != y_in,
                 "%s: x_out must differ from x, y from x, x_out and y_in", who);
    const ResidualArgs ra{x, x_out, y_in, w_post, nullptr, nullptr, nullptr, nullptr, 1, n, eps};
    constexpr int NB = kPleNB, WG = 64 * NB;
    const size_t lds = (size_t)NB * 256 * 4 + (((size_t)NB * 292 + 15) & ~(size_t)15) + (size_t)NB * 32 * 4 +
                       (size_t)WG / 8 * 4;
    const int wgs = (pd + kPleGateRows - 1) / kPleGateRows + (d_proj + kPleProjRows - 1) / kPleProjRows;
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(wgs), dim3(WG), lds, g4_stream(), (const uint8_t*)w_gate, (const uint8_t*)w_proj,
                           y, pd, d_proj, mul, ra, (unsigned long long*)pairs, seq);
    };
    const bool q5g = type_gate == G4_Q5_K, q5p = type_proj == G4_Q5_K;
    if (!q5g && !q5p) go(ple_fused_kernel<false, false>);
    else if (!q5g) go(ple_fused_kernel<false, true>);
    else if (!q5p) go(ple_fused_kernel<true, false>);
    else go(ple_fused_kernel<true, true>);
    return g4_check_launch("ple_fused_kernel");
}
