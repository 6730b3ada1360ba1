// glue.hip -- per-token step glue on gfx950: embedding lookup, the
// per-layer-embedding (PLE) input, the PLE gate, greedy argmax.
//
// Reference (gemma4-4b/cpu-blas/main.c):
//   emb_lookup       1696-1723 (row dequantized with dequant_q*_k, 172-237)
//   x *= sqrtf(dim)  1849-1854
//   build_ple        1747-1778
//   PLE gate         1988-1993: g = gelu(g); g *= ple[l]
//   greedy sampling  2045-2049: first index of the maximum
//
// Quantized tables are in the planar HBM layout (g4_device.h); the element
// values are the reference's dequantized fp32 values bit for bit.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

// one row of a table (row length dim) -> fp32, times scale
__device__ float table_elem(const void* w, int type, int rows, int dim, int row, int i) {
    switch (type) {
    case G4_F32: return reinterpret_cast<const float*>(w)[(size_t)row * dim + i];
    case G4_F16: return f16_to_f32(reinterpret_cast<const uint16_t*>(w)[(size_t)row * dim + i]);
    case G4_BF16: return bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[(size_t)row * dim + i]);
    default: {
        const int nb = dim / 256;
        return dequant_elem((const uint8_t*)w, type, (size_t)rows * nb, (size_t)row * nb + i / 256, i & 255);
    }
    }
}

__global__ __launch_bounds__(256) void emb_lookup_kernel(float* __restrict__ o, const void* w, int type, int rows,
                                                         int dim, const int* dtok, int tok, int use_scale,
                                                         float scale) {
    const int id = dtok ? *dtok : tok;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim || id < 0 || id >= rows) return;
    const float v = table_elem(w, type, rows, dim, id, i);
    o[i] = use_scale ? v * scale : v;
}

// the decode step's inputs in one launch: workgroups 0 .. ceil(dim/256)-1
// take emb_lookup_kernel's elements, the next two the (cos, sin) tables of
// the two RoPE variants at position *dpos (rope_table_kernel's values)
struct RopeTab {
    float2* tab;
    const float* ff;
    float ts;
    int npair;
};
__global__ __launch_bounds__(256) void emb_rope_kernel(float* __restrict__ o, const void* w, int type, int rows, int dim,
                                                       const int* dtok, float scale, const int* dpos, float fs,
                                                       RopeTab ta, RopeTab tb) {
    const int ne = (dim + 255) / 256;
    if ((int)blockIdx.x >= ne) {
        const RopeTab& t = blockIdx.x == ne ? ta : tb;
        const int p = *dpos;
        for (int j = threadIdx.x; j < t.npair; j += 256) t.tab[j] = rope_pair_cs(p, j, t.ts, fs, t.ff);
        return;
    }
    const int id = *dtok;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim || id < 0 || id >= rows) return;
    o[i] = table_elem(w, type, rows, dim, id, i) * scale;
}

// ... and the PLE context projection of the same row (main.c:1747-1750:
// ctx = W . x, W bf16 [d x dim]) in the same launch: workgroups [0, gx)
// take 8 rows of ctx each (4 waves x 2 rows, gemv_bf16_kernel's dot: the
// same bits), issue their weight loads, then rebuild x = table row * scale
// in LDS themselves (emb_rope_kernel's values) while the weights are in
// flight; workgroup 0 also stores x (and advances the step's sequence word
// *seq, if given).  Workgroups gx and gx + 1 write the two RoPE tables.
template <int RPW, int CPL>
__global__ __launch_bounds__(256) void emb_ple_kernel(float* __restrict__ o, const void* emb, int type, int rows,
                                                      int dim, const int* dtok, float scale,
                                                      const uint16_t* __restrict__ w, float* __restrict__ ctx, int d,
                                                      const int* dpos, float fs, RopeTab ta, RopeTab tb,
                                                      uint32_t* seq) {
    const int gx = (d + 4 * RPW - 1) / (4 * RPW);
    if (seq && blockIdx.x == 0 && threadIdx.x == 0) *seq += 1u;
    if ((int)blockIdx.x >= gx) {
        const RopeTab& t = (int)blockIdx.x == gx ? ta : tb;
        const int p = *dpos;
        for (int j = threadIdx.x; j < t.npair; j += 256) t.tab[j] = rope_pair_cs(p, j, t.ts, fs, t.ff);
        return;
    }
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = (blockIdx.x * 4 + wave) * RPW;
    uint4 v[RPW][CPL];
    bf16_rows_load<RPW, CPL>(w, dim, d, row0, lane, v);
    const int id = *dtok;
    const bool ok = id >= 0 && id < rows;
    for (int i = tid; i < dim; i += 256) {
        const float e = ok ? table_elem(emb, type, rows, dim, id, i) * scale : 0.0f;
        xs[i] = e;
        if (blockIdx.x == 0 && ok) o[i] = e;
    }
    lds_sync();
    float res[RPW];
    bf16_rows_dot<RPW, CPL>(v, xs, dim / 8, lane, res);
#pragma unroll
    for (int r = 0; r < RPW; r++)
        if (lane == 0 && row0 + r < d) ctx[row0 + r] = res[r];
}

// token z = blockIdx.y of a prompt chunk -> row z of o
__global__ __launch_bounds__(256) void emb_lookup_rows_kernel(float* __restrict__ o, const void* w, int type, int rows,
                                                              int dim, const int* __restrict__ dtok, float scale) {
    const int id = dtok[blockIdx.y];
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim || id < 0 || id >= rows) return;
    o[(size_t)blockIdx.y * dim + i] = table_elem(w, type, rows, dim, id, i) * scale;
}

// build_ple after the context projection (main.c:1751-1777): workgroup l
// owns slice l of pd elements.
//   row  = emb_lookup(ple_tok, token)[l*pd + i] * sc_tok
//   ctx  = rmsnorm(ctx[l*pd + i] * sc_ctx, proj_norm)
//   ple  = (row + ctx) * mix
struct PleArgs {
    const void* ple_tok;
    const float* ctx;
    const float* proj_norm;
    float* ple;
    const int* dtok;
    int tok, type, rows, pd, L;
    float sc_tok, sc_ctx, mix, eps;
};

__device__ __forceinline__ void ple_finish_slice(const PleArgs& a, int l, float* __restrict__ ple,
                                                 const float* __restrict__ ctx, int id, float* c, float* red) {
    const int pd = a.pd;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < pd; i += blockDim.x) {
        const float v = ctx[(size_t)l * pd + i] * a.sc_ctx;
        c[i] = v;
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)pd + a.eps);
    if (id < 0 || id >= a.rows) return;
    for (int i = threadIdx.x; i < pd; i += blockDim.x) {
        const float ctxn = (c[i] * s) * a.proj_norm[i];
        const float row = table_elem(a.ple_tok, a.type, a.rows, pd * a.L, id, l * pd + i) * a.sc_tok;
        ple[(size_t)l * pd + i] = (row + ctxn) * a.mix;
    }
}

__global__ __launch_bounds__(256) void ple_finish_kernel(PleArgs a) {
    extern __shared__ __align__(16) float c[];
    __shared__ float red[16];
    ple_finish_slice(a, blockIdx.x, a.ple, a.ctx, a.dtok ? *a.dtok : a.tok, c, red);
}

// token z = blockIdx.y of a prompt chunk: its ple and ctx rows are L*pd apart
__global__ __launch_bounds__(256) void ple_finish_rows_kernel(PleArgs a) {
    extern __shared__ __align__(16) float c[];
    __shared__ float red[16];
    const size_t z = blockIdx.y, off = z * (size_t)a.L * a.pd;
    ple_finish_slice(a, blockIdx.x, a.ple + off, a.ctx + off, a.dtok[z], c, red);
}

// o[z][i] = gelu(g[z][i]) * u[z*ustride + i] (main.c:1976-1980, 1989-1993 for
// m rows of d)
__global__ __launch_bounds__(256) void gelu_mul_rows_kernel(float* __restrict__ o, const float* __restrict__ g,
                                                            const float* __restrict__ u, int d, int ustride) {
    const size_t z = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < d) o[z * d + i] = gelu_ref(g[z * d + i]) * u[z * ustride + i];
}

// g = gelu(g) * ple (main.c:1989-1993), then Q8_K of g for the next GEMV
__global__ __launch_bounds__(256) void gelu_mul_quant_kernel(float* __restrict__ g, const float* __restrict__ ple,
                                                             int n, uint8_t* __restrict__ q8) {
    const int lane = threadIdx.x & 63;
    const int nb = n / 256;
    for (int b = threadIdx.x >> 6; b < nb; b += blockDim.x >> 6) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int i = b * 256 + 4 * lane + e;
            const float t = gelu_ref(g[i]);
            v[e] = t * ple[i];
            g[i] = v[e];
        }
        if (q8) quantize_block_wave(v, lane, q8, nb, b);
    }
}

// ---- argmax, first index of the maximum ------------------------------------
// (keys: argmax_key in g4_device.h)
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPer = 4096;   // elements per partial workgroup

__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(const float* __restrict__ v, int n,
                                                                        unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[4];
    constexpr int E = kArgmaxPer / kArgmaxThreads;
    const int base = blockIdx.x * kArgmaxPer, end = min(n, base + kArgmaxPer);
    // every load issued before any waits (clamped indices; the keys past
    // the end are masked to 0, the reduction's start value)
    float x[E];
#pragma unroll
    for (int j = 0; j < E; j++) x[j] = v[min(base + (int)threadIdx.x + kArgmaxThreads * j, end - 1)];
    unsigned long long k = 0;
#pragma unroll
    for (int j = 0; j < E; j++) {
        const int i = base + (int)threadIdx.x + kArgmaxThreads * j;
        const unsigned long long t = argmax_key(x[j], i) & (i < end ? ~0ull : 0ull);
        k = t > k ? t : k;
    }
    k = block_max_u64(k, red);
    if (threadIdx.x == 0) part[blockIdx.x] = k;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(const unsigned long long* __restrict__ part,
                                                                      int np, int* __restrict__ out,
                                                                      int* __restrict__ dtok, int* __restrict__ dpos) {
    __shared__ unsigned long long red[4];
    unsigned long long k = 0;
    for (int i = threadIdx.x; i < np; i += kArgmaxThreads) k = part[i] > k ? part[i] : k;
    k = block_max_u64(k, red);
    if (threadIdx.x == 0) {
        const int idx = (int)(~(uint32_t)(k & 0xffffffffu));
        if (out) *out = idx;
        if (dtok) *dtok = idx;
        if (dpos) *dpos = *dpos + 1;
    }
}

}  // namespace g4

using namespace g4;

// the last pass of the argmax over np per-workgroup keys (the fused
// LM-head kernel's, or argmax_partial_kernel's)
int g4_argmax_final(const void* part, int np, int* out, int* dtok, int* dpos) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, g4_stream(),
                       (const unsigned long long*)part, np, out, dtok, dpos);
    return g4_check_launch("argmax_final_kernel");
}

static bool table_type_ok(int type) {
    return type == G4_F32 || type == G4_F16 || type == G4_BF16 || type == G4_Q4_K || type == G4_Q5_K ||
           type == G4_Q6_K;
}

// hidden_stats (main.c:1813-1826): sum and sum of squares in double, the
// largest |x|; out = (float)sum, (float)sqrt(sum of squares), amax.  The
// double sums are a tree instead of the reference's loop (the same floats
// unless a sum lands within a double rounding of a float boundary).
__global__ __launch_bounds__(256) void hidden_stats_kernel(const float* __restrict__ v, int n, float* __restrict__ out) {
    __shared__ double s1[256], s2[256];
    __shared__ float s3[256];
    const int tid = threadIdx.x;
    double a = 0.0, b = 0.0;
    float m = 0.0f;
    for (int i = tid; i < n; i += 256) {
        const float x = v[i];
        a += (double)x;
        b += (double)x * (double)x;
        const float ax = x >= 0.0f ? x : -x;
        if (ax > m) m = ax;
    }
    s1[tid] = a;
    s2[tid] = b;
    s3[tid] = m;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) {
            s1[tid] += s1[tid + st];
            s2[tid] += s2[tid + st];
            s3[tid] = s3[tid + st] > s3[tid] ? s3[tid + st] : s3[tid];
        }
        __syncthreads();
    }
    if (tid == 0) {
        out[0] = (float)s1[0];
        out[1] = (float)sqrt(s2[0]);
        out[2] = s3[0];
    }
}

extern "C" int g4_hidden_stats(const float* v, int n, float* out) {
    G4_CHECK_ARG(v && out && n > 0, "g4_hidden_stats: bad arguments");
    hipLaunchKernelGGL(hidden_stats_kernel, dim3(1), dim3(256), 0, g4_stream(), v, n, out);
    return g4_check_launch("hidden_stats_kernel");
}

// logits[i] = cap * tanhf(logits[i] * inv), logits_tied's soft-cap (main.c:1789-1795)
__global__ __launch_bounds__(256) void softcap_kernel(float* __restrict__ v, int n, float cap, float inv) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) v[i] = cap * tanhf(v[i] * inv);
}

extern "C" int g4_softcap(float* v, int n, float cap) {
    G4_CHECK_ARG(v && n > 0 && cap > 0.0f, "g4_softcap: bad arguments");
    const float inv = 1.0f / cap;
    hipLaunchKernelGGL(softcap_kernel, dim3((n + 255) / 256), dim3(256), 0, g4_stream(), v, n, cap, inv);
    return g4_check_launch("softcap_kernel");
}

// emb_lookup(float *o, const void *w, int type, int id, int dim), main.c:1696;
// rows = the table's row count (bounds check; the reference trusts id).
extern "C" int g4_emb_lookup(float* o, const void* w, int type, int rows, int id, int dim) {
    G4_CHECK_ARG(o && w && dim > 0 && rows > 0, "g4_emb_lookup: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    G4_CHECK_ARG(id >= 0 && id < rows, "g4_emb_lookup: id %d out of range (%d rows)", id, rows);
    G4_CHECK_ARG(type < G4_Q4_K || type == G4_BF16 || dim % 256 == 0, "g4_emb_lookup: dim %d", dim);
    hipLaunchKernelGGL(emb_lookup_kernel, dim3((dim + 255) / 256), dim3(256), 0, g4_stream(), o, w, type, rows, dim,
                       nullptr, id, 0, 1.0f);
    return g4_check_launch("emb_lookup_kernel");
}

// Engine form: token from device memory, result times `scale` (main.c:1849-1854).
extern "C" int g4_emb_lookup_dev(float* o, const void* w, int type, int rows, const int* dtok, int dim, float scale) {
    G4_CHECK_ARG(o && w && dtok && dim > 0 && rows > 0, "g4_emb_lookup_dev: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    hipLaunchKernelGGL(emb_lookup_kernel, dim3((dim + 255) / 256), dim3(256), 0, g4_stream(), o, w, type, rows, dim,
                       dtok, 0, 1, scale);
    return g4_check_launch("emb_lookup_kernel");
}

extern "C" int g4_emb_lookup_rope(float* o, const void* w, int type, int rows, const int* dtok, int dim, float scale,
                                  const int* dpos, float* tab_a, int n_rot_a, float base_a, const float* ff_a,
                                  float* tab_b, int n_rot_b, float base_b, const float* ff_b, float freq_scale) {
    G4_CHECK_ARG(o && w && dtok && dim > 0 && rows > 0 && dpos, "g4_emb_lookup_rope: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    G4_CHECK_ARG(tab_a && tab_b && n_rot_a > 0 && n_rot_a % 2 == 0 && n_rot_a <= 2048 && n_rot_b > 0 &&
                     n_rot_b % 2 == 0 && n_rot_b <= 2048,
                 "g4_emb_lookup_rope: bad RoPE table arguments");
    const RopeTab ta{(float2*)tab_a, ff_a, powf(base_a, -2.0f / (float)n_rot_a), n_rot_a / 2};
    const RopeTab tb{(float2*)tab_b, ff_b, powf(base_b, -2.0f / (float)n_rot_b), n_rot_b / 2};
    hipLaunchKernelGGL(emb_rope_kernel, dim3((dim + 255) / 256 + 2), dim3(256), 0, g4_stream(), o, w, type, rows, dim,
                       dtok, scale, dpos, freq_scale, ta, tb);
    return g4_check_launch("emb_rope_kernel");
}

extern "C" int g4_emb_lookup_rope_ple(float* o, const void* w, int type, int rows, const int* dtok, int dim,
                                      float scale, const int* dpos, float* tab_a, int n_rot_a, float base_a,
                                      const float* ff_a, float* tab_b, int n_rot_b, float base_b, const float* ff_b,
                                      float freq_scale, float* ctx, const void* w_ctx, int d_ctx, uint32_t* seq) {
    G4_CHECK_ARG(o && w && dtok && dim > 0 && rows > 0 && dpos && ctx && w_ctx && d_ctx > 0,
                 "g4_emb_lookup_rope_ple: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    G4_CHECK_ARG(dim % 8 == 0 && dim <= 4096 && ((uintptr_t)w_ctx & 15) == 0,
                 "g4_emb_lookup_rope_ple: dim=%d (a multiple of 8, <= 4096), w_ctx 16-byte aligned", dim);
    G4_CHECK_ARG(tab_a && tab_b && n_rot_a > 0 && n_rot_a % 2 == 0 && n_rot_a <= 2048 && n_rot_b > 0 &&
                     n_rot_b % 2 == 0 && n_rot_b <= 2048,
                 "g4_emb_lookup_rope_ple: bad RoPE table arguments");
    const RopeTab ta{(float2*)tab_a, ff_a, powf(base_a, -2.0f / (float)n_rot_a), n_rot_a / 2};
    const RopeTab tb{(float2*)tab_b, ff_b, powf(base_b, -2.0f / (float)n_rot_b), n_rot_b / 2};
    // four rows per wave (every workgroup rebuilds x: fewer, larger ones);
    // 16-byte chunks per lane: dim / 512 rounded up
    const size_t lds = (size_t)dim * 4;
    const uint16_t* wp = (const uint16_t*)w_ctx;
    auto go = [&](auto kern, int rpw) {
        hipLaunchKernelGGL(kern, dim3((d_ctx + 4 * rpw - 1) / (4 * rpw) + 2), dim3(256), lds, g4_stream(), o, w, type,
                           rows, dim, dtok, scale, wp, ctx, d_ctx, dpos, freq_scale, ta, tb, seq);
    };
    const int cpl = (dim / 8 + 63) / 64;
    if (cpl <= 4) go(emb_ple_kernel<4, 4>, 4);
    else if (cpl <= 5) go(emb_ple_kernel<4, 5>, 4);
    else go(emb_ple_kernel<2, 8>, 2);
    return g4_check_launch("emb_ple_kernel");
}

extern "C" int g4_ple_finish(float* ple, const float* ctx, const void* ple_tok, int type, int rows, const float* proj_norm,
                             const int* dtok, int tok, int pd, int L, float sc_tok, float sc_ctx, float mix, float eps) {
    G4_CHECK_ARG(ple && ctx && ple_tok && proj_norm && pd > 0 && pd <= 4096 && L > 0, "g4_ple_finish: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    PleArgs a{ple_tok, ctx, proj_norm, ple, dtok, tok, type, rows, pd, L, sc_tok, sc_ctx, mix, eps};
    hipLaunchKernelGGL(ple_finish_kernel, dim3(L), dim3(256), (size_t)pd * 4, g4_stream(), a);
    return g4_check_launch("ple_finish_kernel");
}

extern "C" int g4_emb_lookup_rows(float* o, const void* w, int type, int rows, const int* dtok, int m, int dim,
                                  float scale) {
    G4_CHECK_ARG(o && w && dtok && dim > 0 && rows > 0 && m > 0 && m <= 65535, "g4_emb_lookup_rows: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    hipLaunchKernelGGL(emb_lookup_rows_kernel, dim3((dim + 255) / 256, m), dim3(256), 0, g4_stream(), o, w, type, rows,
                       dim, dtok, scale);
    return g4_check_launch("emb_lookup_rows_kernel");
}

extern "C" int g4_ple_finish_rows(float* ple, const float* ctx, const void* ple_tok, int type, int rows,
                                  const float* proj_norm, const int* dtok, int m, int pd, int L, float sc_tok,
                                  float sc_ctx, float mix, float eps) {
    G4_CHECK_ARG(ple && ctx && ple_tok && proj_norm && dtok && pd > 0 && pd <= 4096 && L > 0 && m > 0 && m <= 65535,
                 "g4_ple_finish_rows: bad arguments");
    G4_CHECK(table_type_ok(type), G4_ERR_TYPE, "Unsupported emb type %d", type);
    PleArgs a{ple_tok, ctx, proj_norm, ple, dtok, 0, type, rows, pd, L, sc_tok, sc_ctx, mix, eps};
    hipLaunchKernelGGL(ple_finish_rows_kernel, dim3(L, m), dim3(256), (size_t)pd * 4, g4_stream(), a);
    return g4_check_launch("ple_finish_rows_kernel");
}

extern "C" int g4_gelu_mul_rows(float* o, const float* g, const float* u, int d, int m, int ustride) {
    G4_CHECK_ARG(o && g && u && d > 0 && m > 0 && m <= 65535 && ustride >= 0, "g4_gelu_mul_rows: bad arguments");
    hipLaunchKernelGGL(gelu_mul_rows_kernel, dim3((d + 255) / 256, m), dim3(256), 0, g4_stream(), o, g, u, d, ustride);
    return g4_check_launch("gelu_mul_rows_kernel");
}

extern "C" int g4_gelu_mul_quant(float* g, const float* ple, int n, void* q8) {
    G4_CHECK_ARG(g && ple && n > 0 && n % 256 == 0, "g4_gelu_mul_quant: n=%d must be a multiple of 256", n);
    hipLaunchKernelGGL(gelu_mul_quant_kernel, dim3(1), dim3(256), 0, g4_stream(), g, ple, n, (uint8_t*)q8);
    return g4_check_launch("gelu_mul_quant_kernel");
}

extern "C" size_t g4_argmax_part_bytes(int n) { return (size_t)((n + kArgmaxPer - 1) / kArgmaxPer) * 8; }

// first index of the maximum of v[0..n) (main.c:2045-2049) -> *out (device
// int); with dtok/dpos (device, nullable) also stores the token as the next
// step's input and advances the position.  part: g4_argmax_part_bytes(n).
extern "C" int g4_argmax(const float* v, int n, int* out, void* part, int* dtok, int* dpos) {
    G4_CHECK_ARG(v && n > 0 && part, "g4_argmax: bad arguments");
    const int np = (n + kArgmaxPer - 1) / kArgmaxPer;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(np), dim3(kArgmaxThreads), 0, g4_stream(), v, n,
                       (unsigned long long*)part);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, g4_stream(),
                       (const unsigned long long*)part, np, out, dtok, dpos);
    return g4_check_launch("argmax kernels");
}

// ---- step scalars -----------------------------------------------------------
__global__ void store_i32x2_kernel(int* __restrict__ dst, int a, int b) {
    if (threadIdx.x == 0) { dst[0] = a; dst[1] = b; }
}

// dst[0] = a, dst[1] = b, ordered on the library stream (no host staging buffer,
// so consecutive calls never race with their own copies)
extern "C" int g4_store_i32x2(int* dst, int a, int b) {
    G4_CHECK_ARG(dst, "g4_store_i32x2: null pointer");
    hipLaunchKernelGGL(store_i32x2_kernel, dim3(1), dim3(64), 0, g4_stream(), dst, a, b);
    return g4_check_launch("store_i32x2_kernel");
}
