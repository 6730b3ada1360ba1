// attn.hip -- Neox RoPE, KV-cache append and ISWA decode attention on gfx950.
//
// Reference (gemma4-4b/cpu-blas/main.c):
//   apply_rope_neox            1725-1745
//   per-head norms, KV append  1886-1904 (K: k_norm, RoPE, store; V: unweighted
//                              norm, store; Q: q_norm, RoPE)
//   attention block            1909-1950: t_start = max(0, pos+1-window) on
//                              sliding-window layers; per head s = scale*K.q,
//                              softmax, o = V^T p; GQA head h reads kv head
//                              h / (n_heads/n_kv); shared-KV layers read the
//                              donor's cache (main.c:743-746).
//
// KV cache in HBM: one buffer per storing layer and per K/V, slot-major
// [slots][kv_stride] fp32.  Full-attention layers use slot = pos; sliding-
// window layers keep a ring of `ring` slots (slot = pos % ring), which holds
// exactly the window the reference reads from its flat cache.
//
// Decode attention is split over the time axis: workgroup (c, kvh) scores one
// chunk of the window for all q heads of kv head kvh (the K/V rows are read
// once for the GQA group), keeps (max, sum, o) of its chunk, and a merge
// kernel combines the chunks by log-sum-exp.  Equal to the reference's
// softmax-then-PV up to fp32 rounding.
#include <mutex>

#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

// ---- RoPE ----------------------------------------------------------------
// Rotate pairs (j, j + hd/2), j < n_rot/2, of one head held in LDS.  The
// angle of pair j is the reference's chain theta_0 = pos, theta_j =
// theta_{j-1} * ts (one rounding per step), angle = (fs * theta_j) / ff[j].
__device__ __forceinline__ void rope_head_lds(float* seg, int hd, int n_rot, int pos, float ts, float fs,
                                              const float* __restrict__ ff) {
    const int half = hd / 2;
    for (int j = threadIdx.x; j < n_rot / 2; j += blockDim.x) {
        float theta = (float)pos;
        for (int i = 0; i < j; i++) theta *= ts;
        const float f = ff ? ff[j] : 1.0f;
        const float angle = (fs * theta) / f;
        const float cr = cosf(angle), ci = sinf(angle);
        const float v0 = seg[j], v1 = seg[j + half];
        seg[j] = v0 * cr - v1 * ci;
        seg[j + half] = v0 * ci + v1 * cr;
    }
}

// rotate with precomputed (cos, sin) of each pair (same values as the chain)
__device__ __forceinline__ void rope_head_lds_tab(float* seg, int hd, int n_rot, const float2* __restrict__ tab) {
    const int half = hd / 2;
    for (int j = threadIdx.x; j < n_rot / 2; j += blockDim.x) {
        const float2 cs = tab[j];
        const float v0 = seg[j], v1 = seg[j + half];
        seg[j] = v0 * cs.x - v1 * cs.y;
        seg[j + half] = v0 * cs.y + v1 * cs.x;
    }
}

// (cos, sin) of the n_rot/2 pair angles at position *dpos (or pos)
__global__ __launch_bounds__(256) void rope_table_kernel(float2* __restrict__ tab, const int* dpos, int pos, int npair,
                                                         float ts, float fs, const float* __restrict__ ff) {
    const int p = dpos ? *dpos : pos;
    for (int j = threadIdx.x; j < npair; j += blockDim.x) tab[j] = rope_pair_cs(p, j, ts, fs, ff);
}

// rows: position pos0 + blockIdx.x -> tab + blockIdx.x * npair
__global__ __launch_bounds__(256) void rope_table_rows_kernel(float2* __restrict__ tab, int pos0, int npair, float ts,
                                                              float fs, const float* __restrict__ ff) {
    const int p = pos0 + blockIdx.x;
    float2* t = tab + (size_t)blockIdx.x * npair;
    for (int j = threadIdx.x; j < npair; j += blockDim.x) t[j] = rope_pair_cs(p, j, ts, fs, ff);
}

__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ vec, int hd, int n_rot, int pos, float ts,
                                                   float fs, const float* __restrict__ ff) {
    extern __shared__ __align__(16) float seg[];
    float* g = vec + (size_t)blockIdx.x * hd;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) seg[i] = g[i];
    __syncthreads();
    rope_head_lds(seg, hd, n_rot, pos, ts, fs, ff);
    __syncthreads();
    for (int i = threadIdx.x; i < hd; i += blockDim.x) g[i] = seg[i];
}

// ---- per-head norms + RoPE + KV append (main.c:1886-1904) -----------------
struct QKVArgs {
    float* q;              // n_heads*hd, normalised and rotated in place
    const float* q_norm;
    const float* k;        // n_kv*hd (nullptr: layer stores no KV)
    const float* v;
    const float* k_norm;
    float* kc;             // slot 0 of this layer's K cache
    float* vc;
    const int* dpos;       // device position (nullptr: use pos)
    const float* ff;       // rope freq factors (nullptr = 1)
    const float2* tab;     // (cos, sin) per pair at this position (nullptr: compute)
    int pos, n_heads, n_kv, hd, n_rot, kv_stride, ring;
    float ts, fs, eps;
};

__device__ __forceinline__ void qkv_post_body(const QKVArgs& a, int b, float* seg, float* red) {
    const int hd = a.hd;
    const int pos = a.dpos ? *a.dpos : a.pos;
    const float* src;
    const float* w;
    int kind;   // 0 = q, 1 = k, 2 = v
    int head;
    if (b < a.n_heads) { kind = 0; head = b; src = a.q + (size_t)head * hd; w = a.q_norm; }
    else if (b < a.n_heads + a.n_kv) { kind = 1; head = b - a.n_heads; src = a.k + (size_t)head * hd; w = a.k_norm; }
    else { kind = 2; head = b - a.n_heads - a.n_kv; src = a.v + (size_t)head * hd; w = nullptr; }

    float ss = 0.0f;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        const float t = src[i];
        seg[i] = t;
        ss += t * t;
    }
    ss = block_sum(ss, red);
    const float s = 1.0f / sqrtf(ss / (float)hd + a.eps);
    for (int i = threadIdx.x; i < hd; i += blockDim.x) seg[i] = w ? seg[i] * (s * w[i]) : seg[i] * s;
    __syncthreads();
    if (kind != 2) {
        if (a.tab) rope_head_lds_tab(seg, hd, a.n_rot, a.tab);
        else rope_head_lds(seg, hd, a.n_rot, pos, a.ts, a.fs, a.ff);
        __syncthreads();
    }
    float* dst;
    if (kind == 0) {
        dst = a.q + (size_t)head * hd;
    } else {
        const int slot = a.ring > 0 ? pos % a.ring : pos;
        dst = (kind == 1 ? a.kc : a.vc) + (size_t)slot * a.kv_stride + (size_t)head * hd;
    }
    for (int i = threadIdx.x; i < hd; i += blockDim.x) dst[i] = seg[i];
}

__global__ __launch_bounds__(256) void qkv_post_kernel(QKVArgs a) {
    extern __shared__ __align__(16) float seg[];
    __shared__ float red[16];
    qkv_post_body(a, blockIdx.x, seg, red);
}

// token z = blockIdx.y of a prompt chunk: q, k, v rows (n_heads*hd, n_kv*hd
// floats apart), K/V stored to row z of the chunk buffers kc/vc (stride
// kv_stride), RoPE pairs from row z of the position table
__global__ __launch_bounds__(256) void qkv_post_rows_kernel(QKVArgs a) {
    extern __shared__ __align__(16) float seg[];
    __shared__ float red[16];
    const size_t z = blockIdx.y;
    a.q += z * (size_t)a.n_heads * a.hd;
    if (a.k) {
        a.k += z * (size_t)a.n_kv * a.hd;
        a.v += z * (size_t)a.n_kv * a.hd;
        a.kc += z * (size_t)a.kv_stride;
        a.vc += z * (size_t)a.kv_stride;
    }
    a.tab += z * (size_t)(a.n_rot / 2);
    qkv_post_body(a, blockIdx.x, seg, red);
}

// The same operations with a RoPE table, one wave per head (hd = 256 K):
// lane l holds dims 256k + 4l .. 256k + 4l + 3, the sum of squares is a wave
// reduction (no LDS, no barrier), and the pair partner of a dim (j and
// j + hd/2, j < n_rot/2) is lane l ^ 32 (hd 256) or the lane's other float4
// (hd 512).  Workgroup (x, z): heads 4x .. 4x + 3 of row z (z > 0: prompt
// chunk rows, as qkv_post_rows_kernel); g4_qkv_post with a table and
// g4_qkv_post_rows both run it, so a chunk row equals the per-token result
// bit for bit.
template <int HD>
__global__ __launch_bounds__(256) void qkv_post_wave_kernel(QKVArgs a) {
    constexpr int K = HD / 256;
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= a.n_heads + (a.k ? 2 * a.n_kv : 0)) return;   // whole waves
    const size_t z = blockIdx.y;
    if (z > 0) {
        a.q += z * (size_t)a.n_heads * HD;
        if (a.k) {
            a.k += z * (size_t)a.n_kv * HD;
            a.v += z * (size_t)a.n_kv * HD;
            a.kc += z * (size_t)a.kv_stride;
            a.vc += z * (size_t)a.kv_stride;
        }
        a.tab += z * (size_t)(a.n_rot / 2);
    }
    const int pos = a.dpos ? *a.dpos : a.pos;
    const float* src;
    const float* w;
    int kind, head;
    if (b < a.n_heads) { kind = 0; head = b; src = a.q + (size_t)head * HD; w = a.q_norm; }
    else if (b < a.n_heads + a.n_kv) { kind = 1; head = b - a.n_heads; src = a.k + (size_t)head * HD; w = a.k_norm; }
    else { kind = 2; head = b - a.n_heads - a.n_kv; src = a.v + (size_t)head * HD; w = nullptr; }

    float x[K][4];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const float4 t = reinterpret_cast<const float4*>(src)[64 * k + lane];
        x[k][0] = t.x; x[k][1] = t.y; x[k][2] = t.z; x[k][3] = t.w;
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) ss += x[k][c] * x[k][c];
    ss = wave_sum(ss);
    const float s = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
    for (int k = 0; k < K; k++) {
        if (w) {
            const float4 wv = reinterpret_cast<const float4*>(w)[64 * k + lane];
            x[k][0] = x[k][0] * (s * wv.x); x[k][1] = x[k][1] * (s * wv.y);
            x[k][2] = x[k][2] * (s * wv.z); x[k][3] = x[k][3] * (s * wv.w);
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) x[k][c] = x[k][c] * s;
        }
    }
    if (kind != 2) {
        // dim e = 256k + 4 lane + c; first half (e < HD/2): j = e, partner
        // e + HD/2; second half: j = e - HD/2, partner e - HD/2
        float y[K][4];
#pragma unroll
        for (int k = 0; k < K; k++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int e = 256 * k + 4 * lane + c;
                const bool first = e < HD / 2;
                const int j = first ? e : e - HD / 2;
                const float vp = K == 1 ? __shfl_xor(x[k][c], 32) : x[k ^ 1][c];
                y[k][c] = x[k][c];
                if (j < a.n_rot / 2) {
                    const float2 cs = a.tab[j];
                    y[k][c] = first ? x[k][c] * cs.x - vp * cs.y : vp * cs.y + x[k][c] * cs.x;
                }
            }
#pragma unroll
        for (int k = 0; k < K; k++)
#pragma unroll
            for (int c = 0; c < 4; c++) x[k][c] = y[k][c];
    }
    float* dst;
    if (kind == 0) {
        dst = a.q + (size_t)head * HD;
    } else {
        const int slot = a.ring > 0 ? pos % a.ring : pos;
        dst = (kind == 1 ? a.kc : a.vc) + (size_t)slot * a.kv_stride + (size_t)head * HD;
    }
#pragma unroll
    for (int k = 0; k < K; k++)
        reinterpret_cast<float4*>(dst)[64 * k + lane] = make_float4(x[k][0], x[k][1], x[k][2], x[k][3]);
}

// the wave form when it applies (hd 256 or 512, a RoPE table, 16-byte rows)
bool qkv_wave_ok(const QKVArgs& a) {
    auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    return (a.hd == 256 || a.hd == 512) && a.tab && al(a.q) && al(a.q_norm) && (!a.k || (al(a.k) && al(a.v) && al(a.k_norm) &&
           al(a.kc) && al(a.vc) && a.kv_stride % 4 == 0));
}

void launch_qkv_wave(const QKVArgs& a, int m) {
    const dim3 grid((a.n_heads + (a.k ? 2 * a.n_kv : 0) + 3) / 4, m);
    if (a.hd == 256) hipLaunchKernelGGL(qkv_post_wave_kernel<256>, grid, dim3(256), 0, g4_stream(), a);
    else hipLaunchKernelGGL(qkv_post_wave_kernel<512>, grid, dim3(256), 0, g4_stream(), a);
}

// rows z of the chunk buffers -> cache slots of positions pos0 + z (a ring
// keeps the last `ring` of them)
__global__ __launch_bounds__(256) void kv_store_rows_kernel(float* __restrict__ kc, float* __restrict__ vc,
                                                            const float* __restrict__ kin, const float* __restrict__ vin,
                                                            int kv_stride, int ring, int pos0, int kvd) {
    const int z = blockIdx.x, pos = pos0 + z;
    const size_t slot = ring > 0 ? pos % ring : pos;
    for (int i = threadIdx.x; i < kvd; i += blockDim.x) {
        kc[slot * kv_stride + i] = kin[(size_t)z * kv_stride + i];
        vc[slot * kv_stride + i] = vin[(size_t)z * kv_stride + i];
    }
}

// ---- split-T decode attention --------------------------------------------
// Workspace (g4_attn_part_bytes): the partials [n_heads][G][hd+2] =
// (o[hd], max, sum) of every chunk.
struct AttnArgs {
    const float* q;        // n_heads*hd
    const float* kc;       // slot 0 of the source layer's cache
    const float* vc;
    const int* dpos;       // device position (nullptr: t_start/nwin below)
    float* part;           // partials
    float* out;            // n_heads*hd
    uint8_t* q8;           // optional Q8_K of out (n_heads*hd/256 blocks)
    int t_start, nwin;     // used when dpos == nullptr
    int window;            // used with dpos: 0 = full attention
    int kv_stride, ring, n_heads, n_kv, hd, G;
    float scale;
    // fused per-head norms, RoPE and KV append (main.c:1886-1904), all
    // optional: q_norm non-null means q is the raw Q projection; kraw
    // non-null means this layer stores K/V: the raw K/V projections of this
    // position are normalised (K also rotated) and written to slot pos of
    // kstore/vstore, and the workgroup whose chunk holds pos uses them
    // directly for that position
    const float* q_norm;
    const float* kraw;
    const float* vraw;
    const float* k_norm;
    float* kstore;
    float* vstore;
    const float2* tab;     // (cos, sin) of each RoPE pair at this position
    int n_rot;
    float eps;
    // query rows of a prompt chunk (qrows > 0, register kernel only): query
    // z = blockIdx.z sits at position p0 + z and sees its own window; K/V of
    // positions >= p0 come from row t - p0 of kchunk/vchunk (stride
    // kv_stride), earlier ones from the cache; q and out rows n_heads*hd
    // apart, partials part_z floats apart, Q8_K rows q8_row bytes apart
    int qrows, p0;
    const float* kchunk;
    const float* vchunk;
    size_t part_z, q8_row;
};

// the query row of this workgroup (qrows > 0): pointers and window
__device__ __forceinline__ void attn_query_row(AttnArgs& a, bool merge) {
    const size_t z = blockIdx.z;
    const size_t qd = (size_t)a.n_heads * a.hd;
    a.q += z * qd;
    a.part += z * a.part_z;
    if (merge) {
        a.out += z * qd;
        if (a.q8) a.q8 += z * a.q8_row;
    }
    const int pos = a.p0 + (int)z;
    a.t_start = a.window > 0 ? max(0, pos + 1 - a.window) : 0;
    a.nwin = pos + 1 - a.t_start;
}

constexpr int kAttnThreads = 256;
constexpr int kChunkMax = 1024;     // positions per workgroup
constexpr int kMaxChunks = 512;     // chunks (workgroups) per kv head

__device__ __forceinline__ void attn_window(const AttnArgs& a, int& t0, int& nwin) {
    if (a.dpos) {
        const int pos = *a.dpos;
        t0 = a.window > 0 ? max(0, pos + 1 - a.window) : 0;
        nwin = pos + 1 - t0;
    } else {
        t0 = a.t_start;
        nwin = a.nwin;
    }
}

__device__ __forceinline__ float dot4(const float4 a, const float4 b, float acc) {
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    return __builtin_fmaf(a.w, b.w, acc);
}

// LDS (floats): [0, R) work region: q [kvm][HD] + scores [kvm][kChunkMax] during
// the scoring, then [4 waves][kvm][HD] for the PV reduction and the merge;
// [R, R + 2*kvm) the chunk's (max, sum) per head.  R = attn_work_floats().
__host__ __device__ inline int attn_work_floats(int hd, int kvm) {
    const int a = kvm * hd + kvm * kChunkMax, b = 4 * kvm * hd;
    return a > b ? a : b;
}

// start of the fused path's K/V staging (16-byte aligned, after (max, sum))
__host__ __device__ inline int attn_new_kv_off(int hd, int kvm) { return (attn_work_floats(hd, kvm) + 2 * kvm + 3) & ~3; }

__device__ __forceinline__ int attn_slot(const AttnArgs& a, int t) { return a.ring > 0 ? t % a.ring : t; }

// Workgroup (c, kvh) scores chunk c of the window for the kvm q heads of kv
// head kvh (each K/V row read once for the group) and keeps (o, max, sum) of
// its chunk; attn_merge_kernel combines the chunks by log-sum-exp.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float sm[];
    constexpr int KPL = HD / 64;          // float4 per lane of a 16-lane row slice
    constexpr int VPL = HD / 256;         // float4 per lane of a 64-lane row slice
    const int c = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x;
    const int kvm = a.n_heads / a.n_kv;
    const int R = attn_work_floats(HD, kvm);
    int t0, nwin;
    attn_window(a, t0, nwin);
    const int cs = (nwin + a.G - 1) / a.G;
    const int cb = t0 + c * cs;
    // the launcher sizes G so that a chunk fits kChunkMax; the clamp only keeps
    // LDS accesses in bounds
    const int cnt = min(kChunkMax, max(0, min(cb + cs, t0 + nwin) - cb));
    float* qs = sm;
    float* sc = sm + kvm * HD;
    float* ml = sm + R;
    float* kn = sm + attn_new_kv_off(HD, kvm);   // this position's K, V (fused append)
    float* vn = kn + HD;
    const int sub = tid >> 4, sl = tid & 15;
    const int wave = tid >> 6, lane = tid & 63;
    const float* kbase = a.kc + (size_t)kvh * HD;
    const float* vbase = a.vc + (size_t)kvh * HD;
    const int pos = t0 + nwin - 1;
    const int tl = pos - cb;                              // pos inside this chunk
    const bool owner = a.kraw != nullptr && cnt > 0 && tl >= 0 && tl < cnt;
    // cache slot of chunk position i (one modulo per workgroup: the chunk is
    // shorter than the ring, so it wraps at most once)
    const int s0 = attn_slot(a, cb);
    auto slot_of = [&](int i) {
        const int sl_ = s0 + i;
        return (a.ring > 0 && sl_ >= a.ring) ? sl_ - a.ring : sl_;
    };
    // K rows of positions it+sub, it+16+sub (phase 1) and V rows of positions
    // it+wave+4u (phase 3); the first ones are issued before q is staged
    float4 ka[KPL], kb[KPL];
    auto load_k = [&](int it) {
        const float4* ra = reinterpret_cast<const float4*>(kbase + (size_t)slot_of(min(it + sub, cnt - 1)) * a.kv_stride);
        const float4* rb = reinterpret_cast<const float4*>(kbase + (size_t)slot_of(min(it + 16 + sub, cnt - 1)) * a.kv_stride);
#pragma unroll
        for (int k = 0; k < KPL; k++) ka[k] = ra[sl + 16 * k];
#pragma unroll
        for (int k = 0; k < KPL; k++) kb[k] = rb[sl + 16 * k];
    };
    constexpr int VU = 8;                 // V rows in flight per wave
    float4 vv[VU][VPL];
    auto load_v = [&](int it) {
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = min(it + wave + 4 * u, cnt - 1);
            const float4* vr = reinterpret_cast<const float4*>(vbase + (size_t)slot_of(t) * a.kv_stride);
#pragma unroll
            for (int k = 0; k < VPL; k++) vv[u][k] = vr[lane + 64 * k];
        }
    };
    if (cnt > 0) {
        load_k(0);
        load_v(0);
    }
    // norm weights of this lane's elements and the RoPE pair of this thread,
    // also issued before anything waits (np = n_rot/2 divides 256)
    const bool fuse = a.q_norm != nullptr;
    const int np = fuse ? a.n_rot / 2 : 1, per = kAttnThreads / np;
    float wq[HD / 64], wk[HD / 64];
    float2 cs2 = make_float2(1.0f, 0.0f);
    if (fuse) {
#pragma unroll
        for (int e = 0; e < HD / 64; e++) {
            wq[e] = a.q_norm[lane + 64 * e];
            wk[e] = owner ? a.k_norm[lane + 64 * e] : 0.0f;
        }
        if (tid < per * np) cs2 = a.tab[tid % np];
    }
    const float* qsrc = a.q + (size_t)kvh * kvm * HD;
    for (int i = tid; i < kvm * HD; i += kAttnThreads) qs[i] = qsrc[i];
    if (owner) {
        for (int i = tid; i < HD; i += kAttnThreads) {
            kn[i] = a.kraw[(size_t)kvh * HD + i];
            vn[i] = a.vraw[(size_t)kvh * HD + i];
        }
    }
    __syncthreads();
    if (fuse) {
        // rmsnorm_head_inplace (q: q_norm, k: k_norm) / _noweight (v), one
        // wave per head vector: seg *= s * w with s = 1/sqrt(mean(seg^2)+eps)
        const int nvec = kvm + (owner ? 2 : 0);
        for (int vi = wave; vi < nvec; vi += kAttnThreads / 64) {
            float* seg = vi < kvm ? qs + vi * HD : (vi == kvm ? kn : vn);
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < HD / 64; e++) {
                const float t = seg[lane + 64 * e];
                ss += t * t;
            }
            ss = wave_sum(ss);
            const float sf = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
            for (int e = 0; e < HD / 64; e++) {
                const int i = lane + 64 * e;
                seg[i] = vi < kvm ? seg[i] * (sf * wq[e]) : vi == kvm ? seg[i] * (sf * wk[e]) : seg[i] * sf;
            }
        }
        __syncthreads();
        // RoPE (apply_rope_neox) of the q heads and k: pair j = tid % np of
        // vectors tid / np, + per, ...
        if (tid < per * np) {
            const int j = tid % np, nv = kvm + (owner ? 1 : 0);
            for (int vi = tid / np; vi < nv; vi += per) {
                float* seg = vi < kvm ? qs + vi * HD : kn;
                const float v0 = seg[j], v1 = seg[j + HD / 2];
                seg[j] = v0 * cs2.x - v1 * cs2.y;
                seg[j + HD / 2] = v0 * cs2.y + v1 * cs2.x;
            }
        }
        __syncthreads();
    }
    if (owner) {
        const size_t off = (size_t)attn_slot(a, pos) * a.kv_stride + (size_t)kvh * HD;
        for (int i = tid; i < HD; i += kAttnThreads) {
            a.kstore[off + i] = kn[i];
            a.vstore[off + i] = vn[i];
        }
    }

    // phase 1: scores; 16 subgroups of 16 lanes, two positions per subgroup
    for (int it = 0; it < cnt; it += 32) {
        if (it > 0) load_k(it);
        const int ta = it + sub, tb = it + 16 + sub;
        if (owner && (ta == tl || tb == tl)) {
            // this position's K is not in the cache yet: take it from LDS
            const float4* kr = reinterpret_cast<const float4*>(kn);
#pragma unroll
            for (int k = 0; k < KPL; k++) {
                if (ta == tl) ka[k] = kr[sl + 16 * k];
                else kb[k] = kr[sl + 16 * k];
            }
        }
        for (int h = 0; h < kvm; h++) {
            const float4* qh = reinterpret_cast<const float4*>(qs + h * HD);
            float da = 0.0f, db = 0.0f;
#pragma unroll
            for (int k = 0; k < KPL; k++) {
                const float4 qv = qh[sl + 16 * k];
                da = dot4(ka[k], qv, da);
                db = dot4(kb[k], qv, db);
            }
            // sum over the 16 lanes of the row (DPP; the xor-8..1 butterfly's bits)
            da += dpp_f<kDppXor1>(da);
            db += dpp_f<kDppXor1>(db);
            da += dpp_f<kDppXor2>(da);
            db += dpp_f<kDppXor2>(db);
            da += dpp_f<kDppHalfMirror>(da);
            db += dpp_f<kDppHalfMirror>(db);
            da += dpp_f<kDppMirror>(da);
            db += dpp_f<kDppMirror>(db);
            if (sl == 0) {
                if (ta < cnt) sc[h * kChunkMax + ta] = a.scale * da;
                if (tb < cnt) sc[h * kChunkMax + tb] = a.scale * db;
            }
        }
    }
    __syncthreads();

    // phase 2: chunk max / exp / sum per head (one wave per head)
    for (int h = wave; h < kvm; h += kAttnThreads / 64) {
        float* s = sc + h * kChunkMax;
        float m = -INFINITY;
        for (int t = lane; t < cnt; t += 64) m = fmaxf(m, s[t]);
        m = wave_max(m);
        float l = 0.0f;
        for (int t = lane; t < cnt; t += 64) {
            const float e = expf(s[t] - m);
            s[t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) { ml[2 * h] = m; ml[2 * h + 1] = l; }
    }
    __syncthreads();

    // phase 3: o[h] = sum_t p[h][t] V[t]; wave w takes positions w, w+4, ...,
    // VU rows in flight per wave
    float4 acc[8][VPL];
#pragma unroll
    for (int h = 0; h < 8; h++)
#pragma unroll
        for (int k = 0; k < VPL; k++) acc[h][k] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int it = 0; it < cnt; it += 4 * VU) {
        if (it > 0) load_v(it);
        if (owner) {
#pragma unroll
            for (int u = 0; u < VU; u++) {
                if (it + wave + 4 * u == tl) {
#pragma unroll
                    for (int k = 0; k < VPL; k++) vv[u][k] = reinterpret_cast<const float4*>(vn)[lane + 64 * k];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int t = it + wave + 4 * u;
            if (t < cnt) {
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    if (h < kvm) {
                        const float p = sc[h * kChunkMax + t];
#pragma unroll
                        for (int k = 0; k < VPL; k++) {
                            acc[h][k].x = __builtin_fmaf(p, vv[u][k].x, acc[h][k].x);
                            acc[h][k].y = __builtin_fmaf(p, vv[u][k].y, acc[h][k].y);
                            acc[h][k].z = __builtin_fmaf(p, vv[u][k].z, acc[h][k].z);
                            acc[h][k].w = __builtin_fmaf(p, vv[u][k].w, acc[h][k].w);
                        }
                    }
                }
            }
        }
    }
    __syncthreads();   // scores are dead; the work region becomes [4][kvm][HD]
    float* rs = sm;
#pragma unroll
    for (int h = 0; h < 8; h++) {
        if (h < kvm) {
#pragma unroll
            for (int k = 0; k < VPL; k++)
                reinterpret_cast<float4*>(rs + ((size_t)wave * kvm + h) * HD)[lane + 64 * k] = acc[h][k];
        }
    }
    __syncthreads();
    for (int i = tid; i < kvm * HD; i += kAttnThreads) {
        const int h = i / HD, dd = i - h * HD;
        float o = 0.0f;
        for (int w = 0; w < kAttnThreads / 64; w++) o += rs[((size_t)w * kvm + h) * HD + dd];
        float* p = a.part + ((size_t)(kvh * kvm + h) * a.G + c) * (HD + 2);
        p[dd] = o;
        if (dd == 0) { p[HD] = cnt > 0 ? ml[2 * h] : -INFINITY; p[HD + 1] = cnt > 0 ? ml[2 * h + 1] : 0.0f; }
    }

}

// ---- register-resident chunk kernel ---------------------------------------
// Same partials as attn_decode_kernel, computed without LDS round trips
// between the phases.  Every wave holds its vectors in the HVec layout (lane
// l: elements W*l .. W*l+W-1 and their RoPE partners HD/2 further), so
//  - each wave loads and normalises all KVM q heads itself (a wave sum per
//    head) and rotates them in registers, with no lane exchanges;
//  - a round gives each wave PPW positions; its PPW x KVM partial dot
//    products are summed over the wave by a transposed butterfly: each
//    exchange step over a lane bit halves the number of values a lane
//    carries (in-row DPP steps first, while there are many values, the two
//    cross-row steps last), so that score j = h*PPW + p ends in the lanes
//    whose bits 3, 2, 1, 0, 4 (in that order, most significant first) spell
//    j, and head h's scores fill the lanes whose leading bits spell h;
//  - the chunk's online softmax (max, exp, sum) reduces over those lanes,
//    and o_h += p * V_p takes each p by a readlane (an SGPR operand);
//  - the four waves' (max, sum, o) are combined once through LDS.
// The fused K/V append is computed by every wave of the owner workgroup;
// the wave whose round holds position pos uses it in place of the (stale)
// cache row, and wave 0 stores it.
// On a sliding-window layer whose ring holds exactly the window, chunk c
// takes fixed ring slots, so its K/V loads do not wait for the position:
// the softmax does not depend on the order of the positions, and a slot is
// valid once the ring is full (pos >= ring-1) or if it does not exceed pos.
template <int M>
__device__ __forceinline__ float lane_xchg(float x) {   // partner lane across lane bit M
    if constexpr (M >= 16) return __shfl_xor(x, M, 64);
    else if constexpr (M == 8) return dpp_f<kDppMirror>(x);
    else if constexpr (M == 4) return dpp_f<kDppHalfMirror>(x);
    else if constexpr (M == 2) return dpp_f<kDppXor2>(x);
    else return dpp_f<kDppXor1>(x);
}

// lane bits in the order the transposed butterfly consumes them
__host__ __device__ constexpr int xbit(int k) { return k == 0 ? 8 : k == 1 ? 4 : k == 2 ? 2 : k == 3 ? 1 : k == 4 ? 16 : 32; }

// lane holding score j of an nb-bit index (free bits zero)
__host__ __device__ constexpr int xlane(int j, int nb) {
    int l = 0;
    for (int k = 0; k < nb; k++) l |= ((j >> (nb - 1 - k)) & 1) ? xbit(k) : 0;
    return l;
}
__host__ __device__ constexpr int xfree(int nb) {   // lane bits not part of the index
    int m = 0;
    for (int k = nb; k < 6; k++) m |= xbit(k);
    return m;
}

// step K of the butterfly on N values (N == 1: plain all-reduce steps)
template <int K, int N>
__device__ __forceinline__ float xpose_sum_step(float (&v)[32], int lane) {
    if constexpr (K >= 6) {
        return v[0];
    } else if constexpr (N == 1) {
        v[0] += lane_xchg<xbit(K)>(v[0]);
        return xpose_sum_step<K + 1, 1>(v, lane);
    } else {
        const bool up = (lane & xbit(K)) != 0;
#pragma unroll
        for (int i = 0; i < N / 2; i++) {
            const float a = v[i], b = v[i + N / 2];
            v[i] = (up ? b : a) + lane_xchg<xbit(K)>(up ? a : b);
        }
        return xpose_sum_step<K + 1, N / 2>(v, lane);
    }
}

// max / sum over the lanes that share index bits 0..K0-1 (steps K0..5)
template <int K>
__device__ __forceinline__ float group_max(float x) {
    if constexpr (K < 6) return group_max<K + 1>(fmaxf(x, lane_xchg<xbit(K)>(x)));
    else return x;
}
template <int K>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (K < 6) return group_sum<K + 1>(x + lane_xchg<xbit(K)>(x));
    else return x;
}

// A head vector as one lane holds it: elements W*l .. W*l+W-1 and, HD/2
// further, their RoPE partners (W = HD/128: a float2 or float4 load per
// half, 512 B or 1 KB per wave instruction).
template <int HD>
struct HVec {
    static constexpr int W = HD / 128;
    float v[2][W];
    __device__ __forceinline__ void load(const float* __restrict__ p, int lane) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            if constexpr (W == 2) {
                const float2 t = reinterpret_cast<const float2*>(p)[64 * k + lane];
                v[k][0] = t.x; v[k][1] = t.y;
            } else {
                const float4 t = reinterpret_cast<const float4*>(p)[64 * k + lane];
                v[k][0] = t.x; v[k][1] = t.y; v[k][2] = t.z; v[k][3] = t.w;
            }
        }
    }
    __device__ __forceinline__ void store(float* p, int lane) const {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            if constexpr (W == 2) reinterpret_cast<float2*>(p)[64 * k + lane] = make_float2(v[k][0], v[k][1]);
            else reinterpret_cast<float4*>(p)[64 * k + lane] = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
        }
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int w = 0; w < W; w++) v[k][w] = 0.0f;
    }
};

template <int HD>
__device__ __forceinline__ float hdot(const HVec<HD>& a, const HVec<HD>& b, float acc) {
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int w = 0; w < HD / 128; w++) acc = __builtin_fmaf(a.v[k][w], b.v[k][w], acc);
    return acc;
}

// rmsnorm_head_inplace (w) / rmsnorm_head_noweight_inplace (w == null) of
// one head vector: x * (s * w) or x * s, s = 1/sqrt(mean(x^2) + eps)
template <int HD>
__device__ __forceinline__ void norm_vec(HVec<HD>& x, const HVec<HD>* w, float eps) {
    float ss = hdot(x, x, 0.0f);
    ss = wave_sum(ss);
    const float s = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
        for (int i = 0; i < HD / 128; i++) x.v[k][i] = w ? x.v[k][i] * (s * w->v[k][i]) : x.v[k][i] * s;
}

// Neox rotation of pairs (j, j + HD/2), j = W*lane + i < n_rot/2, both in
// this lane; cs[i] = (cos, sin) of pair j
template <int HD>
__device__ __forceinline__ void rope_vec(HVec<HD>& x, const float2 (&cs)[HD / 128], int lane, int n_rot) {
#pragma unroll
    for (int i = 0; i < HD / 128; i++) {
        if ((HD / 128) * lane + i < n_rot / 2) {
            const float v0 = x.v[0][i], v1 = x.v[1][i];
            x.v[0][i] = v0 * cs[i].x - v1 * cs[i].y;
            x.v[1][i] = v0 * cs[i].y + v1 * cs[i].x;
        }
    }
}

template <int HD, int KVM>
__host__ __device__ constexpr int chunk_ppw() {   // positions per wave per round
    return (HD == 256 ? 8 : 4) < 32 / KVM ? (HD == 256 ? 8 : 4) : 32 / KVM;
}

__host__ __device__ inline size_t attn_chunk_lds(int hd, int kvm_pow2, int nw = kAttnThreads / 64) {
    return (size_t)nw * kvm_pow2 * (hd + 2) * 4;
}

// DB: two register sets, round r + 1's rows loading while round r is
// reduced (decode: few workgroups, each one's latency counts); without it
// the register count allows twice the workgroups per CU (prompt-chunk rows:
// thousands of workgroups, occupancy counts)
// FZ: 0 the fused norms decided at run time (a.q_norm), 1 fused (known at
// compile time: the SPL form below), 2 not fused
template <int HD, int KVM, bool DB, int NTH = kAttnThreads, int PPW_ = 0, int FZ = 0>
__global__ __launch_bounds__(NTH) void attn_chunk_kernel(AttnArgs a) {
    if (a.qrows) attn_query_row(a, false);
    constexpr int W = HD / 128;
    constexpr int NW = NTH / 64;
    constexpr int PPW = PPW_ ? PPW_ : chunk_ppw<HD, KVM>();
    constexpr int V = PPW * KVM;                  // score values per wave and round
    constexpr int LV = V == 32 ? 5 : V == 16 ? 4 : V == 8 ? 3 : V == 4 ? 2 : V == 2 ? 1 : 0;
    constexpr int LK = KVM == 8 ? 3 : KVM == 4 ? 2 : KVM == 2 ? 1 : 0;
    static_assert(V <= 32 && (1 << LV) == V, "score values per round");
    extern __shared__ __align__(16) float sm[];   // [NW][KVM][HD] o, then [NW][KVM] (max, sum)
    const int c = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvm = a.n_heads / a.n_kv;
    const bool fuse = FZ == 1 || (FZ == 0 && a.q_norm != nullptr);
    const bool append = fuse && a.kraw != nullptr;

    // q heads of this kv head (heads past kvm repeat the last one; unused),
    // the norm weights, the RoPE pairs and the raw K/V of this position:
    // issued first, so their arithmetic waits only for them.  SPL (fused, a
    // wave for each vector): wave w < KVM takes q head w, wave KVM this
    // position's K, wave KVM + 1 its V; each normalises (and rotates) its
    // vector alone and every wave reads all of them back from LDS, instead of
    // every wave repeating the KVM + 2 norms
    constexpr bool SPL = FZ == 1 && NW >= KVM + 2;
    HVec<HD> q[KVM];
    HVec<HD> wq, wk, kn, vn, mine, wmine;
    float2 rc[W];
    const int wvu = __builtin_amdgcn_readfirstlane(wave);   // the wave index as a scalar
    if (SPL && fuse) {
        // every wave loads one vector and one weight vector (no load under a
        // condition: the pointers are selected per wave)
        const bool kv_wave = append && (wvu == KVM || wvu == KVM + 1);
        const float* src = wvu < KVM ? a.q + (size_t)(kvh * kvm + min(wvu, kvm - 1)) * HD
                           : kv_wave ? (wvu == KVM ? a.kraw : a.vraw) + (size_t)kvh * HD
                                     : a.q;
        mine.load(src, lane);
        wmine.load(wvu == KVM && append ? a.k_norm : a.q_norm, lane);
#pragma unroll
        for (int i = 0; i < W; i++) rc[i] = a.tab[min(W * lane + i, a.n_rot / 2 - 1)];
    } else {
#pragma unroll
        for (int h = 0; h < KVM; h++) q[h].load(a.q + (size_t)(kvh * kvm + min(h, kvm - 1)) * HD, lane);
    }
    if (!SPL && fuse) {
        wq.load(a.q_norm, lane);
#pragma unroll
        // every lane loads a pair (clamped: n_rot >= 2 is checked at
        // launch; rope_vec leaves pairs past n_rot/2 alone): a load under a
        // lane condition is followed by a wait for every load issued
        // before it
        for (int i = 0; i < W; i++) rc[i] = a.tab[min(W * lane + i, a.n_rot / 2 - 1)];
        if (append) {
            wk.load(a.k_norm, lane);
            kn.load(a.kraw + (size_t)kvh * HD, lane);
            vn.load(a.vraw + (size_t)kvh * HD, lane);
        }
    }

    // the chunk: cnt cache slots from slot s0 (wrapping once at the ring end)
    const bool slotm = a.dpos != nullptr && a.ring > 0 && a.window == a.ring;
    int cnt, s0, t0 = 0, nwin = 0, cb = 0;
    if (slotm) {
        const int css = (a.ring + a.G - 1) / a.G;
        s0 = c * css;
        cnt = max(0, min(css, a.ring - s0));
    } else {
        attn_window(a, t0, nwin);
        const int cs = (nwin + a.G - 1) / a.G;
        cb = t0 + c * cs;
        // the launcher sizes G so that a chunk fits kChunkMax; the clamp only
        // keeps the loads in bounds
        cnt = min(kChunkMax, max(0, min(cb + cs, t0 + nwin) - cb));
        s0 = attn_slot(a, cb);
    }
    auto slot_of = [&](int i) {
        const int sl = s0 + i;
        return (a.ring > 0 && sl >= a.ring) ? sl - a.ring : sl;
    };
    const float* kbase = a.kc + (size_t)kvh * HD;
    const float* vbase = a.vc + (size_t)kvh * HD;
    HVec<HD> kr[PPW], vr[PPW], kr2[DB ? PPW : 1], vr2[DB ? PPW : 1];
    // an empty chunk (cnt 0) loads one row it will not use, in bounds: slot 0
    // of a ring, else the window's last position (so the first round's loads
    // are issued unconditionally: behind a branch the compiler made the
    // norms below wait for them)
    const int t_last = t0 + max(nwin, 1) - 1;
    auto load_kv = [&](HVec<HD>* K, HVec<HD>* Vv, int r) {
#pragma unroll
        for (int p = 0; p < PPW; p++) {
            const int i = min(r * NW * PPW + wave * PPW + p, max(cnt - 1, 0));
            const int t = cnt > 0 ? cb + i : t_last;   // position (position mode; prompt-chunk rows only)
            if (a.kchunk && t >= a.p0) {
                const size_t off = (size_t)(t - a.p0) * a.kv_stride + (size_t)kvh * HD;
                K[p].load(a.kchunk + off, lane);
                Vv[p].load(a.vchunk + off, lane);
            } else {
                const int sl = cnt > 0 ? slot_of(i) : slotm ? 0 : attn_slot(a, t_last);
                K[p].load(kbase + (size_t)sl * a.kv_stride, lane);
                Vv[p].load(vbase + (size_t)sl * a.kv_stride, lane);
            }
        }
    };
    load_kv(kr, vr, 0);
    // the position (slot mode: not needed by the loads above)
    const int dpv = slotm ? *a.dpos : 0;
    __builtin_amdgcn_sched_barrier(0);   // the loads are in flight before anything waits

    // per-head norms and RoPE (q; this position's K and V, whichever
    // workgroup turns out to own the position)
    if (SPL && fuse) {
        __shared__ __align__(16) float stg[SPL ? (KVM + 2) * HD : 1];
        if (wvu < KVM || (append && wvu < KVM + 2)) {
            const bool isv = wvu == KVM + 1;
            norm_vec<HD>(mine, isv ? nullptr : &wmine, a.eps);
            if (!isv) rope_vec<HD>(mine, rc, lane, a.n_rot);
            mine.store(stg + wvu * HD, lane);
        }
        lds_sync();
#pragma unroll
        for (int h = 0; h < KVM; h++) q[h].load(stg + h * HD, lane);
        if (append) {
            kn.load(stg + KVM * HD, lane);
            vn.load(stg + (KVM + 1) * HD, lane);
        }
    } else if (fuse) {
#pragma unroll
        for (int h = 0; h < KVM; h++) {
            norm_vec<HD>(q[h], &wq, a.eps);
            rope_vec<HD>(q[h], rc, lane, a.n_rot);
        }
        if (append) {
            norm_vec<HD>(kn, &wk, a.eps);
            rope_vec<HD>(kn, rc, lane, a.n_rot);
            norm_vec<HD>(vn, nullptr, a.eps);
        }
    }

    // valid positions: a prefix of nvalid chunk entries; tl = this
    // position's entry
    int nvalid, tl, pos;
    if (slotm) {
        pos = dpv;
        nvalid = pos >= a.ring - 1 ? cnt : min(cnt, max(0, pos + 1 - s0));
        tl = pos % a.ring - s0;
    } else {
        nvalid = cnt;
        pos = t0 + nwin - 1;
        tl = pos - cb;
    }
    const bool owner = append && tl >= 0 && tl < nvalid;
    if (owner && wave == 0) {
        const size_t off = (size_t)attn_slot(a, pos) * a.kv_stride + (size_t)kvh * HD;
        kn.store(a.kstore + off, lane);
        vn.store(a.vstore + off, lane);
    }

    // per-head online softmax state of this wave (m, l uniform over the
    // head's lanes; o in every lane)
    float m = -INFINITY, l = 0.0f;
    HVec<HD> o[KVM];
#pragma unroll
    for (int h = 0; h < KVM; h++) o[h].zero();
    const int nrounds = (nvalid + NW * PPW - 1) / (NW * PPW);
    int jl = 0;                                   // score index this lane ends with
#pragma unroll
    for (int k = 0; k < LV; k++) jl |= ((lane & xbit(k)) ? 1 : 0) << (LV - 1 - k);
    const int hl = jl / PPW, pl = jl - hl * PPW;
    const bool counted = (lane & xfree(LV)) == 0;   // one lane of each score's copies
    auto round = [&](HVec<HD>* kr, HVec<HD>* vr, int r) {
        const int base = r * NW * PPW + wave * PPW;
        if (owner && tl >= base && tl < base + PPW) {
#pragma unroll
            for (int p = 0; p < PPW; p++)
                if (base + p == tl) {
                    kr[p] = kn;
                    vr[p] = vn;
                }
        }
        float sv[32];
#pragma unroll
        for (int h = 0; h < KVM; h++)
#pragma unroll
            for (int p = 0; p < PPW; p++) sv[h * PPW + p] = hdot(kr[p], q[h], 0.0f);
        const float sraw = xpose_sum_step<0, V>(sv, lane);
        const bool valid = base + pl < nvalid && hl < kvm;
        const float sc = valid ? a.scale * sraw : -INFINITY;
        const float mn = fmaxf(m, group_max<LK>(sc));
        const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
        const float pv = valid ? expf(sc - mn) : 0.0f;
        l = l * alpha + group_sum<LK>(counted ? pv : 0.0f);
        m = mn;
#pragma unroll
        for (int h = 0; h < KVM; h++) {
            const float ah = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), xlane(h, LK)));
#pragma unroll
            for (int k = 0; k < 2; k++)
#pragma unroll
                for (int i = 0; i < W; i++) o[h].v[k][i] *= ah;
#pragma unroll
            for (int p = 0; p < PPW; p++) {
                // entries past nvalid were loaded before the position was
                // known (ring slots no position has written yet may hold any
                // bits): their weight is 0, but 0 * NaN is not, so skip them
                if (base + p >= nvalid) continue;
                const float ph = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), xlane(h * PPW + p, LV)));
#pragma unroll
                for (int k = 0; k < 2; k++)
#pragma unroll
                    for (int i = 0; i < W; i++) o[h].v[k][i] = __builtin_fmaf(ph, vr[p].v[k][i], o[h].v[k][i]);
            }
        }
    };
    // rounds in pairs over the two register sets; the next round's loads
    // are issued unconditionally (a clamped round past the last one reloads
    // rows already in cache) so that no branch separates them from their use
    if (!DB) {
        for (int r = 0; r < nrounds; r++) {
            if (r > 0) load_kv(kr, vr, r);
            round(kr, vr, r);
        }
    } else if (nrounds == 1) {
        round(kr, vr, 0);                         // one round (sliding windows): no second set
    } else {
        for (int r = 0; r < nrounds; r += 2) {
            load_kv(kr2, vr2, min(r + 1, nrounds - 1));
            round(kr, vr, r);
            load_kv(kr, vr, min(r + 2, nrounds - 1));
            if (r + 1 < nrounds) round(kr2, vr2, r + 1);
        }
    }

    // combine the waves: LDS [NW][KVM][HD] o and [NW][KVM] (max, sum)
    float* so = sm;
    float* sml = sm + NW * KVM * HD;
#pragma unroll
    for (int h = 0; h < KVM; h++) {
        o[h].store(so + (size_t)(wave * KVM + h) * HD, lane);
        if (lane == xlane(h, LK)) {
            sml[2 * (wave * KVM + h)] = m;
            sml[2 * (wave * KVM + h) + 1] = l;
        }
    }
    __syncthreads();
    // a thread per (head, 4 dims): the waves' weights exp(m_w - M) once,
    // then its dims (the partial rows are 8-byte aligned: float2 stores)
    constexpr int Q4 = HD / 4;
    for (int i = tid; i < kvm * Q4; i += NTH) {
        const int h = i / Q4, d4 = i - h * Q4;
        float mw[NW], M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            mw[w] = sml[2 * (w * KVM + h)];
            M = fmaxf(M, mw[w]);
        }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = mw[w] == -INFINITY ? 0.0f : expf(mw[w] - M);
            const float4 ow = reinterpret_cast<const float4*>(so + (size_t)(w * KVM + h) * HD)[d4];
            acc.x = __builtin_fmaf(f, ow.x, acc.x);
            acc.y = __builtin_fmaf(f, ow.y, acc.y);
            acc.z = __builtin_fmaf(f, ow.z, acc.z);
            acc.w = __builtin_fmaf(f, ow.w, acc.w);
            L = __builtin_fmaf(f, sml[2 * (w * KVM + h) + 1], L);
        }
        float* pp = a.part + ((size_t)(kvh * kvm + h) * a.G + c) * (HD + 2);
        reinterpret_cast<float2*>(pp)[2 * d4] = make_float2(acc.x, acc.y);
        reinterpret_cast<float2*>(pp)[2 * d4 + 1] = make_float2(acc.z, acc.w);
        if (d4 == 0) {
            pp[HD] = M;
            pp[HD + 1] = L;
        }
    }
}

// Merge of the G chunk partials of one q head: workgroup (h, slice) owns
// 256 output dims.  Every load is issued first: each thread's dim of the
// first MR chunks and the (max, sum) of the chunks it reduces; then
// the chunk weights f_g = exp(max_g - M) and the total L = sum_g sum_g f_g
// (through LDS), the thread's dim over the chunks (the rest of them, if G
// is larger, streamed eight at a time) and, if asked, the Q8_K block of the
// workgroup's 256 outputs.
// MR chunk rows per thread are loaded at once (clamped indices: loads under
// a condition would wait for everything issued before them); the launcher
// picks MR >= G up to 128.
template <int HD, int MR>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    if (a.qrows) attn_query_row(a, true);
    __shared__ float fw[kMaxChunks];
    __shared__ float red[16];
    __shared__ __align__(16) float mo[256];
    const int h = blockIdx.x, slice = blockIdx.y, tid = threadIdx.x;
    const int G = a.G;
    const float* ph = a.part + (size_t)h * G * (HD + 2);
    const int dd = slice * 256 + tid;
    const float* pd = ph + dd;
    float v[MR];
#pragma unroll
    for (int u = 0; u < MR; u++) v[u] = pd[(size_t)min(u, G - 1) * (HD + 2)];
    float mg[kMaxChunks / 256], lg[kMaxChunks / 256];
#pragma unroll
    for (int k = 0; k < kMaxChunks / 256; k++) {
        const int g = tid + 256 * k;
        mg[k] = g < G ? ph[(size_t)g * (HD + 2) + HD] : -INFINITY;
        lg[k] = g < G ? ph[(size_t)g * (HD + 2) + HD + 1] : 0.0f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMaxChunks / 256; k++) M = fmaxf(M, mg[k]);
    M = wave_max(M);
    if ((tid & 63) == 0) red[tid >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float L = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxChunks / 256; k++) {
        const int g = tid + 256 * k;
        if (g < G) {
            const float f = lg[k] > 0.0f ? expf(mg[k] - M) : 0.0f;
            fw[g] = f;
            L += lg[k] * f;
        }
    }
    L = block_sum(L, red + 4);   // its barrier also publishes fw
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < MR; u++)
        if (u < G) o = __builtin_fmaf(v[u], fw[u], o);
    int g = MR;
    for (; g + 8 <= G; g += 8) {
        float w8[8];
#pragma unroll
        for (int u = 0; u < 8; u++) w8[u] = pd[(size_t)(g + u) * (HD + 2)];
#pragma unroll
        for (int u = 0; u < 8; u++) o = __builtin_fmaf(w8[u], fw[g + u], o);
    }
    for (; g < G; g++) o = __builtin_fmaf(pd[(size_t)g * (HD + 2)], fw[g], o);
    const float r = L > 0.0f ? o / L : 0.0f;
    a.out[(size_t)h * HD + dd] = r;
    if (a.q8) {
        mo[tid] = r;
        __syncthreads();
        if (tid < 64) {
            const float4 f4 = reinterpret_cast<const float4*>(mo)[tid];
            const float v4[4] = {f4.x, f4.y, f4.z, f4.w};
            quantize_block_wave(v4, tid, a.q8, a.n_heads * HD / 256, h * (HD / 256) + slice);
        }
    }
}

// The same merge for 32 < G <= 128 with 1024 threads: thread (c, dim), c =
// tid / 256, takes chunks c, c + 4, ..., so a workgroup has four times the
// loads of the 256-thread form in flight (32 a thread, all issued first, on
// clamped indices); the four chunk groups' sums are added through LDS in a
// fixed order.  The barriers wait for LDS only, so the partial loads stay in
// flight while the chunk weights are formed.
template <int HD>
__global__ __launch_bounds__(1024) void attn_merge_wide_kernel(AttnArgs a) {
    if (a.qrows) attn_query_row(a, true);
    constexpr int CG = 4, MR = 32;
    __shared__ float fw[CG * MR];
    __shared__ float redm[16], redl[16];
    __shared__ __align__(16) float po[CG][256];
    __shared__ __align__(16) float mo[256];
    const int h = blockIdx.x, slice = blockIdx.y, tid = threadIdx.x, c = tid >> 8, t = tid & 255;
    const int G = a.G;
    const float* ph = a.part + (size_t)h * G * (HD + 2);
    const int dd = slice * 256 + t;
    const float* pd = ph + dd;
    float v[MR];
#pragma unroll
    for (int u = 0; u < MR; u++) v[u] = pd[(size_t)min(c + CG * u, G - 1) * (HD + 2)];
    const int gi = min(tid, G - 1);
    const float mr = ph[(size_t)gi * (HD + 2) + HD], lr = ph[(size_t)gi * (HD + 2) + HD + 1];
    const float mg = tid < G ? mr : -INFINITY, lg = tid < G ? lr : 0.0f;
    const float wm = wave_max(mg);
    if ((tid & 63) == 0) redm[tid >> 6] = wm;
    lds_sync();
    float M = redm[0];
#pragma unroll
    for (int i = 1; i < 16; i++) M = fmaxf(M, redm[i]);
    const float f = tid < G && lg > 0.0f ? expf(mg - M) : 0.0f;
    if (tid < CG * MR) fw[tid] = f;
    const float wl = wave_sum(lg * f);
    if ((tid & 63) == 0) redl[tid >> 6] = wl;
    lds_sync();
    float L = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) L += redl[i];
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < MR; u++) o = c + CG * u < G ? __builtin_fmaf(v[u], fw[c + CG * u], o) : o;
    po[c][t] = o;
    lds_sync();
    if (c == 0) {
        const float sum = (po[0][t] + po[1][t]) + (po[2][t] + po[3][t]);
        const float r = L > 0.0f ? sum / L : 0.0f;
        a.out[(size_t)h * HD + dd] = r;
        mo[t] = r;
    }
    if (a.q8) {
        lds_sync();
        if (tid < 64) {
            const float4 f4 = reinterpret_cast<const float4*>(mo)[tid];
            const float v4[4] = {f4.x, f4.y, f4.z, f4.w};
            quantize_block_wave(v4, tid, a.q8, a.n_heads * HD / 256, h * (HD / 256) + slice);
        }
    }
}

// ---- query rows of a prompt chunk on the matrix cores ---------------------
// The same partials as attn_chunk_kernel's query-row mode (one (o, max, sum)
// per row, q head and chunk, merged by attn_merge_kernel), for 16 query rows
// at once: workgroup (c, kvh, rb) takes rows 16rb .. 16rb+15 and chunk c of
// the key range those rows see, and wave h is q head kvh*4 + h (4 q heads per
// kv head).  Each 16-key tile of K and V is read from HBM once for the 16
// rows and 4 heads and staged in LDS; per tile and wave
//   S^T (16 keys x 16 rows) = K . Q^T      HD/4 v_mfma_f32_16x16x4_f32
//   O^T (HD x 16 rows)     += V^T . P^T    HD/4 v_mfma_f32_16x16x4_f32
// with fp32 products and sums (the reference's per-row dot products and
// weighted V sums, gemma4-4b/cpu-blas/main.c:1909-1950, in another order).
// 16x16x4 operands: lane l = 16g + j supplies A[j][g] and B[g][j] and holds
// D[4g + r][j] in register r.  S^T: the K index of step s is dim
// (HD/4)g + s, so a lane reads 4 consecutive dims of key j (LDS) and of row
// j's q (registers).  P^T for the second product is S^T's registers as they
// are: step r takes key 4g + r of lane group g, so A of step r is
// V[4g + r][.]; A row j of O tile b is dim (HD/16)j + b, so a lane's V reads
// are 4 consecutive dims too and register r of O tile b in lane 16g + j is
// dim (HD/16)(4g + r) + b of row j.
// Chunks: the rows' key range [lo, hi] (lo = the first row's window start,
// hi = the last row's position) in G pieces of a multiple of 16 keys; keys
// outside a row's own window get weight 0 (and a chunk without any of a
// row's keys leaves (0, -inf, 0), which the merge ignores).  Keys are
// loaded clamped to the chunk, so every row read is a position in [lo, hi]
// that the cache or the chunk's K/V rows hold.
constexpr int kRowsKVM = 4;
constexpr float kRowsLazy = 8.0f;
typedef float f4_t __attribute__((ext_vector_type(4)));
// a global-memory f4_t: the integer select between the cache and the chunk's
// rows below would otherwise leave a generic pointer, i.e. flat loads, which
// the LDS waits also count
typedef __attribute__((address_space(1))) const f4_t g4_gf4_t;

template <int HD>
__global__ __launch_bounds__(64 * kRowsKVM) __attribute__((amdgpu_waves_per_eu(HD == 256 ? 2 : 1))) void attn_rows_mfma_kernel(AttnArgs a) {
    constexpr int NTH = 64 * kRowsKVM;
    constexpr int RS = HD + 4;            // K row stride (floats): conflict-free 16-byte reads
    constexpr int RV = HD / 16 * 20;      // V row: every 16 dims followed by 4 floats of padding
    constexpr int QS = HD / 4;            // score steps; q values per lane
    constexpr int NB = HD / 16;           // O tiles
    constexpr int LU = 16 * (HD / 4) / NTH;   // float4 of K (and of V) per thread and tile
    static_assert(LU * NTH == 16 * (HD / 4), "tile staging");
    __shared__ __align__(16) float ks[16 * RS];
    __shared__ __align__(16) float vs[16 * RV];
    const int c = blockIdx.x, kvh = blockIdx.y, rb = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, j = lane & 15;
    const int head = kvh * kRowsKVM + wave;
    const int M = a.qrows;
    const int z0 = 16 * rb, z1 = min(z0 + 16, M) - 1;
    const int lo = a.window > 0 ? max(0, a.p0 + z0 + 1 - a.window) : 0;
    const int hi = a.p0 + z1;
    const int cs = ((hi - lo + a.G) / a.G + 15) & ~15;    // ceil((hi - lo + 1) / G), whole tiles
    const int cb = lo + c * cs, ce = min(cb + cs, hi + 1);
    // this lane's query row, its position and window start
    const int z = z0 + j;
    const int qp = a.p0 + z;
    const int qlo = a.window > 0 ? max(0, qp + 1 - a.window) : 0;

    // K/V of a tile: thread tid stages float4 c4 of key `key` for u < LU
    // (the next tile's are loaded while this one is used; past the last tile
    // the last one is loaded again, so that no branch guards the loads)
    f4_t kr[LU], vr[LU];   // (HIP's float4 copies as a struct: an array of them stays in scratch)
    const float* kcb = a.kc + (size_t)kvh * HD;
    const float* vcb = a.vc + (size_t)kvh * HD;
    const float* kqb = a.kchunk + (size_t)kvh * HD;
    const float* vqb = a.vchunk + (size_t)kvh * HD;
    const int tl = ce - 1;
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int idx = u * NTH + tid, key = idx / (HD / 4), c4 = idx - key * (HD / 4);
            const int t = min(t0 + key, tl);
            const bool own = t >= a.p0;
            const size_t off = (size_t)(own ? t - a.p0 : attn_slot(a, t)) * a.kv_stride;
            const uintptr_t kb = own ? (uintptr_t)kqb : (uintptr_t)kcb;
            const uintptr_t vb = own ? (uintptr_t)vqb : (uintptr_t)vcb;
            kr[u] = reinterpret_cast<const g4_gf4_t*>(kb + 4 * off)[c4];
            vr[u] = reinterpret_cast<const g4_gf4_t*>(vb + 4 * off)[c4];
        }
    };
    load_tile(cb);   // an empty chunk (cb > hi) loads position hi: ce - 1 = hi

    float q[QS];
    {
        const float4* qv = reinterpret_cast<const float4*>(a.q + (size_t)min(z, M - 1) * a.n_heads * HD +
                                                           (size_t)head * HD + QS * g);
#pragma unroll
        for (int s = 0; s < QS / 4; s++) {
            const float4 t = qv[s];
            q[4 * s] = t.x;
            q[4 * s + 1] = t.y;
            q[4 * s + 2] = t.z;
            q[4 * s + 3] = t.w;
        }
    }

    float m = -INFINITY, lsum = 0.0f;   // lsum: this lane's keys only (summed over the groups at the end)
    f4_t o[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) o[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = cb; t0 < ce; t0 += 16) {
        __syncthreads();   // every wave is done with the previous tile
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int idx = u * NTH + tid, key = idx / (HD / 4), c4 = idx - key * (HD / 4);
            *reinterpret_cast<f4_t*>(ks + key * RS + 4 * c4) = kr[u];
            *reinterpret_cast<f4_t*>(vs + key * RV + 4 * c4 + 4 * (c4 >> 2)) = vr[u];
        }
        __syncthreads();
        load_tile(t0 + 16 < ce ? t0 + 16 : t0);

        // scores: four accumulators, so that no step waits for the previous one
        f4_t acc[4];
#pragma unroll
        for (int k = 0; k < 4; k++) acc[k] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        const float* kl = ks + j * RS + QS * g;
#pragma unroll
        for (int s = 0; s < QS / 4; s++) {
            const f4_t k4 = *reinterpret_cast<const f4_t*>(kl + 4 * s);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[0], q[4 * s], acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[1], q[4 * s + 1], acc[1], 0, 0, 0);
            acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[2], q[4 * s + 2], acc[2], 0, 0, 0);
            acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[3], q[4 * s + 3], acc[3], 0, 0, 0);
        }
        const f4_t sc = (acc[0] + acc[1]) + (acc[2] + acc[3]);

        // online softmax over the tile's keys 4g + r of row j
        float sv[4], mt = -INFINITY;
        bool val[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int kt = t0 + 4 * g + r;
            val[r] = kt < ce && kt >= qlo && kt <= qp;
            sv[r] = val[r] ? a.scale * sc[r] : -INFINITY;
            mt = fmaxf(mt, sv[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        // the running max moves only when a score exceeds it by more than
        // kRowsLazy (weights stay <= e^kRowsLazy); o and lsum are rescaled
        // only then, and only in waves where some row moved it
        const bool up = mt > m + kRowsLazy;   // also the first finite score (m = -inf)
        const float mn = up ? mt : m;
        const float alpha = !up ? 1.0f : m == -INFINITY ? 0.0f : expf(m - mn);
        float p[4], ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            p[r] = val[r] ? expf(sv[r] - mn) : 0.0f;
            ps += p[r];
        }
        lsum = lsum * alpha + ps;
        m = mn;
        if (__ballot(up)) {
#pragma unroll
            for (int b = 0; b < NB; b++) o[b] *= alpha;
        }

        // O^T += V^T . P^T
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float* vl = vs + (4 * g + r) * RV + NB / 16 * 20 * j;   // dim NB*j
#pragma unroll
            for (int b = 0; b < NB; b += 4) {
                const f4_t v4 = *reinterpret_cast<const f4_t*>(vl + b + 4 * (b >> 4));
                o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[0], p[r], o[b], 0, 0, 0);
                o[b + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[1], p[r], o[b + 1], 0, 0, 0);
                o[b + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[2], p[r], o[b + 2], 0, 0, 0);
                o[b + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4[3], p[r], o[b + 3], 0, 0, 0);
            }
        }
    }

    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (z < M) {
        float* pp = a.part + (size_t)z * a.part_z + ((size_t)head * a.G + c) * (HD + 2);
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int b = 0; b < NB; b += 2)
                *reinterpret_cast<float2*>(pp + NB * (4 * g + r) + b) = make_float2(o[b][r], o[b + 1][r]);
        if (g == 0) {
            pp[HD] = m;
            pp[HD + 1] = lsum;
        }
    }
}

// ---- query rows on the fp16 matrix cores, split operands -----------------
// attn_rows_mfma_kernel's partials with its products on v_mfma_f32_16x16x32
// / 16x16x16 f16 instead of 16x16x4 f32: every operand v is split into fp16
// hi = fp16(v) and lo = fp16(v - hi) (v - hi is exact in fp32), and a product
// a.b is hi_a.hi_b + hi_a.lo_b + lo_a.hi_b (three MFMAs), summed in fp32.
// Error of the split: |v - hi - lo| <= max(2^-22 |v|, 2^-25) -- relative while
// lo is an fp16 normal, and half the fp16 subnormal spacing (2^-24) once lo
// falls below 2^-14, i.e. for |v| below about 2^-3 -- and the dropped lo.lo
// is below 2^-22 |a.b|; so a product carries at most about
// 3 * 2^-22 |a.b| + 2^-25 (|a| + |b|).  The softmax weights (<= e^kRowsLazy)
// are split as 16 p (below fp16's maximum; the partial o is scaled back by
// 1/16, exactly), which moves their absolute floor to 2^-29: a weight of
// 1e-3 keeps 2^-19 of relative precision instead of 2^-15.  K and V are the
// RMS-normalised rows (elements of order 1, at most sqrt(head_dim)) and q
// the normalised query, well inside fp16's range; operands far smaller than
// that (V of order 1e-3) would meet the 2^-25 floor.  Per 16-key tile and
// wave:
//   S^T = K . Q^T   HD/32 steps of three 16x16x32 MFMAs: lane (j, g) gives K
//                   row j and its q row j, dims 32s + 8g .. +7
//   O^T += V^T.P^T  HD/16 blocks of three 16x16x16 MFMAs: lane (j, g) gives
//                   V^T row (dim) 16b + j at keys 4g .. 4g+3 (V staged
//                   transposed) and its own weights p[0..3] (keys 4g + r of
//                   row j), the layout the softmax leaves them in
// so that the matrix-core work per tile is about a fifth of the fp32 form's.
typedef _Float16 ah4_t __attribute__((ext_vector_type(4)));
typedef _Float16 ah8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ _Float16 split_hi(float v) { return (_Float16)v; }
__device__ __forceinline__ _Float16 split_lo(float v, _Float16 h) { return (_Float16)(v - (float)h); }

template <int HD>
__global__ __launch_bounds__(64 * kRowsKVM) __attribute__((amdgpu_waves_per_eu(HD == 256 ? 2 : 1))) void attn_rows_h16_kernel(AttnArgs a) {
    constexpr int NTH = 64 * kRowsKVM;
    constexpr int KS = HD + 8;            // K row stride (fp16)
    constexpr int VS = 16 + 4;            // V^T row stride (fp16): 16 keys + pad
    constexpr int NS = HD / 32;           // score steps
    constexpr int NB = HD / 16;           // O tiles
    constexpr int LU = 16 * (HD / 4) / NTH;   // float4 of K (and of V) per thread and tile
    static_assert(LU * NTH == 16 * (HD / 4), "tile staging");
    __shared__ __align__(16) _Float16 kh[16 * KS], kl[16 * KS];
    __shared__ __align__(16) _Float16 vh[HD * VS], vl[HD * VS];
    const int c = blockIdx.x, kvh = blockIdx.y, rb = blockIdx.z;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, j = lane & 15;
    const int head = kvh * kRowsKVM + wave;
    const int M = a.qrows;
    const int z0 = 16 * rb, z1 = min(z0 + 16, M) - 1;
    const int lo = a.window > 0 ? max(0, a.p0 + z0 + 1 - a.window) : 0;
    const int hi = a.p0 + z1;
    const int cs = ((hi - lo + a.G) / a.G + 15) & ~15;    // ceil((hi - lo + 1) / G), whole tiles
    const int cb = lo + c * cs, ce = min(cb + cs, hi + 1);
    const int z = z0 + j;
    const int qp = a.p0 + z;
    const int qlo = a.window > 0 ? max(0, qp + 1 - a.window) : 0;

    f4_t kr[LU], vr[LU];
    const float* kcb = a.kc + (size_t)kvh * HD;
    const float* vcb = a.vc + (size_t)kvh * HD;
    const float* kqb = a.kchunk + (size_t)kvh * HD;
    const float* vqb = a.vchunk + (size_t)kvh * HD;
    const int tl = ce - 1;
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int idx = u * NTH + tid, key = idx / (HD / 4), c4 = idx - key * (HD / 4);
            const int t = min(t0 + key, tl);
            const bool own = t >= a.p0;
            const size_t off = (size_t)(own ? t - a.p0 : attn_slot(a, t)) * a.kv_stride;
            const uintptr_t kb = own ? (uintptr_t)kqb : (uintptr_t)kcb;
            const uintptr_t vb = own ? (uintptr_t)vqb : (uintptr_t)vcb;
            kr[u] = reinterpret_cast<const g4_gf4_t*>(kb + 4 * off)[c4];
            vr[u] = reinterpret_cast<const g4_gf4_t*>(vb + 4 * off)[c4];
        }
    };
    load_tile(cb);   // an empty chunk (cb > hi) loads position hi: ce - 1 = hi

    ah8_t qh[NS], ql[NS];
    {
        const float* qrow = a.q + (size_t)min(z, M - 1) * a.n_heads * HD + (size_t)head * HD + 8 * g;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const float4 t0 = reinterpret_cast<const float4*>(qrow + 32 * s)[0];
            const float4 t1 = reinterpret_cast<const float4*>(qrow + 32 * s)[1];
            const float v[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const _Float16 h = split_hi(v[t]);
                qh[s][t] = h;
                ql[s][t] = split_lo(v[t], h);
            }
        }
    }

    float m = -INFINITY, lsum = 0.0f;   // lsum: this lane's keys only (summed over the groups at the end)
    f4_t o[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) o[b] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = cb; t0 < ce; t0 += 16) {
        __syncthreads();   // every wave is done with the previous tile
#pragma unroll
        for (int u = 0; u < LU; u++) {
            const int idx = u * NTH + tid, key = idx / (HD / 4), c4 = idx - key * (HD / 4);
            ah4_t h4, l4;
#pragma unroll
            for (int x = 0; x < 4; x++) {
                const _Float16 h = split_hi(kr[u][x]);
                h4[x] = h;
                l4[x] = split_lo(kr[u][x], h);
            }
            *reinterpret_cast<ah4_t*>(kh + key * KS + 4 * c4) = h4;
            *reinterpret_cast<ah4_t*>(kl + key * KS + 4 * c4) = l4;
#pragma unroll
            for (int x = 0; x < 4; x++) {
                const _Float16 h = split_hi(vr[u][x]);
                vh[(4 * c4 + x) * VS + key] = h;
                vl[(4 * c4 + x) * VS + key] = split_lo(vr[u][x], h);
            }
        }
        __syncthreads();
        load_tile(t0 + 16 < ce ? t0 + 16 : t0);

        // scores: hi.hi, hi.lo and lo.hi in three accumulators
        f4_t acc[3];
#pragma unroll
        for (int k = 0; k < 3; k++) acc[k] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
        const _Float16* kph = kh + j * KS + 8 * g;
        const _Float16* kpl = kl + j * KS + 8 * g;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const ah8_t Ah = *reinterpret_cast<const ah8_t*>(kph + 32 * s);
            const ah8_t Al = *reinterpret_cast<const ah8_t*>(kpl + 32 * s);
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, qh[s], acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ah, ql[s], acc[1], 0, 0, 0);
            acc[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Al, qh[s], acc[2], 0, 0, 0);
        }
        const f4_t sc = acc[0] + (acc[1] + acc[2]);

        // online softmax over the tile's keys 4g + r of row j (as in attn_rows_mfma_kernel)
        float sv[4], mt = -INFINITY;
        bool val[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int kt = t0 + 4 * g + r;
            val[r] = kt < ce && kt >= qlo && kt <= qp;
            sv[r] = val[r] ? a.scale * sc[r] : -INFINITY;
            mt = fmaxf(mt, sv[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const bool up = mt > m + kRowsLazy;
        const float mn = up ? mt : m;
        const float alpha = !up ? 1.0f : m == -INFINITY ? 0.0f : expf(m - mn);
        float p[4], ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            p[r] = val[r] ? expf(sv[r] - mn) : 0.0f;
            ps += p[r];
        }
        lsum = lsum * alpha + ps;
        m = mn;
        if (__ballot(up)) {
#pragma unroll
            for (int b = 0; b < NB; b++) o[b] *= alpha;
        }

        // O^T += V^T . P^T
        ah4_t Ph, Pl;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p16 = 16.0f * p[r];      // <= 16 e^kRowsLazy < 65504; exact
            const _Float16 h = split_hi(p16);
            Ph[r] = h;
            Pl[r] = split_lo(p16, h);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const ah4_t Vh = *reinterpret_cast<const ah4_t*>(vh + (16 * b + j) * VS + 4 * g);
            const ah4_t Vl = *reinterpret_cast<const ah4_t*>(vl + (16 * b + j) * VS + 4 * g);
            o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(Vh, Ph, o[b], 0, 0, 0);
            o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(Vh, Pl, o[b], 0, 0, 0);
            o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(Vl, Ph, o[b], 0, 0, 0);
        }
    }

    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (z < M) {
        // o[b][r] is dim 16b + 4g + r of row z
        float* pp = a.part + (size_t)z * a.part_z + ((size_t)head * a.G + c) * (HD + 2);
        constexpr float kUn16 = 1.0f / 16.0f;   // the weights' factor 16, exactly
#pragma unroll
        for (int b = 0; b < NB; b++) {
            *reinterpret_cast<float2*>(pp + 16 * b + 4 * g) = make_float2(o[b][0] * kUn16, o[b][1] * kUn16);
            *reinterpret_cast<float2*>(pp + 16 * b + 4 * g + 2) = make_float2(o[b][2] * kUn16, o[b][3] * kUn16);
        }
        if (g == 0) {
            pp[HD] = m;
            pp[HD + 1] = lsum;
        }
    }
}

// partial kernel LDS: work region + (max, sum) pairs [+ this position's K, V]
size_t attn_lds(int hd, int kvm, bool fused) {
    return 4 * (fused ? (size_t)attn_new_kv_off(hd, kvm) + 2 * (size_t)hd
                      : (size_t)attn_work_floats(hd, kvm) + 2 * (size_t)kvm);
}

template <int HD>
void launch_chunk(const AttnArgs& a, int kp, const dim3& grid) {
    const size_t lds = attn_chunk_lds(HD, kp);
    if (a.qrows) {
        if (kp == 1) hipLaunchKernelGGL((attn_chunk_kernel<HD, 1, false>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
        else if (kp == 2) hipLaunchKernelGGL((attn_chunk_kernel<HD, 2, false>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
        else if (kp == 4) hipLaunchKernelGGL((attn_chunk_kernel<HD, 4, false>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
        else hipLaunchKernelGGL((attn_chunk_kernel<HD, 8, false>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
        return;
    }
    // decode with 4 q heads per kv head: eight waves per workgroup, twice
    // the rows in flight per CU.  hd 256: two register sets of 4 positions
    // per wave (172 VGPRs); hd 512: one set.  Over 32K positions: 34.6
    // against 38.6 us at hd 256, 55.1 against 56.1 us at hd 512 (chunk +
    // merge); the E4B decode step with its 512-slot rings in 16 chunks:
    // 2.258 against 2.292 ms
    if (kp == 4) {
        const size_t l8 = attn_chunk_lds(HD, kp, 8);
        if constexpr (HD == 256) {
            if (a.q_norm) hipLaunchKernelGGL((attn_chunk_kernel<HD, 4, true, 512, 4, 1>), grid, dim3(512), l8, g4_stream(), a);
            else hipLaunchKernelGGL((attn_chunk_kernel<HD, 4, true, 512, 4, 2>), grid, dim3(512), l8, g4_stream(), a);
        } else {
            if (a.q_norm) hipLaunchKernelGGL((attn_chunk_kernel<HD, 4, false, 512, 0, 1>), grid, dim3(512), l8, g4_stream(), a);
            else hipLaunchKernelGGL((attn_chunk_kernel<HD, 4, false, 512, 0, 2>), grid, dim3(512), l8, g4_stream(), a);
        }
        return;
    }
    if (kp == 1) hipLaunchKernelGGL((attn_chunk_kernel<HD, 1, true>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
    else if (kp == 2) hipLaunchKernelGGL((attn_chunk_kernel<HD, 2, true>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
    else if (kp == 4) hipLaunchKernelGGL((attn_chunk_kernel<HD, 4, true>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
    else hipLaunchKernelGGL((attn_chunk_kernel<HD, 8, true>), grid, dim3(kAttnThreads), lds, g4_stream(), a);
}

template <int HD>
void launch_merge(const AttnArgs& a, const dim3& grid) {
    if (a.G <= 16) hipLaunchKernelGGL((attn_merge_kernel<HD, 16>), grid, dim3(256), 0, g4_stream(), a);
    else if (a.G <= 32) hipLaunchKernelGGL((attn_merge_kernel<HD, 32>), grid, dim3(256), 0, g4_stream(), a);
    else if (a.G <= 128) hipLaunchKernelGGL((attn_merge_wide_kernel<HD>), grid, dim3(1024), 0, g4_stream(), a);
    else hipLaunchKernelGGL((attn_merge_kernel<HD, 128>), grid, dim3(256), 0, g4_stream(), a);
}

int launch_attn(const AttnArgs& a) {
    const int kvm = a.n_heads / a.n_kv;
    const int zq = a.qrows > 0 ? a.qrows : 1;
    const dim3 grid(a.G, a.n_kv, zq);
    // q heads per kv head rounded up to a power of two (the register kernel's
    // template); its LDS must fit the default 64 KB
    const int kp = kvm <= 1 ? 1 : kvm <= 2 ? 2 : kvm <= 4 ? 4 : 8;
    if (a.qrows && kvm == kRowsKVM) {
        const dim3 rgrid(a.G, a.n_kv, (a.qrows + 15) / 16);
        if (a.hd == 256) {
            hipLaunchKernelGGL(attn_rows_h16_kernel<256>, rgrid, dim3(64 * kRowsKVM), 0, g4_stream(), a);
            launch_merge<256>(a, dim3(a.n_heads, 1, zq));
        } else {
            // (the split form needs 35 VGPRs more than a wave has at hd 512)
            hipLaunchKernelGGL(attn_rows_mfma_kernel<512>, rgrid, dim3(64 * kRowsKVM), 0, g4_stream(), a);
            launch_merge<512>(a, dim3(a.n_heads, 2, zq));
        }
        return g4_check_launch("attn_rows_h16_kernel/attn_rows_mfma_kernel/attn_merge_kernel");
    }
    if (attn_chunk_lds(a.hd, kp) <= 65536) {
        // no out: the partials only, merged by the caller (g4_mm_attn_merge)
        if (a.hd == 256) {
            launch_chunk<256>(a, kp, grid);
            if (a.out) launch_merge<256>(a, dim3(a.n_heads, 1, zq));
        } else {
            launch_chunk<512>(a, kp, grid);
            if (a.out) launch_merge<512>(a, dim3(a.n_heads, 2, zq));
        }
        return g4_check_launch("attn_chunk_kernel/attn_merge_kernel");
    }
    if (a.qrows) return g4_fail(G4_ERR_ARG, "attention over query rows: %d q heads per kv head at head_dim %d unsupported", kvm, a.hd);
    const size_t lds = attn_lds(a.hd, kvm, a.q_norm != nullptr);
    if (a.hd == 256) {
        hipLaunchKernelGGL(attn_decode_kernel<256>, grid, dim3(kAttnThreads), lds, g4_stream(), a);
        launch_merge<256>(a, dim3(a.n_heads, 1));
    } else {
        hipLaunchKernelGGL(attn_decode_kernel<512>, grid, dim3(kAttnThreads), lds, g4_stream(), a);
        launch_merge<512>(a, dim3(a.n_heads, 2));
    }
    return g4_check_launch("attn_decode_kernel/attn_merge_kernel");
}

int check_attn_shape(const char* who, int n_heads, int n_kv, int hd, int G, bool fused = false) {
    if (hd != 256 && hd != 512) return g4_fail(G4_ERR_ARG, "%s: head_dim %d unsupported (256 or 512)", who, hd);
    if (n_kv <= 0 || n_heads <= 0 || n_heads % n_kv || n_heads / n_kv > 8)
        return g4_fail(G4_ERR_ARG, "%s: n_heads=%d n_kv=%d (need n_heads/n_kv in 1..8)", who, n_heads, n_kv);
    if (G < 1 || G > kMaxChunks) return g4_fail(G4_ERR_ARG, "%s: %d chunks (1..%d)", who, G, kMaxChunks);
    if (attn_lds(hd, n_heads / n_kv, fused) > 65536)
        return g4_fail(G4_ERR_ARG, "%s: %d q heads per kv head at head_dim %d exceed the LDS budget", who,
                       n_heads / n_kv, hd);
    return G4_OK;
}

// library-owned workspace for the host-position entry points.  It only
// grows; growing waits for the whole device, since launches on any stream
// may still read the old buffer.  Calls that overlap in time share it, so
// concurrent callers on different streams race (one host thread and stream
// per process is the supported use); the mutex keeps the pointer and size
// themselves consistent.
void* g_ws = nullptr;
size_t g_ws_bytes = 0;
std::mutex g_ws_mu;

int workspace(size_t bytes, uint8_t** p) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (bytes > g_ws_bytes) {
        if (g_ws) {
            G4_HIP(hipDeviceSynchronize());
            G4_HIP(hipFree(g_ws));
            g_ws = nullptr;
            g_ws_bytes = 0;
        }
        if (hipMalloc(&g_ws, bytes) != hipSuccess) return g4_fail(G4_ERR_NOMEM, "attention workspace (%zu B)", bytes);
        g_ws_bytes = bytes;
    }
    *p = (uint8_t*)g_ws;
    return G4_OK;
}

// ---- scratch of the allocation-free entry point ---------------------------
// g4_attn_decode_noalloc keeps its chunk partials in this file-scope device
// array instead of the library workspace: one copy per GPU, held until the
// process ends.  In host code `scratch` names a host-side stand-in, not a
// device address: g4_init resolves each device's address once
// (attn_scratch_setup) and only that address is handed to kernels.
constexpr int kScratchDevices = 64;
__device__ __align__(256) uint8_t scratch[G4_ATTN_NOALLOC_SCRATCH];
void* g_scratch_dev[kScratchDevices];   // device address of `scratch` per device

}  // namespace g4

int g4_attn_scratch_setup(int device) {
    G4_CHECK_ARG(device >= 0 && device < g4::kScratchDevices, "attention scratch: device %d beyond %d", device,
                 g4::kScratchDevices);
    if (g4::g_scratch_dev[device]) return G4_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g4::scratch));
    if (e != hipSuccess || !p)
        return g4_fail(G4_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g4::g_scratch_dev[device] = p;
    return G4_OK;
}

namespace g4 {

// about 16 positions per workgroup, at most 64 chunks per kv head unless a
// chunk would exceed kChunkMax positions
int chunks_for(int nwin) {
    int G = (nwin + 31) / 32;          // about 32 positions per workgroup, 1..128 chunks
    if (G < 1) G = 1;
    if (G > 128) G = 128;
    while ((nwin + G - 1) / G > kChunkMax) G++;
    return G;
}

}  // namespace g4

using namespace g4;

// ---------------------------------------------------------------------------
// entry points
// ---------------------------------------------------------------------------
extern "C" int g4_apply_rope_neox(float* vec, int n_heads, int head_dim, int n_rot, int pos, float freq_base,
                                  float freq_scale, const float* freq_factors) {
    G4_CHECK_ARG(vec && n_heads > 0 && head_dim > 0 && head_dim % 2 == 0, "g4_apply_rope_neox: bad arguments");
    G4_CHECK_ARG(n_rot >= 0 && n_rot <= head_dim, "g4_apply_rope_neox: n_rot=%d > head_dim=%d", n_rot, head_dim);
    // theta scale on the host with the C library's powf, as main.c:1727
    const float ts = powf(freq_base, -2.0f / (float)n_rot);
    hipLaunchKernelGGL(rope_kernel, dim3(n_heads), dim3(256), (size_t)head_dim * 4, g4_stream(), vec, head_dim,
                       n_rot, pos, ts, freq_scale, freq_factors);
    return g4_check_launch("rope_kernel");
}

extern "C" int g4_rope_table(float* tab, const int* dpos, int pos, int n_rot, float freq_base, float freq_scale,
                             const float* freq_factors) {
    G4_CHECK_ARG(tab && n_rot > 0 && n_rot % 2 == 0 && n_rot <= 2048, "g4_rope_table: bad arguments");
    const float ts = powf(freq_base, -2.0f / (float)n_rot);
    hipLaunchKernelGGL(rope_table_kernel, dim3(1), dim3(256), 0, g4_stream(), (float2*)tab, dpos, pos, n_rot / 2, ts,
                       freq_scale, freq_factors);
    return g4_check_launch("rope_table_kernel");
}

extern "C" int g4_qkv_post(float* q, const float* q_norm, const float* k, const float* v, const float* k_norm, float* kc,
                           float* vc, int kv_stride, int ring, const int* dpos, int pos, int n_heads, int n_kv, int hd,
                           int n_rot, float freq_base, float freq_scale, const float* ff, float eps,
                           const float* rope_tab) {
    G4_CHECK_ARG(q && q_norm && hd > 0 && hd <= 1024 && n_rot <= hd, "qkv_post: bad arguments");
    G4_CHECK_ARG(!k || (v && k_norm && kc && vc && kv_stride >= n_kv * hd), "qkv_post: bad K/V arguments");
    QKVArgs a;
    a.q = q; a.q_norm = q_norm; a.k = k; a.v = v; a.k_norm = k_norm; a.kc = kc; a.vc = vc;
    a.dpos = dpos; a.ff = ff; a.pos = pos; a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.n_rot = n_rot;
    a.kv_stride = kv_stride; a.ring = ring;
    a.ts = powf(freq_base, -2.0f / (float)n_rot);
    a.fs = freq_scale; a.eps = eps;
    a.tab = (const float2*)rope_tab;
    if (qkv_wave_ok(a)) {
        launch_qkv_wave(a, 1);
        return g4_check_launch("qkv_post_wave_kernel");
    }
    const int grid = n_heads + (k ? 2 * n_kv : 0);
    hipLaunchKernelGGL(qkv_post_kernel, dim3(grid), dim3(256), (size_t)hd * 4, g4_stream(), a);
    return g4_check_launch("qkv_post_kernel");
}

extern "C" int g4_kv_append_rope(float* k, float* v, const float* k_norm, float* kc, float* vc, int kv_stride,
                                 int ring, int pos, int n_kv, int hd, int n_rot, float freq_base, float freq_scale,
                                 const float* freq_factors, float eps) {
    G4_CHECK_ARG(k && v && k_norm && kc && vc && n_kv > 0 && pos >= 0, "g4_kv_append_rope: bad arguments");
    G4_CHECK_ARG(kv_stride >= n_kv * hd, "g4_kv_append_rope: kv_stride %d < n_kv*hd", kv_stride);
    QKVArgs a;
    a.q = nullptr; a.q_norm = nullptr; a.k = k; a.v = v; a.k_norm = k_norm; a.kc = kc; a.vc = vc;
    a.dpos = nullptr; a.ff = freq_factors; a.pos = pos; a.n_heads = 0; a.n_kv = n_kv; a.hd = hd; a.n_rot = n_rot;
    a.kv_stride = kv_stride; a.ring = ring;
    a.ts = powf(freq_base, -2.0f / (float)n_rot);
    a.fs = freq_scale; a.eps = eps;
    a.tab = nullptr;
    hipLaunchKernelGGL(qkv_post_kernel, dim3(2 * n_kv), dim3(256), (size_t)hd * 4, g4_stream(), a);
    return g4_check_launch("qkv_post_kernel");
}

extern "C" size_t g4_attn_part_bytes(int n_heads, int hd, int G) { return (size_t)n_heads * G * (hd + 2) * 4; }

// (cos, sin) tables of positions pos0 .. pos0+m-1, n_rot/2 pairs each
extern "C" int g4_rope_table_rows(float* tab, int pos0, int m, int n_rot, float freq_base, float freq_scale,
                                  const float* freq_factors) {
    G4_CHECK_ARG(tab && pos0 >= 0 && m > 0 && n_rot > 0 && n_rot % 2 == 0 && n_rot <= 2048,
                 "g4_rope_table_rows: bad arguments");
    const float ts = powf(freq_base, -2.0f / (float)n_rot);
    hipLaunchKernelGGL(rope_table_rows_kernel, dim3(m), dim3(256), 0, g4_stream(), (float2*)tab, pos0, n_rot / 2, ts,
                       freq_scale, freq_factors);
    return g4_check_launch("rope_table_rows_kernel");
}

// qkv_post over m tokens: q rows normalised and rotated in place; k/v rows
// (nullable) normalised (k rotated) into rows of kout/vout (stride kv_stride)
extern "C" int g4_qkv_post_rows(float* q, const float* q_norm, const float* k, const float* v, const float* k_norm,
                                float* kout, float* vout, int kv_stride, const float* tab_rows, int m, int n_heads,
                                int n_kv, int hd, int n_rot, float eps) {
    G4_CHECK_ARG(q && q_norm && tab_rows && m > 0 && m <= 65535 && hd > 0 && hd <= 1024 && n_rot > 0 && n_rot <= hd,
                 "qkv_post_rows: bad arguments");
    G4_CHECK_ARG(!k || (v && k_norm && kout && vout && kv_stride >= n_kv * hd), "qkv_post_rows: bad K/V arguments");
    QKVArgs a{};
    a.q = q; a.q_norm = q_norm; a.k = k; a.v = v; a.k_norm = k_norm; a.kc = kout; a.vc = vout;
    a.dpos = nullptr; a.ff = nullptr; a.pos = 0; a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.n_rot = n_rot;
    a.kv_stride = kv_stride; a.ring = 0; a.ts = 1.0f; a.fs = 1.0f; a.eps = eps;
    a.tab = (const float2*)tab_rows;
    if (qkv_wave_ok(a)) {
        launch_qkv_wave(a, m);
        return g4_check_launch("qkv_post_wave_kernel");
    }
    const int grid = n_heads + (k ? 2 * n_kv : 0);
    hipLaunchKernelGGL(qkv_post_rows_kernel, dim3(grid, m), dim3(256), (size_t)hd * 4, g4_stream(), a);
    return g4_check_launch("qkv_post_rows_kernel");
}

// rows 0..m-1 of kin/vin (stride kv_stride) -> the cache slots of positions
// pos0 .. pos0+m-1 (slot = pos % ring with a ring; only the last `ring`
// rows are kept)
extern "C" int g4_kv_store_rows(float* kc, float* vc, const float* kin, const float* vin, int kv_stride, int ring,
                                int pos0, int m, int kvd) {
    G4_CHECK_ARG(kc && vc && kin && vin && m > 0 && pos0 >= 0 && kvd > 0 && kv_stride >= kvd && ring >= 0,
                 "g4_kv_store_rows: bad arguments");
    const int first = ring > 0 && m > ring ? m - ring : 0;
    hipLaunchKernelGGL(kv_store_rows_kernel, dim3(m - first), dim3(256), 0, g4_stream(), kc, vc,
                       kin + (size_t)first * kv_stride, vin + (size_t)first * kv_stride, kv_stride, ring, pos0 + first,
                       kvd);
    return g4_check_launch("kv_store_rows_kernel");
}

// The attention block for m query rows of a prompt chunk at positions
// p0 .. p0+m-1: q already normalised and rotated (n_heads*hd floats per row),
// the chunk's own K/V in rows of kchunk/vchunk (stride kv_stride), earlier
// positions in the (ring) cache; window 0 = full attention.  part holds
// m * g4_attn_part_bytes(n_heads, hd, G) bytes; out gets n_heads*hd floats
// per row and, if q8, the Q8_K rows (g4_q8K_row_stride(n_heads*hd) apart).
extern "C" int g4_attn_decode_rows(const float* q, const float* kc, const float* vc, const float* kchunk,
                                   const float* vchunk, int kv_stride, int ring, int p0, int m, int window, int n_heads,
                                   int n_kv, int hd, float attn_scale, int G, float* part, float* out, void* q8) {
    int rc = check_attn_shape("attn_decode_rows", n_heads, n_kv, hd, G);
    if (rc) return rc;
    G4_CHECK_ARG(q && kc && vc && kchunk && vchunk && part && out && p0 >= 0 && m > 0 && m <= 65535,
                 "attn_decode_rows: bad arguments");
    G4_CHECK_ARG(kv_stride >= n_kv * hd && ring >= 0 && window >= 0, "attn_decode_rows: bad cache arguments");
    G4_CHECK_ARG(ring == 0 || (window > 0 && window <= ring), "attn_decode_rows: a ring needs window <= ring");
    const int nmax = window > 0 && window < p0 + m ? window : p0 + m;
    G4_CHECK_ARG((nmax + G - 1) / G <= kChunkMax, "attn_decode_rows: %d chunks too few for %d positions", G, nmax);
    AttnArgs a = {};
    a.q = q; a.kc = kc; a.vc = vc; a.dpos = nullptr; a.out = out; a.q8 = (uint8_t*)q8; a.part = part;
    a.window = window; a.kv_stride = kv_stride; a.ring = ring;
    a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.scale = attn_scale; a.G = G;
    a.qrows = m; a.p0 = p0; a.kchunk = kchunk; a.vchunk = vchunk;
    a.part_z = g4_attn_part_bytes(n_heads, hd, G) / 4;
    a.q8_row = q8 ? g4_q8K_row_stride(n_heads * hd) : 0;
    return launch_attn(a);
}

static int attn_common(const char* who, AttnArgs& a) {
    int rc = check_attn_shape(who, a.n_heads, a.n_kv, a.hd, a.G);
    if (rc) return rc;
    G4_CHECK_ARG(a.q && a.kc && a.vc && a.out, "%s: null pointer", who);
    G4_CHECK_ARG(a.kv_stride >= a.n_kv * a.hd, "%s: kv_stride %d < n_kv*hd", who, a.kv_stride);
    uint8_t* ws = nullptr;
    rc = workspace(g4_attn_part_bytes(a.n_heads, a.hd, a.G), &ws);
    if (rc) return rc;
    a.part = (float*)ws;
    return launch_attn(a);
}

// The attention block of main.c:1909-1950 over a flat cache (position t at
// kc + t*kv_stride), positions t_start .. t_start+nwin-1.
extern "C" int g4_attn_decode(const float* q, const float* kc, const float* vc, int kv_stride, int t_start,
                              int nwin, int n_heads, int n_kv, int hd, float attn_scale, float* out) {
    G4_CHECK_ARG(t_start >= 0 && nwin >= 0, "g4_attn_decode: t_start=%d nwin=%d", t_start, nwin);
    AttnArgs a = {};
    a.q = q; a.kc = kc; a.vc = vc; a.dpos = nullptr; a.out = out; a.q8 = nullptr;
    a.t_start = t_start; a.nwin = nwin; a.window = 0; a.kv_stride = kv_stride; a.ring = 0;
    a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.scale = attn_scale; a.G = chunks_for(nwin);
    return attn_common("g4_attn_decode", a);
}

// g4_attn_decode with its partials in the per-GPU scratch array: the same
// kernels and chunk count, so the same bits; no allocation, no memset (the
// chunk kernel writes every partial the merge reads, whatever the previous
// call left there).  Calls that overlap in time on one GPU share the array
// and race.
extern "C" int g4_attn_decode_noalloc(const float* q, const float* kc, const float* vc, int kv_stride, int t_start,
                                      int nwin, int n_heads, int n_kv, int hd, float attn_scale, float* out) {
    G4_CHECK_ARG(t_start >= 0 && nwin >= 0, "g4_attn_decode_noalloc: t_start=%d nwin=%d", t_start, nwin);
    AttnArgs a = {};
    a.q = q; a.kc = kc; a.vc = vc; a.dpos = nullptr; a.out = out; a.q8 = nullptr;
    a.t_start = t_start; a.nwin = nwin; a.window = 0; a.kv_stride = kv_stride; a.ring = 0;
    a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.scale = attn_scale; a.G = chunks_for(nwin);
    int rc = check_attn_shape("g4_attn_decode_noalloc", n_heads, n_kv, hd, a.G);
    if (rc) return rc;
    G4_CHECK_ARG(q && kc && vc && out, "g4_attn_decode_noalloc: null pointer");
    G4_CHECK_ARG(kv_stride >= n_kv * hd, "g4_attn_decode_noalloc: kv_stride %d < n_kv*hd", kv_stride);
    const size_t need = g4_attn_part_bytes(n_heads, hd, a.G);
    G4_CHECK_ARG(need <= G4_ATTN_NOALLOC_SCRATCH,
                 "g4_attn_decode_noalloc: %zu B of partials (%d heads x %d chunks x head_dim %d) exceed the %u B "
                 "scratch", need, n_heads, a.G, hd, (unsigned)G4_ATTN_NOALLOC_SCRATCH);
    int dev = -1;
    G4_HIP(hipGetDevice(&dev));
    G4_CHECK(dev >= 0 && dev < kScratchDevices && g_scratch_dev[dev], G4_ERR_STATE,
             "g4_attn_decode_noalloc: g4_init has not set up device %d", dev);
    a.part = (float*)g_scratch_dev[dev];
    return launch_attn(a);
}

// Same block over a ring cache of `ring` slots (slot = t % ring) at position
// pos with a sliding window (window <= ring; 0 = full attention, then ring
// must be 0 or >= pos+1).
extern "C" int g4_attn_decode_ring(const float* q, const float* kc, const float* vc, int kv_stride, int ring,
                                   int pos, int window, int n_heads, int n_kv, int hd, float attn_scale, float* out) {
    G4_CHECK_ARG(pos >= 0 && ring >= 0 && window >= 0, "g4_attn_decode_ring: bad pos/ring/window");
    const int t0 = window > 0 ? (pos + 1 - window > 0 ? pos + 1 - window : 0) : 0;
    const int nwin = pos + 1 - t0;
    G4_CHECK_ARG(ring == 0 || nwin <= ring, "g4_attn_decode_ring: window %d exceeds ring %d", nwin, ring);
    AttnArgs a = {};
    a.q = q; a.kc = kc; a.vc = vc; a.dpos = nullptr; a.out = out; a.q8 = nullptr;
    a.t_start = t0; a.nwin = nwin; a.window = window; a.kv_stride = kv_stride; a.ring = ring;
    a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.scale = attn_scale; a.G = chunks_for(nwin);
    return attn_common("g4_attn_decode_ring", a);
}

// Engine form: position read from device memory, fixed chunk count G (so a
// captured graph stays valid as pos advances; G * 1024 must cover the
// window), caller-owned workspace of g4_attn_part_bytes(n_heads, hd, G) bytes,
// optional fused Q8_K output.
extern "C" int g4_attn_decode_dev(const float* q, const float* kc, const float* vc, int kv_stride, int ring,
                                  const int* dpos, int window, int n_heads, int n_kv, int hd, float attn_scale, int G,
                                  float* part, float* out, void* q8) {
    int rc = check_attn_shape("attn_decode_dev", n_heads, n_kv, hd, G);
    if (rc) return rc;
    G4_CHECK_ARG(q && kc && vc && dpos && part && out && G >= 1 && G <= kMaxChunks, "attn_decode_dev: bad arguments");
    AttnArgs a = {};
    a.q = q; a.kc = kc; a.vc = vc; a.dpos = dpos; a.out = out; a.q8 = (uint8_t*)q8;
    a.part = part;
    a.window = window; a.kv_stride = kv_stride; a.ring = ring;
    a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.scale = attn_scale; a.G = G;
    return launch_attn(a);
}

// qkv_post + attention in one pass (main.c:1886-1950): q_raw is the raw Q
// projection (left unchanged); k_raw/v_raw (null on shared-KV layers) are
// this position's raw K/V projections, stored normalised (K rotated) at slot
// pos of kstore/vstore.  Otherwise as g4_attn_decode_dev.
extern "C" int g4_attn_decode_fused(const float* q_raw, const float* q_norm, const float* k_raw, const float* v_raw,
                                    const float* k_norm, float* kstore, float* vstore, const float* kc, const float* vc,
                                    int kv_stride, int ring, const int* dpos, int window, int n_heads, int n_kv, int hd,
                                    int n_rot, const float* rope_tab, float eps, float attn_scale, int G, float* part,
                                    float* out, void* q8) {
    int rc = check_attn_shape("attn_decode_fused", n_heads, n_kv, hd, G, true);
    if (rc) return rc;
    G4_CHECK_ARG(q_raw && q_norm && rope_tab && kc && vc && dpos && part, "attn_decode_fused: null pointer");
    G4_CHECK_ARG(out || (!q8 && attn_chunk_lds(hd, n_heads / n_kv <= 1 ? 1 : n_heads / n_kv <= 2 ? 2 : n_heads / n_kv <= 4 ? 4 : 8) <= 65536),
                 "attn_decode_fused: out is required with q8, or where the partials need the merge kernel");
    G4_CHECK_ARG(n_rot > 0 && n_rot % 2 == 0 && n_rot <= hd && (2 * kAttnThreads) % n_rot == 0,
                 "attn_decode_fused: n_rot=%d (hd %d; n_rot/2 must divide %d)", n_rot, hd, kAttnThreads);
    G4_CHECK_ARG(!k_raw || (v_raw && k_norm && kstore && vstore), "attn_decode_fused: incomplete K/V append arguments");
    G4_CHECK_ARG(kv_stride >= n_kv * hd, "attn_decode_fused: kv_stride %d < n_kv*hd", kv_stride);
    AttnArgs a = {};
    a.q = q_raw; a.kc = kc; a.vc = vc; a.dpos = dpos; a.out = out; a.q8 = (uint8_t*)q8;
    a.part = part;
    a.window = window; a.kv_stride = kv_stride; a.ring = ring;
    a.n_heads = n_heads; a.n_kv = n_kv; a.hd = hd; a.scale = attn_scale; a.G = G;
    a.q_norm = q_norm; a.kraw = k_raw; a.vraw = v_raw; a.k_norm = k_norm; a.kstore = kstore; a.vstore = vstore;
    a.tab = (const float2*)rope_tab; a.n_rot = n_rot; a.eps = eps;
    return launch_attn(a);
}
