// sample.hip -- the reference's token sampler on the device, so that a
// sampled decode step needs no logits read-back and can be replayed as one
// HIP graph together with the forward pass.
//
// Reference (gemma4-4b/cpu-blas/main.c):
//   apply_repetition_penalty  2114-2126 (generate applies it at 2408-2410 to
//                             the tokens generated so far, before sampling)
//   rng_f32 (xorshift64*)     2035-2040
//   sample_token              2044-2112: temp <= 0: first index of the
//                             maximum; else insertion top-k (DEFAULT_TOP_K 40),
//                             softmax((v - max) / temp) with sequential fp32
//                             sums, then a plain draw or a top-p draw
//
// Top-k.  The insertion sort keeps equal values in index order and admits a
// value at the full list's end only if it is strictly larger, so its list
// is the first k of all (value descending, index ascending) pairs.  A 64-bit
// key (order-preserving value bits, then the complemented index) orders the
// pairs exactly so; selecting the k largest keys reproduces the list.
//
// Selection of the k largest of a workgroup's keys (16 per thread) without
// sequential pops: each thread's largest key (its head) is ranked among the
// 256 heads; T = the k-th largest head.  The k heads >= T are k keys, so the
// k largest keys are all >= T: those keys (about k for k << 256) are gathered
// in LDS and each one's rank among them (the number of larger ones; keys are
// distinct) is its position in the descending list.  Zero keys fill the
// positions past the last real key.
//
// Pass 1 (G = n / 4096 workgroups): the penalty for the ids of the
// workgroup's slice (occurrences in the history window counted in LDS, each
// logit penalised that many times, written back to the logits as the
// reference does), then the slice's k largest keys.  Pass 2 (one workgroup):
// the same selection over the G*k candidates, then wave 0 runs the
// reference's softmax / top-p / draw over the k sorted values: the
// exponentials one per lane, the sums and cdf walks in the reference's
// sequential order over the lanes' values.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {
namespace {

constexpr int kSampleThreads = 256;
constexpr int kSamplePer = 4096;            // logits per pass-1 workgroup (16 per thread)
constexpr int kSampleMaxK = 64;
constexpr int kSampleMaxParts = 64;         // pass 2 holds kSampleMaxParts * kSampleMaxK keys

typedef unsigned long long u64;

// A NaN logit gets key 0, below every number: the reference's insertion
// (main.c:2055-2073) compares with '<' and '>', which a NaN never passes once
// the list holds topk entries.  (A NaN among the first topk logits would
// enter the reference's list unordered; the keys treat it as masked.)
__device__ __forceinline__ u64 sample_key(float v, int i) {
    if (v != v) return 0;
    uint32_t u = __float_as_uint(v + 0.0f);   // -0.0 == +0.0, as the C comparison
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((u64)u << 32) | (uint32_t)(~(uint32_t)i);
}
__device__ __forceinline__ float key_value(u64 k) {
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
    return __uint_as_float(u);
}
__device__ __forceinline__ int key_index(u64 k) { return (int)(~(uint32_t)(k & 0xffffffffu)); }

// out[0..kk) = the kk largest of the workgroup's keys k[0..R) per thread,
// descending (kk <= 64 <= 4 * blockDim.x / 16).  hb: blockDim.x keys of LDS,
// cand: R * blockDim.x keys of LDS, misc: two words of LDS.  out may be LDS
// or global; every thread reaches every barrier.
template <int R>
__device__ void wg_topk(const u64 (&k)[R], int kk, u64* out, u64* hb, u64* cand, u64* misc) {
    const int tid = threadIdx.x, nt = blockDim.x;
    u64 head = k[0];
#pragma unroll
    for (int j = 1; j < R; j++) head = k[j] > head ? k[j] : head;
    hb[tid] = head;
    if (tid == 0) { misc[0] = ~0ull; misc[1] = 0ull; }
    if (tid < kk) out[tid] = 0ull;
    __syncthreads();
    int r = 0;
#pragma unroll 16
    for (int j = 0; j < nt; j += 2) {   // 16 reads in flight per wait
        const ulonglong2 h2 = *reinterpret_cast<const ulonglong2*>(hb + j);
        r += (h2.x > head) + (h2.y > head);
    }
    // T = the smallest head ranked below kk (heads are distinct keys or 0)
    if (r < kk) atomicMin(&misc[0], head);
    __syncthreads();
    const u64 T = misc[0];
    unsigned int* cnt = reinterpret_cast<unsigned int*>(&misc[1]);
#pragma unroll
    for (int j = 0; j < R; j++)
        if (k[j] >= T) cand[atomicAdd(cnt, 1u)] = k[j];
    __syncthreads();
    // thread t ranks candidate t (one pass for the workgroup; zero keys are
    // the pre-filled tail)
    const int C = (int)*cnt;
    for (int t = tid; t < C; t += nt) {
        const u64 v = cand[t];
        if (v == 0ull) continue;
        int rank = 0;
#pragma unroll 8
        for (int i = 0; i < C; i++) rank += cand[i] > v;
        if (rank < kk) out[rank] = v;
    }
}

struct SampleArgs {
    float* logits;
    int n, topk;
    int* hist;             // generated tokens (device), *hist_n of them
    int* hist_n;
    int hist_cap;
    float penalty;
    int last_n;
    float temp, topp;
    u64* rng;
    u64* part;
    int* out;
    int* dtok;
    int* dpos;
};

// Pass 1: workgroup g takes logits [4096 g, 4096 g + 4096).  Every thread
// loads its 16 logits first (clamped indices: no load waits on a lane
// condition); meanwhile the workgroup counts, in LDS, how often each logit of
// the slice occurs in the penalty window of the token history; each logit is
// then penalised that many times (main.c:2408-2430 applies the penalty once
// per occurrence, in history order; the operation keeps the sign, so c
// occurrences are c applications of the same step) and written back if it
// changed; then the slice's top-k keys go to part[g].
__global__ __launch_bounds__(kSampleThreads) void sample_partial_kernel(SampleArgs a) {
    __shared__ __align__(16) u64 hb[kSampleThreads];
    __shared__ u64 misc[2];
    __shared__ u64 cand[kSamplePer];
    int* cnt = reinterpret_cast<int*>(cand);   // the penalty counts, done before the selection
    const int tid = threadIdx.x;
    const int base = blockIdx.x * kSamplePer;
    const int end = min(base + kSamplePer, a.n);
    float v[16];
    if (end - base == kSamplePer) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 t = *reinterpret_cast<const float4*>(a.logits + base + 4 * (tid + kSampleThreads * q));
            v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = a.logits[min(base + 4 * (tid + kSampleThreads * (j >> 2)) + (j & 3), end - 1)];
    }
    const bool pen = a.penalty > 1.0f;
    if (pen) {
        for (int i = tid; i < kSamplePer; i += kSampleThreads) cnt[i] = 0;
        __syncthreads();
        const int nh = min(*a.hist_n, a.hist_cap);
        const int start = a.last_n > 0 && nh > a.last_n ? nh - a.last_n : 0;
        for (int i = start + tid; i < nh; i += kSampleThreads) {
            const int id = a.hist[i];
            if (id >= base && id < end) atomicAdd(&cnt[id - base], 1);
        }
        __syncthreads();
    }
    u64 k[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int i = base + 4 * (tid + kSampleThreads * (j >> 2)) + (j & 3);
        if (pen && i < end) {
            const int c = cnt[i - base];
            if (c > 0) {
                float x = v[j];
                for (int r = 0; r < c; r++) x = x >= 0.0f ? x / a.penalty : x * a.penalty;
                v[j] = x;
                a.logits[i] = x;
            }
        }
        k[j] = sample_key(v[j], i) & (i < end ? ~0ull : 0ull);
    }
    wg_topk<16>(k, a.topk, a.part + (size_t)blockIdx.x * kSampleMaxK, hb, cand, misc);
}

__device__ __forceinline__ float rng_f32(u64* s) {
    u64 x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return (float)((x * 0x2545F4914F6CDD1DULL) >> 40) / (float)(1 << 24);
}

__device__ __forceinline__ float lane_val(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

__global__ __launch_bounds__(kSampleThreads) void sample_final_kernel(SampleArgs a, int G) {
    __shared__ __align__(16) u64 hb[kSampleThreads];
    __shared__ u64 misc[2], top[kSampleMaxK];
    __shared__ u64 cand[16 * kSampleThreads];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // thread t holds entries 16 (t & 3) .. +15 of list t / 4 (G <= 64), so
    // the heads include every list's maximum: a tight threshold.  (Every
    // lane loads: clamped into the G lists, masked after.)
    const int wl = tid >> 2, r0 = 16 * (tid & 3);
    u64 k[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int c = wl * kSampleMaxK + r0 + j;
        k[j] = a.part[min(c, G * kSampleMaxK - 1)] & (wl < G && r0 + j < a.topk ? ~0ull : 0ull);
    }
    wg_topk<16>(k, a.topk, top, hb, cand, misc);
    __syncthreads();
    if (wave != 0) return;
    // wave 0, every lane the same path: lane i holds the i-th value's weight
    int result;
    if (a.temp <= 0.0f) {
        result = key_index(top[0]);
    } else {
        // sample_token (main.c:2090-2112) over the sorted top-k
        const int np = a.topk;
        const float mx = key_value(top[0]);
        const float e = lane < np ? expf((key_value(top[lane]) - mx) / a.temp) : 0.0f;
        float sum = 0.0f;
        for (int i = 0; i < np; i++) sum += lane_val(e, i);
        const float pl = e / sum;
        u64 st = *a.rng;
        const float coin = rng_f32(&st);
        if (a.topp <= 0.0f || a.topp >= 1.0f) {
            float cdf = 0.0f;
            result = key_index(top[np - 1]);
            for (int i = 0; i < np; i++) {
                cdf += lane_val(pl, i);
                if (coin < cdf) { result = key_index(top[i]); break; }
            }
        } else {
            float cum = 0.0f;
            int last = np - 1;
            for (int i = 0; i < np; i++) {
                cum += lane_val(pl, i);
                if (cum > a.topp) { last = i; break; }
            }
            const float r = rng_f32(&st) * cum;
            float cdf = 0.0f;
            result = key_index(top[last]);
            for (int i = 0; i <= last; i++) {
                cdf += lane_val(pl, i);
                if (r < cdf) { result = key_index(top[i]); break; }
            }
        }
        if (lane == 0) *a.rng = st;
    }
    if (lane != 0) return;
    if (a.out) *a.out = result;
    if (a.dtok) *a.dtok = result;
    if (a.dpos) *a.dpos = *a.dpos + 1;
    if (a.hist_n) {
        const int nh = *a.hist_n;
        if (nh < a.hist_cap) {
            a.hist[nh] = result;
            *a.hist_n = nh + 1;
        }
    }
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" size_t g4_sample_part_bytes(int n) {
    return n > 0 ? (size_t)((n + kSamplePer - 1) / kSamplePer) * kSampleMaxK * sizeof(u64) : 0;
}

extern "C" int g4_sample(float* logits, int n, float temp, float topp, int topk, float penalty, int penalty_last_n,
                         int* hist, int* hist_n, int hist_cap, unsigned long long* rng, void* part, int* out, int* dtok,
                         int* dpos) {
    G4_CHECK_ARG(logits && part && n > 0, "g4_sample: bad arguments");
    G4_CHECK_ARG(((uintptr_t)logits & 15) == 0, "g4_sample: logits must be 16-byte aligned");
    const int G = (n + kSamplePer - 1) / kSamplePer;
    G4_CHECK_ARG(G <= kSampleMaxParts, "g4_sample: n=%d exceeds %d", n, kSampleMaxParts * kSamplePer);
    G4_CHECK_ARG(topk >= 1 && topk <= kSampleMaxK && topk <= n, "g4_sample: top-k %d not in 1..%d", topk,
                 kSampleMaxK);
    G4_CHECK_ARG(temp <= 0.0f || rng, "g4_sample: sampling needs the rng state");
    G4_CHECK_ARG(penalty <= 1.0f || (hist && hist_n), "g4_sample: the penalty needs the token history");
    G4_CHECK_ARG(!hist_n || (hist && hist_cap >= 0), "g4_sample: history without storage");
    SampleArgs a = {};
    a.logits = logits; a.n = n; a.topk = temp <= 0.0f ? 1 : topk;
    a.hist = hist; a.hist_n = hist_n; a.hist_cap = hist_cap;
    a.penalty = penalty; a.last_n = penalty_last_n;
    a.temp = temp; a.topp = topp; a.rng = rng; a.part = (u64*)part;
    a.out = out; a.dtok = dtok; a.dpos = dpos;
    hipLaunchKernelGGL(sample_partial_kernel, dim3(G), dim3(kSampleThreads), 0, g4_stream(), a);
    int rc = g4_check_launch("sample_partial_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(sample_final_kernel, dim3(1), dim3(kSampleThreads), 0, g4_stream(), a, G);
    return g4_check_launch("sample_final_kernel");
}
