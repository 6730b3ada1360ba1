// probe.hip -- measurement probes for the floors the decode-step design is
// sized against (bench.py --workload floors): what a dependent launch costs
// with no work in it, how fast a plain streaming read runs at the byte counts
// of the step's kernels, and what handing results from every workgroup to one
// last workgroup costs inside a kernel instead of through a launch boundary.
// They compute nothing of the model.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {
namespace {

// nothing: the cost of one launch in a chain of dependent launches
__global__ __launch_bounds__(64) void probe_empty_kernel() {}

// streaming read of n4 float4 with 1 KB per wave instruction (one float4 per
// lane, U loads in flight per lane before any is used); each workgroup adds
// its values and writes one float, so nothing is optimised away
constexpr int kProbeU = 8;
__global__ __launch_bounds__(256) void probe_read_kernel(const float4* __restrict__ p, size_t n4,
                                                         float* __restrict__ sink) {
    __shared__ float red[16];
    const size_t stride = (size_t)gridDim.x * 256 * kProbeU;
    float acc = 0.0f;
    for (size_t base = (size_t)blockIdx.x * 256 * kProbeU + threadIdx.x; base < n4; base += stride) {
        float4 v[kProbeU];
#pragma unroll
        for (int u = 0; u < kProbeU; u++) {
            const size_t i = base + (size_t)u * 256;
            v[u] = p[i < n4 ? i : n4 - 1];
        }
#pragma unroll
        for (int u = 0; u < kProbeU; u++) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    acc = block_sum(acc, red);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

// every workgroup writes kHandVals values and counts itself in; the one
// that arrives last reads every value (all its loads issued at once) and
// resets the counter for the next launch: the in-kernel alternative to a
// second launch.  mode 0: the stores only (the baseline); 1: plain stores,
// a device-scope release fence before the count and an acquire after it;
// 2: the values stored and read as device-scope relaxed atomics (coherent
// without the L2 write-back of a release fence), the count issued once the
// stores have completed.
constexpr int kHandVals = 16;
constexpr int kHandMaxPerThread = 40;   // 640 workgroups x 16 values over 256 threads
__global__ __launch_bounds__(256) void probe_handoff_kernel(float* __restrict__ vals, unsigned int* __restrict__ count,
                                                            float* __restrict__ out, int mode) {
    __shared__ int last;
    __shared__ float red[4];
    const int tid = threadIdx.x;
    const float v = (float)(blockIdx.x * kHandVals + tid);
    float* const dst = vals + blockIdx.x * kHandVals + tid;
    if (mode == 2) {
        if (tid < kHandVals) __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (tid < kHandVals) {
        *dst = v;
    }
    if (mode == 0) return;
    if (mode == 2) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        if (mode == 1) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    if (mode == 1) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const int n = gridDim.x * kHandVals;
    float x[kHandMaxPerThread];
#pragma unroll
    for (int j = 0; j < kHandMaxPerThread; j++) {
        const int i = min(tid + 256 * j, n - 1);
        x[j] = mode == 2 ? __hip_atomic_load(vals + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : vals[i];
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kHandMaxPerThread; j++) s += tid + 256 * j < n ? x[j] : 0.0f;
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        *out = (red[0] + red[1]) + (red[2] + red[3]);
        __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace
}  // namespace g4

using namespace g4;

extern "C" int g4_probe_empty(int workgroups) {
    G4_CHECK_ARG(workgroups > 0, "g4_probe_empty: workgroups=%d", workgroups);
    hipLaunchKernelGGL(probe_empty_kernel, dim3(workgroups), dim3(64), 0, g4_stream());
    return g4_check_launch("probe_empty_kernel");
}

extern "C" int g4_probe_read(const void* p, size_t bytes, float* sink, int workgroups) {
    G4_CHECK_ARG(p && sink && bytes >= 16 && bytes % 16 == 0 && workgroups > 0, "g4_probe_read: bad arguments");
    G4_CHECK_ARG(((uintptr_t)p & 15) == 0, "g4_probe_read: p must be 16-byte aligned");
    hipLaunchKernelGGL(probe_read_kernel, dim3(workgroups), dim3(256), 0, g4_stream(), (const float4*)p, bytes / 16,
                       sink);
    return g4_check_launch("probe_read_kernel");
}

extern "C" int g4_probe_handoff(float* vals, unsigned int* count, float* out, int workgroups, int mode) {
    G4_CHECK_ARG(vals && count && out && workgroups > 0 && workgroups * kHandVals <= 256 * kHandMaxPerThread &&
                     mode >= 0 && mode <= 2,
                 "g4_probe_handoff: bad arguments (workgroups %d, mode %d)", workgroups, mode);
    hipLaunchKernelGGL(probe_handoff_kernel, dim3(workgroups), dim3(256), 0, g4_stream(), vals, count, out, mode);
    return g4_check_launch("probe_handoff_kernel");
}
