// q8k.hip -- Q8_K activation quantization on gfx950 (drop-in for
// quantize_row_q8_K, gemma4-4b/cpu-blas/main.c:247-340).
//
// One wavefront per 256-element block; lane t owns elements 4t..4t+3.
// Bit-exact with the reference: first index of max |x| wins (strict '>'
// scan, main.c:252-257), iscale = -127/maxv and d = 1/iscale with IEEE
// division, round-half-even, clamp at +127 only, zero block -> all zero.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float* __restrict__ x, uint8_t* __restrict__ y,
                                                             int nb) {
    const int b = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int lane = threadIdx.x & 63;
    if (b >= nb) return;   // uniform per wave
    const float4 f = reinterpret_cast<const float4*>(x + (size_t)b * 256)[lane];
    const float v[4] = {f.x, f.y, f.z, f.w};
    quantize_block_wave(v, lane, y, nb, b);
}

// device Q8_K layout -> reference BlockQ8_K[nb] (292 B each), for tests;
// row blockIdx.y of a batch starts ystride bytes after the previous one
__global__ void q8k_to_ref_kernel(const uint8_t* __restrict__ y, uint8_t* __restrict__ out, int nb, size_t ystride) {
    const int b = blockIdx.x;
    const int t = threadIdx.x;   // 64 threads: word t of GGUF order
    if (b >= nb) return;
    y += blockIdx.y * ystride;
    uint8_t* o = out + ((size_t)blockIdx.y * nb + b) * 292;
    const uint32_t w = reinterpret_cast<const uint32_t*>(y + (size_t)b * 256)[q8k_word_dev(t)];
    for (int e = 0; e < 4; e++) o[4 + 4 * t + e] = (uint8_t)(w >> (8 * e));
    if (t < 16) {
        const int16_t s = reinterpret_cast<const int16_t*>(y + q8k_bsums_off(nb))[b * 16 + t];
        o[260 + 2 * t] = (uint8_t)(s & 0xff);
        o[261 + 2 * t] = (uint8_t)((uint16_t)s >> 8);
    }
    if (t == 0) {
        const uint32_t d = __float_as_uint(reinterpret_cast<const float*>(y + q8k_d_off(nb))[b]);
        for (int e = 0; e < 4; e++) o[e] = (uint8_t)(d >> (8 * e));
    }
}

// reference BlockQ8_K[nb] -> device layout (tests feed shared fixtures)
__global__ void q8k_from_ref_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ y, int nb) {
    const int b = blockIdx.x;
    const int t = threadIdx.x;
    if (b >= nb) return;
    const uint8_t* s = in + (size_t)b * 292;
    const uint32_t w = (uint32_t)s[4 + 4 * t] | ((uint32_t)s[5 + 4 * t] << 8) | ((uint32_t)s[6 + 4 * t] << 16) |
                       ((uint32_t)s[7 + 4 * t] << 24);
    reinterpret_cast<uint32_t*>(y + (size_t)b * 256)[q8k_word_dev(t)] = w;
    if (t < 16) {
        const int16_t v = (int16_t)((uint16_t)s[260 + 2 * t] | ((uint16_t)s[261 + 2 * t] << 8));
        reinterpret_cast<int16_t*>(y + q8k_bsums_off(nb))[b * 16 + t] = v;
    }
    if (t == 0) {
        const uint32_t d = (uint32_t)s[0] | ((uint32_t)s[1] << 8) | ((uint32_t)s[2] << 16) | ((uint32_t)s[3] << 24);
        reinterpret_cast<float*>(y + q8k_d_off(nb))[b] = __uint_as_float(d);
    }
}

}  // namespace g4

using namespace g4;

extern "C" int g4_quantize_row_q8_K(const float* x, void* y, int k) {
    G4_CHECK_ARG(x && y, "g4_quantize_row_q8_K: null pointer");
    G4_CHECK_ARG(k > 0 && k % 256 == 0, "g4_quantize_row_q8_K: k=%d is not a positive multiple of 256", k);
    const int nb = k / 256;
    hipLaunchKernelGGL(quantize_q8k_kernel, dim3((nb + 3) / 4), dim3(256), 0, g4_stream(), x, (uint8_t*)y, nb);
    return g4_check_launch("quantize_q8k_kernel");
}

extern "C" int g4_download_q8K(const void* y, void* host_blocks, int k) {
    G4_CHECK_ARG(y && host_blocks, "g4_download_q8K: null pointer");
    G4_CHECK_ARG(k > 0 && k % 256 == 0, "g4_download_q8K: k=%d is not a positive multiple of 256", k);
    const int nb = k / 256;
    void* tmp = nullptr;
    G4_HIP(hipMalloc(&tmp, (size_t)nb * 292));
    hipLaunchKernelGGL(q8k_to_ref_kernel, dim3(nb), dim3(64), 0, g4_stream(), (const uint8_t*)y, (uint8_t*)tmp, nb,
                       (size_t)0);
    int rc = g4_check_launch("q8k_to_ref_kernel");
    if (rc == 0) rc = g4_hip_status(hipMemcpyAsync(host_blocks, tmp, (size_t)nb * 292, hipMemcpyDeviceToHost, g4_stream()));
    if (rc == 0) rc = g4_hip_status(hipStreamSynchronize(g4_stream()));
    (void)hipFree(tmp);
    return rc;
}

extern "C" int g4_download_q8K_rows(const void* y, void* host_blocks, int k, int m) {
    G4_CHECK_ARG(y && host_blocks, "g4_download_q8K_rows: null pointer");
    G4_CHECK_ARG(k > 0 && k % 256 == 0, "g4_download_q8K_rows: k=%d is not a positive multiple of 256", k);
    G4_CHECK_ARG(m > 0 && m <= 65535, "g4_download_q8K_rows: m=%d rows (1..65535)", m);
    const int nb = k / 256;
    const size_t bytes = (size_t)m * nb * 292;
    void* tmp = nullptr;
    G4_HIP(hipMalloc(&tmp, bytes));
    hipLaunchKernelGGL(q8k_to_ref_kernel, dim3(nb, m), dim3(64), 0, g4_stream(), (const uint8_t*)y, (uint8_t*)tmp, nb,
                       g4_q8K_row_stride(k));
    int rc = g4_check_launch("q8k_to_ref_kernel");
    if (rc == 0) rc = g4_hip_status(hipMemcpyAsync(host_blocks, tmp, bytes, hipMemcpyDeviceToHost, g4_stream()));
    if (rc == 0) rc = g4_hip_status(hipStreamSynchronize(g4_stream()));
    (void)hipFree(tmp);
    return rc;
}

extern "C" int g4_upload_q8K(void* y, const void* host_blocks, int k) {
    G4_CHECK_ARG(y && host_blocks, "g4_upload_q8K: null pointer");
    G4_CHECK_ARG(k > 0 && k % 256 == 0, "g4_upload_q8K: k=%d is not a positive multiple of 256", k);
    const int nb = k / 256;
    void* tmp = nullptr;
    G4_HIP(hipMalloc(&tmp, (size_t)nb * 292));
    int rc = g4_hip_status(hipMemcpyAsync(tmp, host_blocks, (size_t)nb * 292, hipMemcpyHostToDevice, g4_stream()));
    if (rc == 0) {
        hipLaunchKernelGGL(q8k_from_ref_kernel, dim3(nb), dim3(64), 0, g4_stream(), (const uint8_t*)tmp, (uint8_t*)y, nb);
        rc = g4_check_launch("q8k_from_ref_kernel");
    }
    if (rc == 0) rc = g4_hip_status(hipStreamSynchronize(g4_stream()));
    (void)hipFree(tmp);
    return rc;
}

extern "C" size_t g4_q8K_bytes(int k) { return k > 0 ? (size_t)(k / 256) * 292 : 0; }
