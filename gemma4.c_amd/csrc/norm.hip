// norm.hip -- RMSNorm family on gfx950, plus the fused residual/norm/quantize
// step kernel of the decode engine.
//
// Reference operations (gemma4-4b/cpu-blas/main.c):
//   rmsnorm                       1451-1456: o[i] = (x[i] * s) * w[i]
//   rmsnorm_head_inplace          1458-1466: v[i] = v[i] * (s * w[i])
//   rmsnorm_head_noweight_inplace 1468-1476: v[i] = v[i] * s
// with s = 1 / sqrtf(sum(x^2) / n + eps).  The elementwise products are
// evaluated in the reference's order; the sum of squares is a tree (the
// reference sums sequentially), so results agree to fp32 tolerance.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

constexpr int kNormThreads = 1024;

// rms scale of x[0..n) by the whole workgroup
__device__ __forceinline__ float rms_scale(const float* __restrict__ x, int n, float eps, float* red) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, red);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(float* __restrict__ o, const float* __restrict__ x,
                                                               const float* __restrict__ w, int n, float eps) {
    __shared__ float red[16];
    const float s = rms_scale(x, n, eps, red);
    for (int i = threadIdx.x; i < n; i += blockDim.x) o[i] = (x[i] * s) * w[i];
}

// one workgroup per head; w == nullptr is the no-weight variant
__global__ __launch_bounds__(256) void rmsnorm_heads_kernel(float* __restrict__ v, const float* __restrict__ w, int hd,
                                                            float eps) {
    __shared__ float red[16];
    float* seg = v + (size_t)blockIdx.x * hd;
    const float s = rms_scale(seg, hd, eps, red);
    __syncthreads();   // every thread has read seg before it is overwritten
    for (int i = threadIdx.x; i < hd; i += blockDim.x) seg[i] = w ? seg[i] * (s * w[i]) : seg[i] * s;
}

// ---------------------------------------------------------------------------
// Fused step kernel (one workgroup, n <= kResidualMax):
//   if y:       x[i] = x[i] + (y[i] * s_y) * w_post[i]        (main.c:1960-1962,
//               1982-1984, 1995-1997: post-norm then residual add)
//   if oscale:  x[i] = x[i] * oscale[0]                       (main.c:1999-2003)
//   if w_next:  xb2[i] = (x[i] * s_x) * w_next[i]             (main.c:1878, 1973)
//   if q8:      q8 = quantize_row_q8_K(qsrc == 0 ? xb2 : x)   (main.c:1884, 1975)
// ---------------------------------------------------------------------------
constexpr int kResidualMax = 16384;

// EPT elements per thread (n <= EPT * blockDim.x)
template <int EPT>
__global__ __launch_bounds__(kNormThreads) void residual_norm_kernel(ResidualArgs a) {
    extern __shared__ __align__(16) float buf[];   // n floats: the vector to quantize
    __shared__ float red[16];
    residual_core<EPT>(a, buf, red, true);
    if (a.q8) {
        __syncthreads();
        quantize_blocks_wg(buf, a.q8, a.n / 256);
    }
}

// The same step with one float4 of each vector per thread (n/4 threads, n a
// multiple of 256 up to 4096; residual4_load / residual4_finish): wave w
// holds Q8_K block w and quantizes it from its registers (no LDS round trip),
// with one LDS-only barrier per norm.  The residual prologues of
// g4_mm_residual_q8 run the same code, so for these n every form of the step
// gives the same bits.  Row z = blockIdx.x of m rows (x, y, xb2 n apart, q8
// rows q8row bytes apart; m = 1: the decode step).
__global__ __launch_bounds__(1024) void residual4_kernel(ResidualArgs a, size_t q8row) {
    __shared__ float red[2][16];
    const size_t off = (size_t)blockIdx.x * a.n;
    Res4 r;
    residual4_load(a, r, off);
    float q[4], nv[4];
    residual4_finish(a, r, red, true, off, q, nv);
    if (a.q8) quantize_block_wave(q, threadIdx.x & 63, a.q8 + blockIdx.x * q8row, a.n / 256, threadIdx.x >> 6);
}

bool residual4_ok(const void* x, const void* y, const void* xb2, int n) {
    auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    return n % 256 == 0 && n <= 4096 && al(x) && al(y) && al(xb2);
}

// row z = blockIdx.x of m rows of n (x, y, xb2 n apart; q8 rows q8row bytes
// apart): the same step per row as residual_norm_kernel (same thread count
// and reduction tree when launched with the same EPT and block size)
template <int EPT>
__global__ __launch_bounds__(kNormThreads) void residual_rows_kernel(ResidualArgs a, size_t q8row) {
    extern __shared__ __align__(16) float buf[];
    __shared__ float red[16];
    const size_t z = blockIdx.x, off = z * (size_t)a.n;
    a.x += off;
    a.x_out += off;
    if (a.y) a.y += off;
    if (a.xb2) a.xb2 += off;
    if (a.q8) a.q8 += z * q8row;
    residual_core<EPT>(a, buf, red, true);
    if (a.q8) {
        __syncthreads();
        quantize_blocks_wg(buf, a.q8, a.n / 256);
    }
}

}  // namespace g4

using namespace g4;

extern "C" int g4_residual_norm(float* x, const float* y, const float* w_post, const float* oscale, const float* w_next,
                     float* xb2, void* q8, int qsrc, int n, float eps) {
    G4_CHECK_ARG(x && n > 0 && n <= kResidualMax, "residual_norm: bad x or n=%d", n);
    G4_CHECK_ARG(!y || w_post, "residual_norm: y without w_post");
    G4_CHECK_ARG(!q8 || n % 256 == 0, "residual_norm: n=%d not a multiple of 256 for Q8_K", n);
    G4_CHECK_ARG(!(q8 && qsrc == 0) || w_next, "residual_norm: quantizing xb2 needs w_next");
    ResidualArgs a{x, x, y, w_post, oscale, w_next, xb2, (uint8_t*)q8, qsrc, n, eps};
    if (residual4_ok(x, y, xb2, n) && (!y || ((uintptr_t)w_post & 15) == 0) && (!w_next || ((uintptr_t)w_next & 15) == 0)) {
        hipLaunchKernelGGL(residual4_kernel, dim3(1), dim3(n / 4), 0, g4_stream(), a, (size_t)0);
        return g4_check_launch("residual4_kernel");
    }
    // EPT elements per thread, as few waves as cover n (n = 2560: 640 threads,
    // one wave per Q8_K block)
    const int ept = n <= kNormThreads ? 1 : n <= 4 * kNormThreads ? 4 : 16;
    const int nt = ((n + ept - 1) / ept + 63) / 64 * 64;
    const dim3 g(1), b(nt);
    const size_t lds = (size_t)n * 4;
    if (ept == 1) hipLaunchKernelGGL(residual_norm_kernel<1>, g, b, lds, g4_stream(), a);
    else if (ept == 4) hipLaunchKernelGGL(residual_norm_kernel<4>, g, b, lds, g4_stream(), a);
    else hipLaunchKernelGGL(residual_norm_kernel<16>, g, b, lds, g4_stream(), a);
    return g4_check_launch("residual_norm_kernel");
}

// g4_residual_norm over m rows (in place on x; y, xb2 n apart; Q8_K rows of
// q8 g4_q8K_row_stride(n) bytes apart).  narrow = 0: the thread layout of
// g4_residual_norm; narrow = 1: 256 threads of n/256 elements, the layout of
// the residual prologues of g4_mm_residual_q8 (n = 2048, 2560 or 4096).
extern "C" int g4_residual_norm_rows(float* x, const float* y, const float* w_post, const float* oscale,
                                     const float* w_next, float* xb2, void* q8, int qsrc, int n, float eps, int m,
                                     int narrow) {
    G4_CHECK_ARG(x && n > 0 && n <= kResidualMax && m > 0, "residual_norm_rows: bad x, n=%d or m=%d", n, m);
    G4_CHECK_ARG(!y || w_post, "residual_norm_rows: y without w_post");
    G4_CHECK_ARG(!q8 || n % 256 == 0, "residual_norm_rows: n=%d not a multiple of 256 for Q8_K", n);
    G4_CHECK_ARG(!(q8 && qsrc == 0) || w_next, "residual_norm_rows: quantizing xb2 needs w_next");
    G4_CHECK_ARG(!narrow || n == 2048 || n == 2560 || n == 4096, "residual_norm_rows: narrow layout needs n = 2048, 2560 or 4096");
    ResidualArgs a{x, x, y, w_post, oscale, w_next, xb2, (uint8_t*)q8, qsrc, n, eps};
    const size_t q8row = g4_q8K_row_stride(n);
    const size_t lds = (size_t)n * 4;
    const bool four = residual4_ok(x, y, xb2, n) && (!y || ((uintptr_t)w_post & 15) == 0) &&
                      (!w_next || ((uintptr_t)w_next & 15) == 0);
    G4_CHECK_ARG(!narrow || four, "residual_norm_rows: the prologue layout needs 16-byte aligned x, y, xb2 and weights");
    if (four) {
        // the layout of g4_residual_norm and of the GEMV prologues for these
        // n (narrow or not), so each row's bits are theirs
        hipLaunchKernelGGL(residual4_kernel, dim3(m), dim3(n / 4), 0, g4_stream(), a, q8row);
        return g4_check_launch("residual4_kernel");
    } else {
        const int ept = n <= kNormThreads ? 1 : n <= 4 * kNormThreads ? 4 : 16;
        const int nt = ((n + ept - 1) / ept + 63) / 64 * 64;
        const dim3 g(m), b(nt);
        if (ept == 1) hipLaunchKernelGGL(residual_rows_kernel<1>, g, b, lds, g4_stream(), a, q8row);
        else if (ept == 4) hipLaunchKernelGGL(residual_rows_kernel<4>, g, b, lds, g4_stream(), a, q8row);
        else hipLaunchKernelGGL(residual_rows_kernel<16>, g, b, lds, g4_stream(), a, q8row);
    }
    return g4_check_launch("residual_rows_kernel");
}

extern "C" int g4_rmsnorm(float* o, const float* x, const float* w, int n, float eps) {
    G4_CHECK_ARG(o && x && w && n > 0, "g4_rmsnorm: bad arguments (n=%d)", n);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(kNormThreads), 0, g4_stream(), o, x, w, n, eps);
    return g4_check_launch("rmsnorm_kernel");
}

extern "C" int g4_rmsnorm_head_inplace(float* v, const float* w, int n_heads, int hd, float eps) {
    G4_CHECK_ARG(v && w && n_heads > 0 && hd > 0, "g4_rmsnorm_head_inplace: bad arguments");
    hipLaunchKernelGGL(rmsnorm_heads_kernel, dim3(n_heads), dim3(256), 0, g4_stream(), v, w, hd, eps);
    return g4_check_launch("rmsnorm_heads_kernel");
}

extern "C" int g4_rmsnorm_head_noweight_inplace(float* v, int n_heads, int hd, float eps) {
    G4_CHECK_ARG(v && n_heads > 0 && hd > 0, "g4_rmsnorm_head_noweight_inplace: bad arguments");
    hipLaunchKernelGGL(rmsnorm_heads_kernel, dim3(n_heads), dim3(256), 0, g4_stream(), v, nullptr, hd, eps);
    return g4_check_launch("rmsnorm_heads_kernel");
}

// softmax(float *x, int n), main.c:1478-1488: max, x = expf(x - max), divide
// by the sum (one workgroup; the sum is a tree)
__global__ __launch_bounds__(kNormThreads) void softmax_kernel(float* __restrict__ x, int n) {
    __shared__ float red[16];
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
    m = wave_max(m);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float mx = -INFINITY;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) mx = fmaxf(mx, red[i]);
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float e = expf(x[i] - mx);
        x[i] = e;
        s += e;
    }
    s = block_sum(s, red);
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = x[i] / s;
}

extern "C" int g4_softmax(float* x, int n) {
    G4_CHECK_ARG(x && n > 0, "g4_softmax: bad arguments");
    hipLaunchKernelGGL(softmax_kernel, dim3(1), dim3(kNormThreads), 0, g4_stream(), x, n);
    return g4_check_launch("softmax_kernel");
}
