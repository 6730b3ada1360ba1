// layout.hip -- GGUF K-quant tensors <-> the planar HBM layout (g4_device.h).
//
// Replaces the zero-copy mmap binding of load_weights/find_tensor
// (gemma4-4b/cpu-blas/main.c:1318-1400): the same bytes are placed so that
// the GEMV lanes issue contiguous 16-byte loads.  The transform is a pure
// permutation of bytes within a tensor, so download(upload(x)) == x.
#include "g4_device.h"
#include "g4_internal.h"

namespace g4 {

// dir 0: raw GGUF blocks [b0, b0+count) -> planar tensor of nblk blocks
// dir 1: planar tensor -> raw GGUF blocks
__global__ void relayout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int type, size_t nblk,
                                size_t b0, size_t count, int dir) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const size_t blk = b0 + i;
    if (type == 12 || type == 13) {
        const int bs = type == 12 ? 144 : 176;
        const int qs_raw = type == 12 ? 16 : 48;
        const size_t hdr_off = type == 12 ? q4k_planes(nblk).hdr : q5k_planes(nblk).hdr;
        const uint8_t* rs = src + i * bs;        // raw side (dir 0)
        uint8_t* rd = dst + i * bs;              // raw side (dir 1)
        const uint8_t* ps = src;                 // planar side (dir 1)
        uint8_t* pd = dst;                       // planar side (dir 0)
        for (int c = 0; c < 16; c++) {
            if (dir == 0) pd[hdr_off + blk * 16 + c] = rs[c];
            else rd[c] = ps[hdr_off + blk * 16 + c];
        }
        if (type == 13) {
            const size_t qh_off = q5k_planes(nblk).qh;
            for (int c = 0; c < 32; c++) {
                if (dir == 0) pd[qh_off + blk * 32 + c] = rs[16 + c];
                else rd[16 + c] = ps[qh_off + blk * 32 + c];
            }
        }
        for (int w = 0; w < 32; w++) {
            const int dw = q4k_word_dev(w);
            for (int c = 0; c < 4; c++) {
                if (dir == 0) pd[blk * 128 + 4 * dw + c] = rs[qs_raw + 4 * w + c];
                else rd[qs_raw + 4 * w + c] = ps[blk * 128 + 4 * dw + c];
            }
        }
    } else {  // Q6_K
        const Q6KPlanes p = q6k_planes(nblk);
        const uint8_t* rs = src + i * 210;
        uint8_t* rd = dst + i * 210;
        for (int L = 0; L < 8; L++) {
            const int h = L >> 2, u = L & 3;
            for (int c = 0; c < 16; c++) {
                const int raw = c < 8 ? 64 * h + 8 * u + c : 64 * h + 32 + 8 * u + (c - 8);
                if (dir == 0) dst[p.ql + blk * 128 + 16 * L + c] = rs[raw];
                else rd[raw] = src[p.ql + blk * 128 + 16 * L + c];
            }
        }
        for (int c = 0; c < 64; c++) {
            if (dir == 0) dst[p.qh + blk * 64 + c] = rs[128 + c];
            else rd[128 + c] = src[p.qh + blk * 64 + c];
        }
        for (int c = 0; c < 16; c++) {
            if (dir == 0) dst[p.sc + blk * 16 + c] = rs[192 + c];
            else rd[192 + c] = src[p.sc + blk * 16 + c];
        }
        for (int c = 0; c < 2; c++) {
            if (dir == 0) dst[p.d + blk * 2 + c] = rs[208 + c];
            else rd[208 + c] = src[p.d + blk * 2 + c];
        }
    }
}

}  // namespace g4

using namespace g4;

static int block_bytes(int type) { return type == 12 ? 144 : type == 13 ? 176 : type == 14 ? 210 : 0; }

extern "C" size_t g4_tensor_bytes(int type, int n, int d) {
    if (n <= 0 || d <= 0) return 0;
    switch (type) {
    case G4_F32: return (size_t)n * d * 4;
    case G4_F16: case G4_BF16: return (size_t)n * d * 2;
    case G4_Q4_K: case G4_Q5_K: case G4_Q6_K:
        return n % 256 ? 0 : (size_t)(n / 256) * block_bytes(type) * d;
    default: return 0;
    }
}

static int check_quant(const char* who, int type, int n, int d) {
    if (type != G4_Q4_K && type != G4_Q5_K && type != G4_Q6_K)
        return g4_fail(G4_ERR_TYPE, "%s: unsupported tensor type %d", who, type);
    if (n <= 0 || d <= 0 || n % 256)
        return g4_fail(G4_ERR_ARG, "%s: n=%d d=%d (n must be a positive multiple of 256)", who, n, d);
    return G4_OK;
}

// chunked so the staging buffer stays small for multi-GB tensors
static const size_t kChunkBlocks = (size_t)1 << 20;

extern "C" int g4_relayout_quant(void* dst, const void* src, int type, int n, int d) {
    int rc = check_quant("g4_relayout_quant", type, n, d);
    if (rc) return rc;
    G4_CHECK_ARG(dst && src && dst != src, "g4_relayout_quant: bad pointers");
    const size_t nblk = (size_t)(n / 256) * d, bs = block_bytes(type);
    for (size_t b0 = 0; b0 < nblk; b0 += kChunkBlocks) {
        const size_t cnt = nblk - b0 < kChunkBlocks ? nblk - b0 : kChunkBlocks;
        hipLaunchKernelGGL(relayout_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, g4_stream(),
                           (const uint8_t*)src + b0 * bs, (uint8_t*)dst, type, nblk, b0, cnt, 0);
        rc = g4_check_launch("relayout_kernel");
        if (rc) return rc;
    }
    return G4_OK;
}

extern "C" int g4_upload_quant(void* dst, const void* host, int type, int n, int d) {
    int rc = check_quant("g4_upload_quant", type, n, d);
    if (rc) return rc;
    G4_CHECK_ARG(dst && host, "g4_upload_quant: null pointer");
    const size_t nblk = (size_t)(n / 256) * d, bs = block_bytes(type);
    const size_t chunk = nblk < kChunkBlocks ? nblk : kChunkBlocks;
    void* tmp = nullptr;
    G4_HIP(hipMalloc(&tmp, chunk * bs));
    for (size_t b0 = 0; b0 < nblk && rc == 0; b0 += kChunkBlocks) {
        const size_t cnt = nblk - b0 < kChunkBlocks ? nblk - b0 : kChunkBlocks;
        rc = g4_hip_status(hipMemcpyAsync(tmp, (const uint8_t*)host + b0 * bs, cnt * bs, hipMemcpyHostToDevice, g4_stream()));
        if (rc) break;
        hipLaunchKernelGGL(relayout_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, g4_stream(),
                           (const uint8_t*)tmp, (uint8_t*)dst, type, nblk, b0, cnt, 0);
        rc = g4_check_launch("relayout_kernel");
        if (rc == 0) rc = g4_hip_status(hipStreamSynchronize(g4_stream()));
    }
    (void)hipFree(tmp);
    return rc;
}

extern "C" int g4_download_quant(void* host, const void* src, int type, int n, int d) {
    int rc = check_quant("g4_download_quant", type, n, d);
    if (rc) return rc;
    G4_CHECK_ARG(host && src, "g4_download_quant: null pointer");
    const size_t nblk = (size_t)(n / 256) * d, bs = block_bytes(type);
    const size_t chunk = nblk < kChunkBlocks ? nblk : kChunkBlocks;
    void* tmp = nullptr;
    G4_HIP(hipMalloc(&tmp, chunk * bs));
    for (size_t b0 = 0; b0 < nblk && rc == 0; b0 += kChunkBlocks) {
        const size_t cnt = nblk - b0 < kChunkBlocks ? nblk - b0 : kChunkBlocks;
        hipLaunchKernelGGL(relayout_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, g4_stream(),
                           (const uint8_t*)src, (uint8_t*)tmp, type, nblk, b0, cnt, 1);
        rc = g4_check_launch("relayout_kernel");
        if (rc == 0)
            rc = g4_hip_status(hipMemcpyAsync((uint8_t*)host + b0 * bs, tmp, cnt * bs, hipMemcpyDeviceToHost, g4_stream()));
        if (rc == 0) rc = g4_hip_status(hipStreamSynchronize(g4_stream()));
    }
    (void)hipFree(tmp);
    return rc;
}
