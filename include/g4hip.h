/*
 * g4hip.h -- C ABI of libg4hip.so, the MI355X (gfx950) decode-step library
 * for Gemma 4 E4B K-quant models.
 *
 * Each compute entry point is a drop-in for a function of the reference CPU
 * engine, thamada/Gemma4.c gemma4-4b/cpu-blas/main.c ("main.c" below), with
 * the same argument order and meaning.  Differences, all deliberate:
 *   - pointers are device pointers (HBM);
 *   - weight tensors are in the library's planar HBM layout, produced by
 *     g4_upload_quant() from GGUF bytes (g4_download_quant() inverts it);
 *   - Q8_K activation buffers have the library's private layout
 *     (g4_q8K_bytes(k) bytes; g4_download_q8K() gives the 292-byte
 *     BlockQ8_K structs of main.c:118-122 back, byte for byte);
 *   - every entry point returns a status (G4_OK == 0) instead of printing
 *     and exit(1)ing (main.c:609-610, 1676-1678, 1690-1692); the message is
 *     in g4_last_error().  g4e_* engine wrappers keep the exit semantics.
 * All work is enqueued asynchronously on the library stream (g4_set_stream,
 * default: the device's null stream).  Calls are not re-entrant across host
 * threads.
 */
#ifndef G4HIP_H
#define G4HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
enum {
    G4_OK = 0,
    G4_ERR_ARG = 1,     /* bad pointer / size / shape                       */
    G4_ERR_TYPE = 2,    /* unsupported tensor type (main.c:609, 1690)       */
    G4_ERR_HIP = 3,     /* HIP runtime error                                */
    G4_ERR_NOMEM = 4,
    G4_ERR_STATE = 5,   /* call out of order (e.g. before g4_init)          */
    G4_ERR_NODEV = 6,   /* no HIP device                                    */
    G4_ERR_FORMAT = 7   /* malformed GGUF (main.c:843)                      */
};

/* ggml tensor type ids, main.c:85-92 */
enum { G4_F32 = 0, G4_F16 = 1, G4_Q4_K = 12, G4_Q5_K = 13, G4_Q6_K = 14, G4_BF16 = 30 };

/* ---------------------------------------------------------------------------
 * Lifecycle and memory.  No reference counterpart (main.c keeps everything in
 * host memory); these replace the mmap/calloc of main.c:2770-2782, 1402-1423.
 * ------------------------------------------------------------------------- */
int         g4_init(int device);
int         g4_device_info(int *cus, char *arch, int arch_len);
int         g4_set_stream(void *hip_stream);
void       *g4_get_stream(void);
int         g4_sync(void);
const char *g4_last_error(void);
int         g4_malloc(void **p, size_t bytes);
int         g4_free(void *p);
int         g4_memcpy_h2d(void *dst, const void *src, size_t bytes);
int         g4_memcpy_d2h(void *dst, const void *src, size_t bytes);
int         g4_event_create(void **ev);
int         g4_event_destroy(void *ev);
int         g4_event_record(void *ev);
int         g4_event_elapsed_ms(void *start, void *stop, float *ms);

/* ---------------------------------------------------------------------------
 * Weight placement.  Replaces the borrowed mmap pointers of load_weights /
 * find_tensor (main.c:1318-1400): a GGUF tensor [d rows x n] of type
 * Q4_K/Q5_K/Q6_K is copied to HBM in the planar layout; F32/F16/BF16 are
 * copied verbatim.  g4_tensor_bytes() == the GGUF byte size
 * (row_bytes_quant, main.c:748-756, times d).
 * ------------------------------------------------------------------------- */
size_t g4_tensor_bytes(int type, int n, int d);
int    g4_upload_quant(void *dst, const void *host_gguf_bytes, int type, int n, int d);
int    g4_download_quant(void *host_gguf_bytes, const void *src, int type, int n, int d);
/* same transform, both sides on the device (raw GGUF bytes already in HBM) */
int    g4_relayout_quant(void *dst, const void *src_gguf_bytes, int type, int n, int d);

/* ---------------------------------------------------------------------------
 * Q8_K activations
 * ------------------------------------------------------------------------- */
size_t g4_q8K_bytes(int k);
/* quantize_row_q8_K(const float *x, BlockQ8_K *y, int k), main.c:282 (AVX2)
 * and main.c:247 (_ref); bit-exact with both. */
int    g4_quantize_row_q8_K(const float *x, void *y, int k);
int    g4_download_q8K(const void *y, void *host_blocks, int k);   /* -> BlockQ8_K[k/256] */
int    g4_upload_q8K(void *y, const void *host_blocks, int k);     /* BlockQ8_K[k/256] -> device */

/* ---------------------------------------------------------------------------
 * K-quant GEMV.  o[d] = W[d x n] . x, W row-major with ne[0] = n
 * (design.md:1038-1045).
 * ------------------------------------------------------------------------- */
/* vec_dot_q4_K_q8_K(int n, const BlockQ4_K *x, const BlockQ8_K *y, float *out),
 * main.c:476-529: x is a one-row tensor (d = 1); *out is a device float.
 * Bit-exact with the reference's AVX2 fp32 order. */
int g4_vec_dot_q4_K_q8_K(int n, const void *x, const void *y, float *out);
/* vec_dot_q5_K_q8_K, main.c:531-593 (AVX2 order, bit-exact) */
int g4_vec_dot_q5_K_q8_K(int n, const void *x, const void *y, float *out);
/* Q6_K x Q8_K integer dot.  No reference counterpart (the reference sends
 * Q6_K through mm_quant_rows with fp32 activations, main.c:1687-1689). */
int g4_vec_dot_q6_K_q8_K(int n, const void *x, const void *y, float *out);
/* mm_quant_dot_rows(float *o, const void *w, int n, int d, int type,
 * const BlockQ8_K *q8), main.c:1558-1566; type Q4_K/Q5_K (bit-exact per row
 * with main.c:476/531) or Q6_K (integer Q6_K x Q8_K, see above). */
int g4_mm_quant_dot_rows(float *o, const void *w, int n, int d, int type, const void *q8);
/* mm_quant_rows(float *o, const float *x, const void *w, int n, int d, int type),
 * main.c:1539-1556: dequantized weights times fp32 x. */
int g4_mm_quant_rows(float *o, const float *x, const void *w, int n, int d, int type);
/* mm_bf16 / mm_f16 / mm_f32, main.c:1494-1537 */
int g4_mm_bf16(float *o, const float *x, const void *w, int n, int d);
/* mm(float *o, const float *x, const void *w, int n, int d, int type,
 * BlockQ8_K *q8, int q8_ready), main.c:1669-1694: Q4_K/Q5_K quantize x into
 * q8 unless q8_ready, then integer dots; Q6_K -> mm_quant_rows; BF16 ->
 * mm_bf16; other types -> G4_ERR_TYPE. */
int g4_mm(float *o, const float *x, const void *w, int n, int d, int type, void *q8, int q8_ready);
/* Fused FFN up-projection: hb[i] = gelu(gate_i . x) * (up_i . x) for
 * i < d, both Q4_K/Q5_K against one Q8_K vector (main.c:1974-1980). */
int g4_mm_gate_up_gelu(float *hb, const void *gate, const void *up, int n, int d, int type, const void *q8);
/* Debug: per-block exact integer sums S_b, M_b (int32, d*nb each) of
 * Q4_K/Q5_K x Q8_K (main.c:500-523 summed over lanes). */
int g4_debug_block_sums(const void *w, int n, int d, int type, const void *q8, int32_t *S, int32_t *M);

#ifdef __cplusplus
}
#endif
#endif /* G4HIP_H */
