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
/* m Q8_K rows of k elements, g4_q8K_row_stride(k) bytes apart (the batched
 * forms' layout) -> BlockQ8_K[m][k/256]; for tests and traces */
int    g4_download_q8K_rows(const void *y, void *host_blocks, int k, int m);

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
 * main.c:1539-1556: dequantized weights times fp32 x; Q6_K, and Q4_K / Q5_K
 * (the reference's --f32-matmul path, main.c:1680-1683). */
int g4_mm_quant_rows(float *o, const float *x, const void *w, int n, int d, int type);
/* mm_bf16 (main.c:1529-1537), mm_f16 (1519-1527), mm_f32 (1494-1517):
 * row-major 16- or 32-bit weights times fp32 x; n a multiple of 8 (4 for
 * f32), at most 16384; w and x 16-byte aligned. */
int g4_mm_bf16(float *o, const float *x, const void *w, int n, int d);
int g4_mm_f16(float *o, const float *x, const void *w, int n, int d);
int g4_mm_f32(float *o, const float *x, const void *w, int n, int d);
/* mm(float *o, const float *x, const void *w, int n, int d, int type,
 * BlockQ8_K *q8, int q8_ready), main.c:1669-1694: Q4_K/Q5_K quantize x into
 * q8 unless q8_ready, then integer dots; Q6_K -> mm_quant_rows; BF16 / F16 /
 * F32 -> mm_bf16 / mm_f16 / mm_f32; other types -> G4_ERR_TYPE. */
int g4_mm(float *o, const float *x, const void *w, int n, int d, int type, void *q8, int q8_ready);
/* PLE gate (main.c:1988-1993): o[i] = gelu(W_i . q8) * mul[i], W Q4_K/Q5_K. */
int g4_mm_quant_dot_rows_gelu_mul(float *o, const void *w, int n, int d, int type, const void *q8, const float *mul);
/* Fused FFN up-projection: hb[i] = gelu(gate_i . x) * (up_i . x) for
 * i < d, both Q4_K/Q5_K against one Q8_K vector (main.c:1974-1980). */
int g4_mm_gate_up_gelu(float *hb, const void *gate, const void *up, int n, int d, int type, const void *q8);
/* Debug: per-block exact integer sums S_b, M_b (int32, d*nb each) of
 * Q4_K/Q5_K x Q8_K (main.c:500-523 summed over lanes). */
int g4_debug_block_sums(const void *w, int n, int d, int type, const void *q8, int32_t *S, int32_t *M);
/* logits_tied's GEMV + soft-cap (main.c:1788-1795): o = cap*tanh(W.x / cap) */
int g4_mm_quant_rows_softcap(float *o, const float *x, const void *w, int n, int d, int type, float cap);
/* tiling knob of the K-quant GEMVs (workgroups per CU targeted; default 4) */
int g4_set_gemv_occupancy(int wg_per_cu);
/* g4_residual_norm followed by g4_mm_quant_dot_rows (or, with mul,
 * g4_mm_quant_dot_rows_gelu_mul; or, with w2, g4_mm_gate_up_gelu with gate
 * w and up w2) on the Q8_K it produces, in one launch: the residual step of
 * main.c:1960-1962 / 1982-1984 / 1995-2003 reads the stream from x and
 * writes it to x_out (which must differ from x when y is given; with
 * y == NULL it is x copied, or nothing if x_out == x), the next norm
 * (main.c:1878, 1973) goes to xb2 (must differ from y) and
 * Q8_K(qsrc == 0 ? normed : x_out) to q8 (each optional), and o = W . Q8_K.
 * W is Q4_K/Q5_K with n in {2048, 2560, 4096}. */
int g4_mm_residual_q8(float *o, const void *w, const void *w2, int n, int d, int type, const float *mul,
                      const float *x, float *x_out, const float *y, const float *w_post, const float *oscale,
                      const float *w_next, float *xb2, void *q8, int qsrc, float eps);
/* g4_mm_residual_q8 with two independent GEMVs of the same type and n on
 * the one Q8_K (e.g. the Q and K projections of a layer, main.c:1883-1891):
 * o1 = W1 . Q8_K (d1 rows), o2 = W2 . Q8_K (d2 rows), one launch. */
int g4_mm_residual_q8_pair(float *o1, const void *w1, int d1, float *o2, const void *w2, int d2, int n, int type,
                           const float *x, float *x_out, const float *y, const float *w_post, const float *oscale,
                           const float *w_next, float *xb2, void *q8, int qsrc, float eps);
/* ... plus a third tensor of type Q6_K (w3, d3 rows) on the fp32 normed
 * vector (xb2), as mm routes Q6_K to mm_quant_rows (main.c:1687-1689): the
 * Q, K and V projections of a layer (main.c:1883-1892) in one launch.
 * Requires w_next (the vector is the normed one). */
int g4_mm_residual_q8_qkv(float *o1, const void *w1, int d1, float *o2, const void *w2, int d2, float *o3,
                          const void *w3, int d3, int type3, int n, int type, const float *x, float *x_out,
                          const float *y, const float *w_post, const float *oscale, const float *w_next, float *xb2,
                          void *q8, float eps);
/* The attention block's end and the output projection in one launch
 * (main.c:1909-1950 then main.c:1955): the G chunk partials that
 * g4_attn_decode_fused left in part (out and q8 NULL) are merged per head by
 * log-sum-exp exactly as its own merge does (same operations and order, so
 * the same vector), quantized to Q8_K and multiplied by W (Q4_K / Q5_K, d
 * rows of n = n_heads * hd) as g4_mm_quant_dot_rows: o[d].  q_out (n floats)
 * and q8 (g4_q8K_bytes(n)) optionally receive the merged vector and its
 * Q8_K.  n = n_heads * hd of 2048 or 4096 (head_dim 256 or 512),
 * G <= G4_MERGE_MAX_CHUNKS. */
#define G4_MERGE_MAX_CHUNKS 16
int g4_mm_attn_merge(float *o, const void *w, int n, int d, int type, const float *part, int G, int n_heads, int hd,
                     float *q_out, void *q8);

/* The PLE gate and projection of a decode layer in one launch
 * (main.c:1982-1994): the residual step of g4_mm_residual_q8 with qsrc 1
 * (post_ffw_norm of y_in into x_out = x + norm(y_in) * w_post, Q8_K of
 * x_out), g = gelu(w_gate . q8) * mul (pd rows, the PLE gate), then
 * y = mm(w_proj, g) (d_proj rows of one block: g quantized to Q8_K as mm()
 * does) -- the same bits as g4_mm_residual_q8(g, w_gate, NULL, n, pd, ...,
 * mul, ..., qsrc 1) followed by g4_mm(y, g, w_proj, pd, d_proj, ...).  The
 * gate values cross workgroups as (value, *seq) pairs in `pairs`
 * (g4_ple_pairs_bytes(pd) bytes of device memory, zeroed before the first
 * call): *seq must differ between calls that share `pairs` and must not be
 * 0 (g4_emb_lookup_rope_ple advances such a word once per decode step; give
 * each layer its own pairs).  The word after the pairs becomes nonzero if a
 * call's projection could not read the gate values (never expected; its y
 * is then invalid).  n = 2560, pd = 256 only; gate and projection Q4_K or
 * Q5_K.  No counterpart in the reference, which runs the two as separate
 * mm() calls. */
size_t g4_ple_pairs_bytes(int pd);
int g4_mm_ple_gate_proj(float *y, const void *w_proj, int type_proj, int d_proj, const void *w_gate, int type_gate,
                        int n, int pd, const float *mul, const float *x, float *x_out, const float *y_in,
                        const float *w_post, float eps, void *pairs, const uint32_t *seq);

/* ---------------------------------------------------------------------------
 * Batched prefill GEMM.  The reference has none: generate() runs forward()
 * once per prompt token (main.c:2366-2384), so for m tokens it performs m
 * times quantize_row_q8_K(x_t) (main.c:282) + mm_quant_dot_rows (main.c:1558).
 * These entry points do the same m products in one launch on the matrix
 * cores.  Q4_K / Q5_K: every block's integer sums S_b and M_b are the
 * per-token dot's exactly (g4_debug_batch_block_sums), the fp32 fold of the
 * blocks runs in another order, so outputs are within 1e-5 of sum |terms| of
 * the per-token dot.  Q6_K / BF16: exact products, sums in another order.
 * ------------------------------------------------------------------------- */
/* Bytes between consecutive Q8_K rows of a batch: g4_q8K_bytes(k) rounded
 * up to 64 (0 if k is not a positive multiple of 256). */
size_t g4_q8K_row_stride(int k);
/* m rows of k floats (row stride k) -> m Q8_K rows at g4_q8K_row_stride(k)
 * bytes apart: quantize_row_q8_K (main.c:282) per row. */
int g4_quantize_rows_q8_K(const float *x, void *y, int k, int m);
/* o[t*d + r] = mm_quant_dot_rows row r on Q8_K row t (main.c:1558-1566,
 * vec_dot_q4_K_q8_K / vec_dot_q5_K_q8_K main.c:476-593), t < m, r < d:
 * the same integer block sums and scales, the code sums on the int8 matrix
 * cores (every S_b, M_b exact in int32), the fp32 fold in another order
 * (within 1e-5 of sum |terms| of the per-token dot).  Q4_K / Q5_K only
 * (others: G4_ERR_TYPE); o, w, q8 16-byte aligned. */
int g4_mm_batch_q8(float *o, const void *w, const void *q8, int n, int d, int m, int type);
/* g4_mm_batch_q8 for nseg (1..4) matrices of one type over the same Q8_K
 * rows in one launch (gate and up, Q and K): o[k][t*d[k] + r] for matrix
 * w[k] of d[k] rows.  Each output equals g4_mm_batch_q8's for that matrix. */
int g4_mm_batch_q8_multi(float *const *o, const void *const *w, const int *d, int nseg, const void *q8, int n, int m,
                         int type);
/* g4_mm_batch_q8 split by K block, for small d (the PLE gate, main.c:1988,
 * 256 rows: one workgroup per 128 rows x 32 tokens x block instead of ten
 * blocks in series): u[(b*m + t)*d + r] = the block-b term of row r for token
 * t before the token's Q8_K d, i.e. fma(d_w, S_b, -dmin_w * M_b) of
 * vec_dot_q4_K_q8_K / q5_K (main.c:476-593) on n/256 blocks.  Folding them
 * in block order, g = fma(d_tb, u_b, g) from 0 (g4_fold_gelu_mul_q8), gives
 * g4_mm_batch_q8's output bit for bit.  u holds (n/256) * m * d floats. */
int g4_mm_batch_q8_blocks(float *u, const void *w, const void *q8, int n, int d, int m, int type);
/* fp16 weight image of a Q4_K / Q5_K matrix for the batched GEMM: each
 * weight's sc * q (sub-block scale times code, get_scale_min_k4 and the
 * dequantize loops of main.c:170-211) in the matrix cores' operand order, d,
 * dmin and the mins per row and block.  Built once (at model load); the
 * decode-step GEMVs keep reading the quantized tensor.  Bytes of the image
 * of d rows x n (0 if n is not a positive multiple of 256). */
size_t g4_kq_image_bytes(int n, int d);
/* write the image of w (Q4_K / Q5_K, d x n, device layout) into img
 * (g4_kq_image_bytes(n, d) bytes, 16-byte aligned) */
int g4_kq_image(void *img, const void *w, int n, int d, int type);
/* g4_mm_batch_q8 / g4_mm_batch_q8_multi on images instead of the quantized
 * tensors (type: the type the image was built from): the same exact integer
 * block sums and the same fold, so g4_mm_batch_q8's outputs bit for bit
 * (within 1e-5 of sum |terms| of mm_quant_dot_rows, main.c:1558-1566) */
int g4_mm_batch_img(float *o, const void *img, const void *q8, int n, int d, int m, int type);
int g4_mm_batch_img_multi(float *const *o, const void *const *img, const int *d, int nseg, const void *q8, int n,
                          int m, int type);
/* g4_mm_batch_img with the tile given: 32*nt tokens x 32*nwv rows per
 * workgroup, (nt, nwv) in (1, 2), (1, 4), (1, 8), (2, 4), (2, 8); shape sweeps */
int g4_mm_batch_img_tile(float *o, const void *img, const void *q8, int n, int d, int m, int type, int nt, int nwv);
/* Debug: the batched GEMM's own per-block integer sums, for m Q8_K rows
 * (g4_q8K_row_stride(n) apart): S[(t*d + r)*nb + b] = S_b and M[...] = M_b
 * of row r, token t, block b (nb = n/256), as the batched kernel forms them
 * on the matrix cores (image 0: from the quantized tensor w; image 1: from
 * its fp16 image) -- the sums of vec_dot_q4_K_q8_K / q5_K (main.c:500-523,
 * 556-590) that g4_debug_block_sums gives per token. */
int g4_debug_batch_block_sums(const void *w, int image, int n, int d, int m, int type, const void *q8, int32_t *S,
                              int32_t *M);
/* the fold of g4_mm_batch_q8_blocks' terms over the Q8_K rows q8 (n wide) ->
 * out[t*d + r]; with ple, out = gelu(fold) * ple[t*pstride + r] instead
 * (main.c:1989-1993, as g4_gelu_mul_rows); with q8o, also the Q8_K rows of
 * out (d a multiple of 256, g4_q8K_row_stride(d) apart, as
 * g4_quantize_rows_q8_K).  d <= 1024, n <= 16384. */
int g4_fold_gelu_mul_q8(const float *u, const void *q8, int n, const float *ple, int pstride, float *out, void *q8o,
                        int d, int m);
/* m tokens through mm(o_t, x_t, w, n, d, type, q8, 0) (main.c:1669): Q4_K /
 * Q5_K quantize all rows into q8 (m * g4_q8K_row_stride(n) bytes) and take
 * g4_mm_batch_q8; Q6_K and BF16 with n a multiple of 256 and 16-byte aligned
 * x, w: one fp32 matrix-core GEMM on the fp32 activations (the reference's
 * dequantized fp32 weights, fp32 sums in another order; q8 unused);
 * otherwise the per-token GEMV m times. */
int g4_mm_batch(float *o, const float *x, const void *w, int n, int d, int m, int type, void *q8);
/* Bytes of m split activation rows of n floats (n a multiple of 256): m * 4n
 * for the rows plus 4m for the per-row scale factors; 0 for bad sizes. */
size_t g4_split_rows_bytes(int n, int m);
/* m fp32 rows (row stride n) -> split rows for g4_mm_batch_split: each row
 * scaled by the power of two 2^-s that brings its largest |x| into
 * [2^14, 2^15), written as two fp16 terms hi + lo (x 2^-s - hi - lo within
 * 2^-22 of |x 2^-s|), permuted into the matrix-core K order; the m factors
 * 2^s follow the rows.  x, xs 16-byte aligned. */
int g4_split_rows_f16(const float *x, void *xs, int n, int m);
/* o[t*d + r] = mm_quant_rows row r of split row t (main.c:1539-1556) for a
 * planar Q6_K w: the exact products sc * (q - 32) * (hi + lo) on the fp16
 * matrix cores (the integer weight split exactly into its fp16 rounding Wh
 * and the rest Wl in {-1, 0, 1}: Wh hi + Wh lo + Wl hi), the block's d and
 * the row's 2^s in fp32; within 1e-5 of sum |w x| of the reference's fp32
 * dot.  Q6_K only (others: G4_ERR_TYPE). */
int g4_mm_batch_split(float *o, const void *w, const void *xs, int n, int d, int m, int type);
/* g4_gelu_mul_rows (o = gelu(g) * u, rows of n, u rows ustride floats apart)
 * followed by g4_split_rows_f16 of o in one launch, without o: the split rows
 * of the FFN's GELU gate (main.c:1976-1980) for the Q6_K down GEMM.  n =
 * 2048 * k for k in {1, 2, 4, 5, 6, 8}; xs as for g4_split_rows_f16, bit for
 * bit what the two launches produce. */
int g4_gelu_mul_split_rows(const float *g, const float *u, int ustride, void *xs, int n, int m);

/* ---------------------------------------------------------------------------
 * Prompt-chunk forms of the step glue (the reference runs forward() once per
 * prompt token, main.c:2366-2384; these run the same per-token operations
 * on m tokens of a chunk in one launch each).  Rows of a chunk are
 * contiguous; Q8_K rows are g4_q8K_row_stride(n) bytes apart.
 * ------------------------------------------------------------------------- */
/* emb_lookup + x * sqrt(dim) (main.c:1696-1723, 1849-1854) of tokens dtok[0..m) */
int g4_emb_lookup_rows(float *o, const void *w, int type, int rows, const int *dtok, int m, int dim, float scale);
/* build_ple after its projection (main.c:1751-1777) for tokens dtok[0..m):
 * ple, ctx rows of L*pd floats */
int g4_ple_finish_rows(float *ple, const float *ctx, const void *ple_tok, int type, int rows, const float *proj_norm,
                       const int *dtok, int m, int pd, int L, float sc_tok, float sc_ctx, float mix, float eps);
/* o[z][i] = gelu(g[z][i]) * u[z*ustride + i]: gelu(gate)*up (main.c:1976-1980)
 * and the PLE gate (main.c:1989-1993) */
int g4_gelu_mul_rows(float *o, const float *g, const float *u, int d, int m, int ustride);
/* g4_residual_norm on m rows of x (in place), each row's bits those of the
 * decode step: narrow = 1 matches the residual prologue of g4_mm_residual_q8
 * (_pair, _qkv, and the single-tensor form; n = 2048, 2560, 4096, all
 * pointers 16-byte aligned), narrow = 0 g4_residual_norm.  For 16-byte
 * aligned rows with n a multiple of 256 up to 4096 the two layouts are the
 * same (one float4 per thread). */
int g4_residual_norm_rows(float *x, const float *y, const float *w_post, const float *oscale, const float *w_next,
                          float *xb2, void *q8, int qsrc, int n, float eps, int m, int narrow);
/* RoPE (cos, sin) tables of positions pos0..pos0+m-1 (main.c:1725-1742), n_rot/2 pairs each */
int g4_rope_table_rows(float *tab, int pos0, int m, int n_rot, float freq_base, float freq_scale,
                       const float *freq_factors);
/* per-head norms + RoPE of m tokens (main.c:1886-1900): q rows in place, k/v
 * rows (nullable) into rows of kout/vout (stride kv_stride) */
int g4_qkv_post_rows(float *q, const float *q_norm, const float *k, const float *v, const float *k_norm, float *kout,
                     float *vout, int kv_stride, const float *tab_rows, int m, int n_heads, int n_kv, int hd, int n_rot,
                     float eps);
/* the KV append (main.c:1901-1904) of positions pos0..pos0+m-1 from rows of kin/vin */
int g4_kv_store_rows(float *kc, float *vc, const float *kin, const float *vin, int kv_stride, int ring, int pos0, int m,
                     int kvd);
/* the attention block (main.c:1909-1950) for m query rows at positions
 * p0..p0+m-1: the chunk's K/V in rows of kchunk/vchunk, earlier positions in
 * the cache (ring: window <= ring); part: m * g4_attn_part_bytes(n_heads, hd, G) */
int g4_attn_decode_rows(const float *q, const float *kc, const float *vc, const float *kchunk, const float *vchunk,
                        int kv_stride, int ring, int p0, int m, int window, int n_heads, int n_kv, int hd,
                        float attn_scale, int G, float *part, float *out, void *q8);

/* ---------------------------------------------------------------------------
 * Norms, RoPE, attention (main.c:1451-1488, 1725-1745, 1886-1950)
 * ------------------------------------------------------------------------- */
/* rmsnorm(float *o, const float *x, const float *w, int n, float eps), main.c:1451 */
int g4_rmsnorm(float *o, const float *x, const float *w, int n, float eps);
/* rmsnorm_head_inplace(float *v, const float *w, int n_heads, int hd, float eps), main.c:1458 */
int g4_rmsnorm_head_inplace(float *v, const float *w, int n_heads, int hd, float eps);
/* rmsnorm_head_noweight_inplace(float *v, int n_heads, int hd, float eps), main.c:1468 */
int g4_rmsnorm_head_noweight_inplace(float *v, int n_heads, int hd, float eps);
/* apply_rope_neox(float *vec, int n_heads, int head_dim, int n_rot, int pos,
 * float freq_base, float freq_scale, const float *freq_factors), main.c:1725 */
int g4_apply_rope_neox(float *vec, int n_heads, int head_dim, int n_rot, int pos, float freq_base, float freq_scale,
                       const float *freq_factors);
/* K/V append of main.c:1895-1904: k <- RoPE(rmsnorm_head(k, k_norm)), v <-
 * rmsnorm_head_noweight(v), stored at slot (ring ? pos % ring : pos) of
 * kc/vc (row stride kv_stride floats).  k and v are left unchanged. */
int g4_kv_append_rope(float *k, float *v, const float *k_norm, float *kc, float *vc, int kv_stride, int ring, int pos,
                      int n_kv, int hd, int n_rot, float freq_base, float freq_scale, const float *freq_factors,
                      float eps);
/* The attention block of main.c:1909-1950 (inline in forward(), no function
 * of its own there): per q head h, s_t = attn_scale * K[t].q_h over
 * t = t_start .. t_start+nwin-1 of kv head h/(n_heads/n_kv), softmax, o_h =
 * sum_t p_t V[t].  kc/vc: position 0 of a flat cache, row stride kv_stride
 * floats (main.c:1798-1809 uses 1024).  hd in {256, 512}. */
int g4_attn_decode(const float *q, const float *kc, const float *vc, int kv_stride, int t_start, int nwin, int n_heads,
                   int n_kv, int hd, float attn_scale, float *out);
/* Same block over a ring cache of `ring` slots (slot = t % ring) with the
 * sliding window of main.c:1910-1915 (window 0 = full attention). */
int g4_attn_decode_ring(const float *q, const float *kc, const float *vc, int kv_stride, int ring, int pos, int window,
                        int n_heads, int n_kv, int hd, float attn_scale, float *out);
/* g4_attn_decode that allocates nothing.  No counterpart in the reference:
 * for callers that cannot call hipMalloc (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  Same arguments,
 * kernels and results (bit for bit) as g4_attn_decode, but the chunk
 * partials live in a per-GPU scratch array of G4_ATTN_NOALLOC_SCRATCH bytes
 * that g4_init sets up, instead of the library's growing workspace.
 * Limit: n_heads * G * (hd + 2) * 4 bytes of partials, G being the chunk
 * count (about nwin / 32, 1..128 up to 131072 positions, more beyond):
 * G4_ERR_ARG above it; G4_ERR_STATE if g4_init was not called for the
 * current device.  Every call on a GPU shares its scratch, so calls that
 * overlap in time on one GPU race. */
#define G4_ATTN_NOALLOC_SCRATCH (8u << 20)
int g4_attn_decode_noalloc(const float *q, const float *kc, const float *vc, int kv_stride, int t_start, int nwin,
                           int n_heads, int n_kv, int hd, float attn_scale, float *out);
/* softmax(float *x, int n), main.c:1478 */
int g4_softmax(float *x, int n);

/* ---------------------------------------------------------------------------
 * Step glue (main.c:1696-1778, 1988-1993, 2045-2049)
 * ------------------------------------------------------------------------- */
/* emb_lookup(float *o, const void *w, int type, int id, int dim), main.c:1696;
 * rows = the table's row count (checked; the reference trusts id). */
int g4_emb_lookup(float *o, const void *w, int type, int rows, int id, int dim);
/* first index of the maximum of v[0..n) (sample_token, temp <= 0,
 * main.c:2045-2049) -> *out (device int).  part: g4_argmax_part_bytes(n)
 * device bytes.  dtok/dpos (device, nullable): also store the token as the
 * next step's input and advance the position by one. */
size_t g4_argmax_part_bytes(int n);
int    g4_argmax(const float *v, int n, int *out, void *part, int *dtok, int *dpos);
/* mm_argmax_row (main.c:1570-1667, logits_tied's lm_mode 2 at main.c:1784-1786,
 * generate's fast_argmax main.c:2348) and the greedy pick after logits_tied
 * (main.c:1788-1795, 2045-2049): the first index of the largest of
 * v = W . x (cap <= 0) or cap * tanh(W . x / cap) (cap > 0) -> *out / *dtok
 * (device ints, each optional), *dpos advanced if given.  v is written to
 * logits (d floats, required).  Q6_K: the LM-head GEMV reduces its rows to
 * per-workgroup argmax keys in the same launch (the reference's fused
 * lm_mode 2); other types: g4_mm (q8: the Q8_K workspace for Q4_K / Q5_K),
 * soft-cap, g4_argmax.  part: g4_mm_argmax_part_bytes(d). */
size_t g4_mm_argmax_part_bytes(int d);
int    g4_mm_argmax_row(const float *x, const void *w, int n, int d, int type, void *q8, float cap, float *logits,
                        void *part, int *out, int *dtok, int *dpos);

/* ---------------------------------------------------------------------------
 * Engine step kernels: fusions of consecutive statements of forward()
 * (main.c:1838-2029) whose position/token come from device memory, so that a
 * captured graph of one decode step is valid at every position.
 * ------------------------------------------------------------------------- */
/* x += rmsnorm(y, w_post) (if y); x *= oscale[0] (if oscale); xb2 =
 * rmsnorm(x, w_next) (if w_next); q8 = Q8_K(qsrc ? x : xb2) (if q8).
 * main.c:1960-1962, 1982-1984, 1995-2003, 1878-1884, 1973-1975, 2021. */
int g4_residual_norm(float *x, const float *y, const float *w_post, const float *oscale, const float *w_next,
                     float *xb2, void *q8, int qsrc, int n, float eps);
/* main.c:1886-1904: q heads q_norm + RoPE in place; if k: k heads k_norm +
 * RoPE and v heads unweighted norm, stored at slot (ring ? pos%ring : pos);
 * pos = *dpos if dpos else pos; rope_tab (nullable): g4_rope_table output for
 * this position and layer type. */
int g4_qkv_post(float *q, const float *q_norm, const float *k, const float *v, const float *k_norm, float *kc,
                float *vc, int kv_stride, int ring, const int *dpos, int pos, int n_heads, int n_kv, int hd, int n_rot,
                float freq_base, float freq_scale, const float *ff, float eps, const float *rope_tab);
/* (cos, sin) of the n_rot/2 RoPE pair angles at pos = *dpos (or pos), the
 * angle chain of main.c:1727-1742; rope_tab argument of g4_qkv_post. */
int g4_rope_table(float *tab, const int *dpos, int pos, int n_rot, float freq_base, float freq_scale,
                  const float *freq_factors);
/* attention block with pos = *dpos, t_start = max(0, pos+1-window) (window 0:
 * 0), G time chunks (fixed, 1..512; <= 1024 positions each), workspace of
 * g4_attn_part_bytes(n_heads, hd, G) bytes, optional Q8_K of the output. */
size_t g4_attn_part_bytes(int n_heads, int hd, int G);
int    g4_attn_decode_dev(const float *q, const float *kc, const float *vc, int kv_stride, int ring, const int *dpos,
                          int window, int n_heads, int n_kv, int hd, float attn_scale, int G, float *part, float *out,
                          void *q8);
/* qkv_post + attention in one launch pair (main.c:1886-1950): per-head
 * rmsnorm of the raw Q projection q_raw with q_norm and RoPE from rope_tab
 * (g4_rope_table at this position; q_raw itself is not modified); if k_raw
 * is non-null (a layer that stores KV), k_raw/v_raw are normalised (K with
 * k_norm and rotated, V without weight) and stored at slot pos (pos % ring
 * when ring > 0) of kstore/vstore, and the attention over kc/vc (the cache
 * read: this layer's own, or the donor's on shared-KV layers) uses them for
 * position pos.  n_rot/2 must divide 256.  Otherwise as g4_attn_decode_dev;
 * with out and q8 NULL only the chunk partials are written to part (G chunks
 * per head, g4_attn_part_bytes), for g4_mm_attn_merge to merge. */
int    g4_attn_decode_fused(const float *q_raw, const float *q_norm, const float *k_raw, const float *v_raw,
                            const float *k_norm, float *kstore, float *vstore, const float *kc, const float *vc,
                            int kv_stride, int ring, const int *dpos, int window, int n_heads, int n_kv, int hd,
                            int n_rot, const float *rope_tab, float eps, float attn_scale, int G, float *part,
                            float *out, void *q8);
/* x = emb_lookup(w, *dtok) * scale (main.c:1849-1854) */
int g4_emb_lookup_dev(float *o, const void *w, int type, int rows, const int *dtok, int dim, float scale);
/* The decode step's inputs in one launch: g4_emb_lookup_dev(o, ..., scale)
 * and g4_rope_table(tab_a, dpos, 0, n_rot_a, base_a, freq_scale, ff_a) and
 * g4_rope_table(tab_b, ...) at the position *dpos -- the same values as the
 * three calls (main.c:1849-1854, 1725-1742). */
int g4_emb_lookup_rope(float *o, const void *w, int type, int rows, const int *dtok, int dim, float scale,
                       const int *dpos, float *tab_a, int n_rot_a, float base_a, const float *ff_a, float *tab_b,
                       int n_rot_b, float base_b, const float *ff_b, float freq_scale);
/* ... and the PLE context projection of build_ple on the same row
 * (main.c:1749-1750: ctx = mm_bf16(w_ctx, o), w_ctx bf16 [d_ctx x dim]) in
 * the same launch: the same values as g4_emb_lookup_rope followed by
 * g4_mm_bf16(ctx, o, w_ctx, dim, d_ctx).  dim a multiple of 8, <= 4096.
 * seq (nullable): a device word the launch increments by one (the step's
 * sequence number for g4_mm_ple_gate_proj). */
int g4_emb_lookup_rope_ple(float *o, const void *w, int type, int rows, const int *dtok, int dim, float scale,
                           const int *dpos, float *tab_a, int n_rot_a, float base_a, const float *ff_a, float *tab_b,
                           int n_rot_b, float base_b, const float *ff_b, float freq_scale, float *ctx,
                           const void *w_ctx, int d_ctx, uint32_t *seq);
/* build_ple after its projection (main.c:1751-1777): ple[l*pd+i] =
 * (emb(ple_tok, tok)[l*pd+i]*sc_tok + rmsnorm(ctx[l*pd..]*sc_ctx, norm)[i]) * mix;
 * tok = *dtok if dtok else tok. */
int g4_ple_finish(float *ple, const float *ctx, const void *ple_tok, int type, int rows, const float *proj_norm,
                  const int *dtok, int tok, int pd, int L, float sc_tok, float sc_ctx, float mix, float eps);
/* g = gelu(g) * ple, then q8 = Q8_K(g) if q8 (main.c:1989-1993) */
int g4_gelu_mul_quant(float *g, const float *ple, int n, void *q8);
/* Sampler of generate (main.c:2035-2126) on the device: the repetition
 * penalty of the last penalty_last_n of the *hist_n tokens in hist (all when
 * penalty_last_n <= 0; skipped when penalty <= 1; written back to logits as
 * apply_repetition_penalty does), then sample_token: temp <= 0 the first
 * index of the maximum, else top-k (1..64, <= n) by (value, first index),
 * softmax((v - max) / temp), a plain draw or, for 0 < topp < 1, a top-p draw
 * from the xorshift64* state *rng (advanced as rng_f32 does).  The token
 * goes to *out, *dtok (nullable) and is appended to hist when *hist_n <
 * hist_cap; *dpos (nullable) advances by one.  n <= 262144, logits 16-byte
 * aligned; part: g4_sample_part_bytes(n) device bytes.  All state is on the
 * device, so the call can be captured in a graph.  Bit-exact except expf,
 * which may differ from glibc's by an ulp (a draw within that distance of
 * a cdf step can pick the neighbour). */
size_t g4_sample_part_bytes(int n);
int g4_sample(float *logits, int n, float temp, float topp, int topk, float penalty, int penalty_last_n, int *hist,
              int *hist_n, int hist_cap, unsigned long long *rng, void *part, int *out, int *dtok, int *dpos);
/* hidden_stats (main.c:1813-1826), the --dump-hidden-at fingerprint of a
 * vector: out[0] = sum, out[1] = l2 norm (both accumulated in double),
 * out[2] = max |v| (device pointers; one launch) */
int g4_hidden_stats(const float *v, int n, float *out);
/* logits_tied's soft-cap (main.c:1789-1795): v[i] = cap * tanhf(v[i] * (1/cap)) */
int g4_softcap(float *v, int n, float cap);
/* dst[0] = a, dst[1] = b on the library stream (the step's token and position) */
int g4_store_i32x2(int *dst, int a, int b);

/* ---------------------------------------------------------------------------
 * Streams, graphs, copies
 * ------------------------------------------------------------------------- */
/* synchronous fill (set-up only, not for captured graphs) */
int g4_memset(void *p, int value, size_t bytes);
int g4_memcpy_h2d_async(void *dst, const void *src, size_t bytes);
int g4_memcpy_d2h_async(void *dst, const void *src, size_t bytes);
int g4_memcpy_d2d_async(void *dst, const void *src, size_t bytes);
int g4_host_alloc(void **p, size_t bytes);   /* pinned host memory */
int g4_host_free(void *p);
int g4_stream_create(void **stream);
int g4_stream_destroy(void *stream);
/* capture the library stream's work into a graph (the stream must be a
 * created one, not the null stream) */
int g4_graph_begin(void);
int g4_graph_end(void **graph_exec);
int g4_graph_launch(void *graph_exec);
int g4_graph_destroy(void *graph_exec);

/* ---------------------------------------------------------------------------
 * Measurement probes (no counterpart in the reference; they compute nothing
 * of the model): the floors the decode step is sized against, timed by
 * bench.py --workload floors.
 * ------------------------------------------------------------------------- */
/* an empty kernel of `workgroups` 64-thread workgroups: a dependent launch's cost */
int g4_probe_empty(int workgroups);
/* a streaming read of `bytes` (16-byte aligned, a multiple of 16) with 1 KB
 * per wave instruction over `workgroups` 256-thread workgroups; sink gets one
 * float per workgroup */
int g4_probe_read(const void *p, size_t bytes, float *sink, int workgroups);
/* every 256-thread workgroup stores 16 values (vals: 16 per workgroup,
 * workgroups <= 640); mode 1: each then releases them device-wide (fence)
 * and counts itself in on *count (zero before the first launch; the last
 * workgroup resets it), and the last one acquires, loads every value at once
 * and adds them into *out; mode 2: the same with the values stored and
 * loaded as device-scope relaxed atomics and no fences; mode 0: the stores
 * only. */
int g4_probe_handoff(float *vals, unsigned int *count, float *out, int workgroups, int mode);

#ifdef __cplusplus
}
#endif
#endif /* G4HIP_H */
