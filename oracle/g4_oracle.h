/*
 * oracle/g4_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the decode-step hot path of thamada/Gemma4.c
 * (gemma4-4b/cpu-blas/main.c).  It is the checker for the HIP library:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and never as the thing measured or shipped.  Every function
 * names the reference lines it follows.
 *
 * fp32 evaluation order is part of the contract: the library is built
 * with gcc -std=c11 (which implies -ffp-contract=off), so a*b+c is two
 * roundings unless fmaf() is written, exactly as the reference's own build
 * (gemma4-4b/cpu-blas/Makefile:7-8) evaluates it.
 *
 * Pinning status (what checks each function; tests/ hold the checks):
 *   - formats, fp16/bf16 decode, dequant, Q8_K quantize, Q4_K/Q5_K dots
 *     (both fp32 orders), mm_quant_rows, mm_bf16/f16, norms, softmax,
 *     gelu, RoPE, emb_lookup, greedy/top-k sampler: bit-exact against the
 *     reference's own functions compiled from main.c into oracle/_ref, plus
 *     closed-form / brute-force checks (exact integer re-derivation of the
 *     block sums, double-precision dot products, RoPE toy example).
 *   - attention block (main.c:1909-1950): its sgemv calls go to OpenBLAS,
 *     which is absent, so the reference cannot be run for it; pinned by a
 *     double-precision brute-force softmax-attention and by the pos=0 /
 *     single-token closed forms.
 *   - vec_dot_q6_K_q8_K: has no counterpart in the reference; pinned by an
 *     exact integer brute force over the dequant formula.
 *   - model level (tests/test_oracle_model.py): or_model_open against the
 *     reference's own parse_gguf/load_weights (configuration, data offset
 *     at two alignments, vocabulary, KV routing); build_ple, every layer
 *     step and the final norm + logits_tied bit for bit against a
 *     composition of the reference's compiled functions over the
 *     reference loader's weight pointers, in forward()'s statement order
 *     (main.c:1838-2029), the attention block in float64; invariants
 *     (zero O/down/proj weights leave out_scale * input exactly; shared
 *     layers read donor 22 or 23 and nothing else); or_hidden_stats bit
 *     for bit against the reference's hidden_stats; or_mm_f32 by float64
 *     brute force.
 */
#ifndef G4_ORACLE_H
#define G4_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_QK_K 256
#define OR_MAX_KV_DIM 1024   /* main.c:75 */
#define OR_MAX_Q_DIM 4096    /* main.c:74 */
#define OR_N_LAYER_KV 24     /* main.c:77 */

/* ggml dtype ids, main.c:85-92 */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_BF16 = 30 };

/* Block layouts, main.c:94-122.  Byte-identical to the reference. */
#pragma pack(push, 1)
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } or_q4K;              /* 144 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } or_q5K; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } or_q6K;      /* 210 B */
#pragma pack(pop)
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } or_q8K;                          /* 292 B */

/* ---- scalar helpers ---------------------------------------------------- */
float    or_f16_to_f32(uint16_t h);                    /* main.c:128-149 */
float    or_bf16_to_f32(uint16_t h);                   /* main.c:151-156 */
uint16_t or_f32_to_f16(float f);                       /* IEEE RNE; generators only */
void     or_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m); /* main.c:162-170 */
void     or_unpack_scales_words(const uint8_t s[12], uint8_t sc[8], uint8_t mn[8]); /* main.c:490-495 */
size_t   or_block_bytes(int type);                     /* main.c:758-765 */

/* ---- dequantizers, main.c:172-237 ------------------------------------- */
void or_dequant_q4K(const or_q4K *x, float *y, int64_t nb);
void or_dequant_q5K(const or_q5K *x, float *y, int64_t nb);
void or_dequant_q6K(const or_q6K *x, float *y, int64_t nb);
void or_dequant_block(const void *blk, int type, float *dst); /* main.c:767-776 */

/* ---- Q8_K activation quantization, main.c:247-340 --------------------- */
void or_quantize_q8K(const float *x, or_q8K *y, int k);

/* ---- per-block exact integer sums ------------------------------------- */
/* Q4_K/Q5_K in the reference AVX2 lane partition (main.c:500-523):
 * sumi[l] covers qs bytes 4l..4l+3 of every 32-byte chunk, prod[k] pairs
 * sub-blocks 2k, 2k+1 of the min term. */
void or_q4K_lane_sums(const or_q4K *x, const or_q8K *y, int32_t sumi[8], int32_t prod[4]);
void or_q5K_lane_sums(const or_q5K *x, const or_q8K *y, int32_t sumi[8], int32_t prod[4]);
/* S_b = sum_j sc_j * sum_{i in j} q_i*q8_i, M_b = sum_k bsums_k * m_{k/2} */
void or_q4K_block_SM(const or_q4K *x, const or_q8K *y, int32_t *S, int32_t *M);
void or_q5K_block_SM(const or_q5K *x, const or_q8K *y, int32_t *S, int32_t *M);
/* Q6_K x Q8_K (no reference counterpart): S_b = sum_s sc_s sum_{i in s} (q6_i-32) q8_i */
int32_t or_q6K_block_S(const or_q6K *x, const or_q8K *y);

/* ---- dot products ------------------------------------------------------ */
float or_vec_dot_q4K_q8K(int n, const or_q4K *x, const or_q8K *y);          /* AVX2 order, main.c:476-529 */
float or_vec_dot_q5K_q8K(int n, const or_q5K *x, const or_q8K *y);          /* AVX2 order, main.c:531-593 */
float or_vec_dot_q4K_q8K_generic(int n, const or_q4K *x, const or_q8K *y);  /* main.c:347-407 */
float or_vec_dot_q5K_q8K_generic(int n, const or_q5K *x, const or_q8K *y);  /* main.c:409-473 */
float or_vec_dot_q6K_q8K(int n, const or_q6K *x, const or_q8K *y);          /* no reference counterpart */
float or_vec_dot_row_q8K(int n, const void *row, int type, const or_q8K *q8); /* main.c:603-613 */

/* ---- GEMV (o[d] = W[d x n] x[n]), main.c:1494-1566, 1669-1694 --------- */
void or_mm_quant_rows(float *o, const float *x, const void *w, int n, int d, int type);
void or_mm_quant_dot_rows(float *o, const void *w, int n, int d, int type, const or_q8K *q8);
void or_mm_q6K_q8K_rows(float *o, const void *w, int n, int d, const or_q8K *q8);
void or_mm_bf16(float *o, const float *x, const uint16_t *w, int n, int d);
void or_mm_f16(float *o, const float *x, const uint16_t *w, int n, int d);
void or_mm_f32(float *o, const float *x, const float *w, int n, int d);     /* plain-loop sgemv */
/* returns 0, or -1 on an unsupported type / n % 256 (the reference exits) */
int  or_mm(float *o, const float *x, const void *w, int n, int d, int type, or_q8K *q8, int q8_ready);

/* ---- step glue, main.c:1451-1492, 1696-1745 --------------------------- */
void  or_rmsnorm(float *o, const float *x, const float *w, int n, float eps);
void  or_rmsnorm_head_inplace(float *v, const float *w, int n_heads, int hd, float eps);
void  or_rmsnorm_head_noweight_inplace(float *v, int n_heads, int hd, float eps);
void  or_softmax(float *x, int n);
float or_gelu(float x);
void  or_apply_rope_neox(float *vec, int n_heads, int head_dim, int n_rot, int pos,
                         float freq_base, float freq_scale, const float *freq_factors);
int   or_emb_lookup(float *o, const void *w, int type, int id, int dim);

/* ---- attention block, main.c:1909-1950 ---------------------------------
 * kc/vc point at position 0 of the source layer's cache; row stride is
 * kv_stride floats (1024 in the reference layout).  att is scratch of
 * n_heads * (t_start + nwin) floats. */
void or_attn_decode(const float *q, const float *kc, const float *vc, int kv_stride,
                    int t_start, int nwin, int n_heads, int n_kv, int hd,
                    float attn_scale, float *att, float *out);

/* ---- sampler, main.c:2035-2126 ---------------------------------------- */
float or_rng_f32(uint64_t *state);
void  or_set_f32_matmul(int on);
int   or_sample_token(const float *logits, int n, float temp, float topp, int topk, uint64_t *rng);
void  or_apply_repetition_penalty(float *logits, const int *tokens, int n_tokens, float penalty, int penalty_last_n);
int   or_argmax_first(const float *v, int n);

/* ---- fingerprints, main.c:1814-1827 ----------------------------------- */
void or_hidden_stats(const float *v, int n, float *sum, float *l2, float *amax);

/* ---- model: GGUF image -> forward(), main.c:623-966, 1318-1445, 1747-2029 */
typedef struct or_model or_model;
/* Parses a GGUF image held in memory (borrowed, must outlive the model).
 * Returns NULL and writes a message to err (if non-NULL) on failure. */
or_model *or_model_open(const uint8_t *data, size_t size, int max_seq, char *err, size_t errlen);
void      or_model_close(or_model *m);
/* config query: dim, hidden, n_layers, n_heads, n_kv, vocab, max_seq, ple_dim, window */
void      or_model_config(const or_model *m, int out[9]);
int       or_forward(or_model *m, int token, int pos, int lm_mode);   /* main.c:1838-2029 */
/* forward() with layer inputs injected: x_in is (n_layers+1) x dim (row l =
 * input of layer l, row n_layers = input of the final norm); x_out gets each
 * layer's output (n_layers x dim).  Checks every layer of a device run in
 * isolation. */
int       or_forward_inject(or_model *m, int token, int pos, int lm_mode, const float *x_in, float *x_out);
/* or_forward_inject with every Q8_K activation taken from q8_in (same
 * layout as or_model_q8_rec) instead of the oracle's own quantization: a
 * layer then differs from a device run only by fp32 summation order. */
int       or_forward_inject_q8(or_model *m, int token, int pos, int lm_mode, const float *x_in,
                               const or_q8K *q8_in, float *x_out);
/* the K/V of every storing layer at pos from injected inputs x_in (as
 * or_forward_inject), without the rest of the layer; q8_in (nullable) as
 * or_forward_inject_q8 */
int       or_forward_inject_kv(or_model *m, int token, int pos, const float *x_in, const or_q8K *q8_in);
/* Pieces of forward() for checks against a composition of the reference's
 * own functions: the embedding and build_ple of a token (m->x, m->ple);
 * one layer from an injected input (its intermediates stay in the state
 * buffers); the final norm + logits_tied from an injected x. */
int       or_embed(or_model *m, int token, int pos);
int       or_layer_inject(or_model *m, int token, int pos, int layer, const float *x_in, float *x_out);
int       or_lm_head_inject(or_model *m, const float *x_in);
/* a state buffer by name: x, xb2, q, k, v, q_out, ple, ple_ctx, ple_gate,
 * hb, hb2, logits (main.c:694-701); NULL for other names */
float    *or_model_state(or_model *m, const char *name);
const float *or_model_logits(const or_model *m);
const float *or_model_x(const or_model *m);
/* Per-layer fingerprints captured during the last forward (sum,l2,max per layer
 * after the layer, plus K_store and q_out of layer 0). n_layers*3 floats. */
const float *or_model_layer_stats(const or_model *m);
const float *or_model_attn_stats(const or_model *m);
/* x after every layer of the last forward (n_layers*dim floats) */
const float *or_model_layer_x(const or_model *m);
/* Quantization points of a layer whose input goes through Q8_K when the
 * matrix is Q4_K/Q5_K (main.c:1884, 1975, and mm's own quantize at 1685 for
 * O, inp_gate and proj): slot s of layer l holds OR_Q8_SLOT_BLOCKS blocks at
 * block offset (l * OR_Q8_SLOTS + s) * OR_Q8_SLOT_BLOCKS. */
enum { OR_Q8_SLOT_ATTN = 0, OR_Q8_SLOT_O, OR_Q8_SLOT_FFN, OR_Q8_SLOT_INP_GATE, OR_Q8_SLOT_PROJ, OR_Q8_SLOTS };
#define OR_Q8_SLOT_BLOCKS 16
/* the oracle's own Q8_K of every slot in the last forward (n_layers x slots) */
const or_q8K *or_model_q8_rec(const or_model *m);
/* Layer-0 dump_kv_fingerprint records of the last forward (main.c:1829-1836,
 * 1880-1951): per tag sum, l2, max, v0..v3; have[t] = 0 for a tag the last
 * forward did not record (K_readN at pos 0). */
enum { OR_FP_ATTN_NORM = 0, OR_FP_K_PRE_NORM, OR_FP_K_PRE_ROPE, OR_FP_K_STORE, OR_FP_K_READ0, OR_FP_K_READN,
       OR_FP_Q_OUT, OR_FP_TAGS };
const float *or_model_fingerprint(const or_model *m, int *have);
/* the layer whose KV cache layer l reads (itself, or donor 22/23), main.c:739-746 */
int or_model_kv_source(const or_model *m, int layer);
/* the K (which 0) or V (1) cache of a storing layer: max_seq rows of
 * OR_MAX_KV_DIM floats (main.c:1798-1809); NULL for other layers */
float *or_model_kv(or_model *m, int layer, int which);
/* Greedy generation loop (main.c:2335-2488 with temp=0): prompt is fed
 * token-serially, then max_new tokens are produced.  out_tokens receives
 * the generated ids; returns the count.  Stops on eos/eot. */
int or_generate_greedy(or_model *m, const int *prompt, int n_prompt, int max_new,
                       int *out_tokens, double *prefill_sec, double *decode_sec);

#ifdef __cplusplus
}
#endif
#endif
