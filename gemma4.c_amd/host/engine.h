/*
 * engine.h -- C11 host engine of the MI355X decode path (libg4engine.so).
 *
 * Keeps the structure of the reference engine, thamada/Gemma4.c
 * gemma4-4b/cpu-blas/main.c: GGUF parse (parse_gguf, main.c:841-966), tensor
 * binding (load_weights, main.c:1328-1400), state allocation (alloc_state,
 * main.c:1402-1423), the per-token forward() (main.c:1838-2029) and the greedy
 * generation loop (generate, main.c:2335-2488).  Every computation is a call
 * into libg4hip.so's C ABI (include/g4hip.h); weights, activations and the
 * KV cache live in HBM.
 *
 * All functions return 0 on success or a G4_ERR_* code; the message is in
 * g4e_last_error().  The reference prints and exit(1)s instead.
 */
#ifndef G4_ENGINE_H
#define G4_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct g4e_model g4e_model;

/* GGUF image in host memory (borrowed for the call only): parse, upload to
 * HBM, allocate the device state.  max_seq <= 0 takes the model's
 * context_length.  device: HIP device ordinal. */
int  g4e_open_image(const void *data, size_t size, int max_seq, int device, g4e_model **out);
/* parse_gguf + the shape/type checks of load_weights, host only (no device):
 * 0 if the image can be opened; out (nullable) gets g4e_config's fields. */
int  g4e_check_image(const void *data, size_t size, int max_seq, int out[9]);
/* same, from a file (mmap'd read-only and private, as main.c:2770-2782) */
int  g4e_open_file(const char *path, int max_seq, int device, g4e_model **out);
void g4e_close(g4e_model *m);
const char *g4e_last_error(void);

/* dim, hidden, n_layers, n_heads, n_kv, vocab, max_seq, ple_dim, window */
void g4e_config(const g4e_model *m, int out[9]);

/* forward(m, token, pos, lm_mode), main.c:1838: lm_mode 0 stops after the
 * layers (prefill), otherwise the logits are computed (soft-capped); lm_mode
 * 2 also picks the greedy token in the LM head's own pass (mm_argmax_row,
 * main.c:1570-1667, 1784-1786; g4e_argmax then returns the same token). */
int g4e_forward(g4e_model *m, int token, int pos, int lm_mode);
int g4e_read_logits(g4e_model *m, float *host);       /* vocab floats */
int g4e_read_x(g4e_model *m, float *host);            /* dim floats   */
/* first index of the maximum logit (sample_token with temp <= 0, main.c:2045-2049) */
int g4e_argmax(g4e_model *m, int *tok);

/* Per-layer capture, for parity checks.  When on, every step (eager or in
 * the captured decode graph) copies x into a device trace of (n_layers + 1)
 * * dim floats: row 0 after the embedding (the input of layer 0), row l+1
 * after layer l; and the Q8_K activation of each quantization point of each
 * layer whose matrix takes Q8_K inputs (G4E_Q8_SLOT_*: attention input, O
 * input, FFN input, PLE inp_gate input, PLE proj input).  g4e_forward and
 * g4e_decode_steps copy the trace of their last step to host buffers:
 * g4e_layer_x, and g4e_layer_q8 as BlockQ8_K structs (main.c:117-122),
 * G4E_Q8_SLOT_ELEMS / 256 blocks per slot at block offset
 * (l * G4E_Q8_SLOTS + slot) * (G4E_Q8_SLOT_ELEMS / 256). */
enum { G4E_Q8_SLOT_ATTN = 0, G4E_Q8_SLOT_O, G4E_Q8_SLOT_FFN, G4E_Q8_SLOT_INP_GATE, G4E_Q8_SLOT_PROJ, G4E_Q8_SLOTS };
#define G4E_Q8_SLOT_ELEMS 4096
int g4e_set_trace(g4e_model *m, int on);
const float *g4e_layer_x(const g4e_model *m);
const void *g4e_layer_q8(const g4e_model *m);

/* generate() with temp <= 0 (main.c:2335-2488): the prompt is fed token by
 * token (lm_mode 0 except the last prompt token), then up to max_new greedy
 * tokens; stops at eos.  Returns the number generated (>= 0) or -code.
 * use_graph: decode steps replay one captured HIP graph (token and position
 * live in device memory and are advanced by the argmax kernel). */
int g4e_generate_greedy(g4e_model *m, const int *prompt, int n_prompt, int max_new, int *out_tokens,
                        double *prefill_sec, double *decode_sec, int use_graph);

/* generate (main.c:2335-2488) with sampling: after each decode step the
 * device sampler (g4_sample) applies the repetition penalty (penalty > 1)
 * over the last penalty_last_n generated tokens and draws from top-k
 * (1..64; the reference uses 40), temperature temp (<= 0: greedy) and top-p
 * topp with the xorshift64* stream seeded by seed (0 means 1, as the
 * reference).  Stops at max_new tokens or eos; returns the count (negative:
 * -status).  use_graph: one captured graph per decode step (forward and
 * sampler; recaptured when the settings change). */
int g4e_generate(g4e_model *m, const int *prompt, int n_prompt, int max_new, float temp, float topp, int topk,
                 float penalty, int penalty_last_n, uint64_t seed, int *out_tokens, double *prefill_sec,
                 double *decode_sec, int use_graph);

/* g4e_decode_steps with the device sampler after every step (settings as
 * g4e_generate; the history starts empty and the rng at seed) */
int g4e_decode_steps_sampled(g4e_model *m, int token, int pos0, int steps, float temp, float topp, int topk,
                             float penalty, int penalty_last_n, uint64_t seed, int use_graph, int *out, double *sec);

/* Timed decode: runs `steps` greedy decode steps from position pos0 with the
 * given input token (after a prefill that filled positions < pos0); returns
 * seconds through *sec.  Tokens are written to out (steps ints, nullable). */
int g4e_decode_steps(g4e_model *m, int token, int pos0, int steps, int use_graph, int *out, double *sec);

/* forward() of n consecutive tokens at positions pos0.. with lm_mode 0, as
 * the prompt loop of generate (main.c:2366-2384) runs them, processed in
 * chunks (g4e_set_prefill_chunk, default G4E_PREFILL_CHUNK tokens) layer by
 * layer: batched GEMMs, attention over the chunk's query rows against the
 * cache and the chunk's own K/V.  Each layer agrees with the token loop to
 * fp32 tolerance; the result does not depend on the chunk length or on how
 * the prompt is split over calls (bit for bit).  The chunk buffers are
 * allocated by the first call.  Returns after the work has completed. */
int g4e_prefill(g4e_model *m, const int *tokens, int n, int pos0);
/* g4e_prefill that also copies each layer's input rows to the host: trace
 * holds (n_layers + 1) x n x dim floats; row (l, t) is the input of layer l
 * for token t, row (n_layers, t) the last layer's output */
int g4e_prefill_trace(g4e_model *m, const int *tokens, int n, int pos0, float *trace);
/* ... and the Q8_K rows of every quantization point (G4E_Q8_SLOT_*) as
 * BlockQ8_K structs: q8trace[l][t][slot][G4E_Q8_SLOT_ELEMS / 256], zero where
 * the layer's matrix takes no Q8_K input */
int g4e_prefill_trace_q8(g4e_model *m, const int *tokens, int n, int pos0, float *trace, void *q8trace);
/* longest prompt chunk of g4e_prefill, and its default */
#define G4E_PREFILL_CHUNK 512
/* tokens per prompt chunk (1..G4E_PREFILL_CHUNK; at most what the chunk
 * buffers hold once g4e_prefill has sized them); 0 makes g4e_generate_greedy
 * prefill token by token as the reference's prompt loop does */
int g4e_set_prefill_chunk(g4e_model *m, int tokens);
/* --dump-hidden-at (main.c:1811, 1857-2010): the forward of position pos
 * (eager decode steps, token-by-token or chunked prompts; generate runs
 * without graphs while it is set) records hidden_stats of x after the
 * embedding, after each layer's attention residual and at each layer's end;
 * -1 turns it off.  g4e_hidden_stats copies the last record: (2 n_layers + 1)
 * x (sum, l2, max) floats, rows 0, then 1 + 2l (attention residual of layer
 * l) and 2 + 2l (end of layer l). */
int g4e_set_dump_hidden_at(g4e_model *m, int pos);
int g4e_hidden_stats(g4e_model *m, float *out);
/* The layer-0 dump_kv_fingerprint records of the same dump (main.c:1829-
 * 1836, 1880-1951): per tag sum, l2, max (hidden_stats) and the first four
 * values v0..v3, 7 floats, in G4E_FP_* order; have[t] = 0 where the tag was
 * not recorded (K_readN at pos 0, K_read0 once a sliding-window ring has
 * overwritten position 0). */
enum { G4E_FP_ATTN_NORM = 0, G4E_FP_K_PRE_NORM, G4E_FP_K_PRE_ROPE, G4E_FP_K_STORE, G4E_FP_K_READ0, G4E_FP_K_READN,
       G4E_FP_Q_OUT, G4E_FP_TAGS };
int g4e_kv_fingerprint(g4e_model *m, float *out, int *have);
/* SHA-256 of a file as 64 lowercase hex digits (hex[64] = 0), and the
 * `sha256sum --check` of the model download (gemma4-4b/Makefile `model`,
 * design.md:107-117): the line of sumfile naming path's base name must carry
 * its digest (G4_ERR_FORMAT otherwise).  Host only. */
int g4e_sha256_file(const char *path, char hex[65]);
int g4e_check_sha256sum(const char *path, const char *sumfile);
/* 1: Q4_K/Q5_K matrices through mm_quant_rows (dequantized weights times
 * fp32 activations) instead of Q8_K integer dots, the reference's
 * --f32-matmul switch (main.c:1680-1683, 2736); 0: the default */
int g4e_set_f32_matmul(g4e_model *m, int on);
/* KV cache of a storing layer: out[0] = floats per slot (n_kv * head_dim),
 * out[1] = slots (the window for a sliding-window ring, else max_seq) */
int g4e_kv_info(const g4e_model *m, int layer, int out[2]);
/* copy slots slot0..slot0+nslots-1 of the layer's K and V caches to the host */
int g4e_read_kv(g4e_model *m, int layer, int slot0, int nslots, float *k, float *v);

/* generate() one step at a time (main.c:2366-2470), for hosts that decide
 * between steps (forced tokens, the thinking budget, logit dumps):
 * g4e_gen_begin resets the generated-token history and seeds the sampler
 * (seed 0 -> 1).  g4e_gen_step runs forward(token, pos) with logits, then,
 * unless the host forces a token (forced >= 0: no draw is taken, as the
 * reference skips sample_token), the repetition penalty over the tokens
 * generated so far and sample_token (temp <= 0: first-index argmax) on the
 * device; the token is appended to that history and returned in next (the
 * logits stay readable with g4e_read_logits).  The prompt goes through
 * g4e_prefill first. */
int g4e_gen_begin(g4e_model *m, uint64_t seed);
int g4e_gen_step(g4e_model *m, int token, int pos, float temp, float topp, int topk, float penalty, int penalty_last_n,
                 int forced, int use_graph, int *next);

#ifdef __cplusplus
}
#endif
#endif
