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
 * layers (prefill), otherwise the logits are computed (soft-capped). */
int g4e_forward(g4e_model *m, int token, int pos, int lm_mode);
int g4e_read_logits(g4e_model *m, float *host);       /* vocab floats */
int g4e_read_x(g4e_model *m, float *host);            /* dim floats   */
/* first index of the maximum logit (sample_token with temp <= 0, main.c:2045-2049) */
int g4e_argmax(g4e_model *m, int *tok);

/* Per-layer capture: when on, forward() copies x into a host buffer of
 * (n_layers + 1) * dim floats (g4e_layer_x): row 0 after the embedding (the
 * input of layer 0), row l+1 after layer l.  Synchronous and slow; for parity
 * checks and fingerprints (dump_kv_fingerprint, main.c:1829-1836). */
int g4e_set_trace(g4e_model *m, int on);
const float *g4e_layer_x(const g4e_model *m);

/* generate() with temp <= 0 (main.c:2335-2488): the prompt is fed token by
 * token (lm_mode 0 except the last prompt token), then up to max_new greedy
 * tokens; stops at eos.  Returns the number generated (>= 0) or -code.
 * use_graph: decode steps replay one captured HIP graph (token and position
 * live in device memory and are advanced by the argmax kernel). */
int g4e_generate_greedy(g4e_model *m, const int *prompt, int n_prompt, int max_new, int *out_tokens,
                        double *prefill_sec, double *decode_sec, int use_graph);

/* Timed decode: runs `steps` greedy decode steps from position pos0 with the
 * given input token (after a prefill that filled positions < pos0); returns
 * seconds through *sec.  Tokens are written to out (steps ints, nullable). */
int g4e_decode_steps(g4e_model *m, int token, int pos0, int steps, int use_graph, int *out, double *sec);

#ifdef __cplusplus
}
#endif
#endif
