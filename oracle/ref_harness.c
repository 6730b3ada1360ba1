/*
 * oracle/ref_harness.c -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is not compiled on its own.  oracle/Makefile streams the
 * BLAS-free hot-path functions of the reference (line ranges of
 * gemma4-4b/cpu-blas/main.c, read where they lie) into gcc followed by
 * this file, which exports them under ref_* names so that tests can call
 * the reference's own code.  Nothing of the reference is stored in the
 * repository; the result is oracle/_ref/libg4ref.so.
 *
 * Everything used below (BlockQ8_K, quantize_row_q8_K, ...) is defined by
 * the reference lines that precede this file in the compiler's input.
 */

void ref_quantize_row_q8_K(const float *x, void *y, int k) { quantize_row_q8_K(x, (BlockQ8_K *)y, k); }
void ref_quantize_row_q8_K_ref(const float *x, void *y, int k) { quantize_row_q8_K_ref(x, (BlockQ8_K *)y, k); }

float ref_vec_dot_q4_K_q8_K(int n, const void *x, const void *y) {
    float o = 0.0f;
    vec_dot_q4_K_q8_K(n, (const BlockQ4_K *)x, (const BlockQ8_K *)y, &o);
    return o;
}
float ref_vec_dot_q5_K_q8_K(int n, const void *x, const void *y) {
    float o = 0.0f;
    vec_dot_q5_K_q8_K(n, (const BlockQ5_K *)x, (const BlockQ8_K *)y, &o);
    return o;
}
float ref_vec_dot_q4_K_q8_K_generic(int n, const void *x, const void *y) {
    float o = 0.0f;
    vec_dot_q4_K_q8_K_generic(n, (const BlockQ4_K *)x, (const BlockQ8_K *)y, &o);
    return o;
}
float ref_vec_dot_q5_K_q8_K_generic(int n, const void *x, const void *y) {
    float o = 0.0f;
    vec_dot_q5_K_q8_K_generic(n, (const BlockQ5_K *)x, (const BlockQ8_K *)y, &o);
    return o;
}

float ref_host_f16f32(unsigned short h) { return host_f16f32(h); }
float ref_host_bf16f32(unsigned short h) { return host_bf16f32(h); }
void ref_get_scale_min_k4(int j, const unsigned char *q, unsigned char *d, unsigned char *m) {
    get_scale_min_k4(j, q, d, m);
}
void ref_dequant_block(const void *blk, int type, float *dst) { dequant_one_block_to(blk, type, dst); }

void ref_mm_quant_rows(float *o, const float *x, const void *w, int n, int d, int type) {
    mm_quant_rows(o, x, w, n, d, type);
}
void ref_mm_quant_dot_rows(float *o, const void *w, int n, int d, int type, const void *q8) {
    mm_quant_dot_rows(o, w, n, d, type, (const BlockQ8_K *)q8);
}
void ref_mm_bf16(float *o, const float *x, const unsigned short *w, int n, int d) { mm_bf16(o, x, w, n, d); }
void ref_mm_f16(float *o, const float *x, const unsigned short *w, int n, int d) { mm_f16(o, x, w, n, d); }

void ref_rmsnorm(float *o, const float *x, const float *w, int n, float eps) { rmsnorm(o, x, w, n, eps); }
void ref_rmsnorm_head_inplace(float *v, const float *w, int nh, int hd, float eps) {
    rmsnorm_head_inplace(v, w, nh, hd, eps);
}
void ref_rmsnorm_head_noweight_inplace(float *v, int nh, int hd, float eps) {
    rmsnorm_head_noweight_inplace(v, nh, hd, eps);
}
void ref_softmax(float *x, int n) { softmax(x, n); }
float ref_gelu(float x) { return gelu_f32(x); }
void ref_apply_rope_neox(float *v, int nh, int hd, int n_rot, int pos, float base, float fs, const float *ff) {
    apply_rope_neox(v, nh, hd, n_rot, pos, base, fs, ff);
}
void ref_emb_lookup(float *o, const void *w, int type, int id, int dim) { emb_lookup(o, w, type, id, dim); }

float ref_rng_f32(unsigned long long *s) { uint64_t t = *s; float r = rng_f32(&t); *s = t; return r; }
int ref_sample_token(float *logits, int n, float temp, float topp, int topk, unsigned long long *rng) {
    uint64_t t = *rng;
    int r = sample_token(logits, n, temp, topp, topk, &t);
    *rng = t;
    return r;
}

void ref_apply_repetition_penalty(float *logits, const int *tokens, int n_tokens, float penalty, int penalty_last_n) {
    apply_repetition_penalty(logits, tokens, n_tokens, penalty, penalty_last_n);
}

/* layer routing, main.c:716-746, on a Config with only the routing fields set */
int ref_is_swa_layer(int n_layers, int swa_pattern, int l) {
    Config c;
    memset(&c, 0, sizeof c);
    c.n_layers = n_layers;
    c.swa_pattern = swa_pattern;
    return is_swa_layer(&c, l);
}
int ref_kv_source_for_layer(int n_layers, int swa_pattern, int l) {
    Config c;
    memset(&c, 0, sizeof c);
    c.n_layers = n_layers;
    c.swa_pattern = swa_pattern;
    return kv_source_for_layer(&c, l);
}
int ref_layer_head_dim(int n_layers, int swa_pattern, int hd_swa, int hd_full, int l) {
    Config c;
    memset(&c, 0, sizeof c);
    c.n_layers = n_layers;
    c.swa_pattern = swa_pattern;
    c.head_dim_swa = hd_swa;
    c.head_dim_full = hd_full;
    return layer_head_dim(&c, l);
}
