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

/* ---- GGUF reader and weight loading, main.c:778-966, 1318-1400 ---------- */
/* The reference's own parse_gguf + init_tokenizer + load_weights over a GGUF
 * image held in memory (borrowed).  Returns the reference's Model. */
void *ref_model_open(const void *data, size_t size) {
    Model *m = (Model *)calloc(1, sizeof(Model));
    m->fdata = (uint8_t *)data;
    m->fsz = size;
    m->fd = -1;
    char **merges = NULL;
    int n_merges = 0;
    parse_gguf(m, &merges, &n_merges);
    init_tokenizer(&m->tok, merges, n_merges);
    load_weights(m);
    return m;
}

/* i: dim, hidden, n_layers, n_heads, n_kv, vocab, max_seq, ple_dim, window,
 * shared_kv, swa_pattern, hd_swa, hd_full, rot_swa, rot_full; f: theta,
 * theta_swa, eps, softcap; doff: the data offset */
void ref_model_config(const void *mp, int *i, float *f, unsigned long long *doff) {
    const Model *m = (const Model *)mp;
    const Config *c = &m->cfg;
    const int v[15] = {c->dim, c->hidden_dim, c->n_layers, c->n_heads, c->n_kv_heads, c->vocab_size, c->max_seq,
                       c->ple_dim, c->sliding_window, c->shared_kv_layers, c->swa_pattern, c->head_dim_swa,
                       c->head_dim_full, c->n_rot_swa, c->n_rot_full};
    memcpy(i, v, sizeof v);
    f[0] = c->rope_theta; f[1] = c->rope_theta_swa; f[2] = c->norm_eps; f[3] = c->logit_softcapping;
    *doff = m->doff;
}

int ref_model_is_swa(const void *mp, int l) { return is_swa_layer(&((const Model *)mp)->cfg, l); }
int ref_model_kv_source(const void *mp, int l) { return kv_source_for_layer(&((const Model *)mp)->cfg, l); }

const void *ref_model_tensor(void *mp, const char *name, int *type) {
    int t = -1;
    const void *p = find_tensor((Model *)mp, name, &t);
    if (type) *type = t;
    return p;
}

/* ---- tokenizer, main.c:968-1312 ---------------------------------------- */
/* bos, eos, eot, add_space_prefix, turn_start, turn_end, turn_user,
 * turn_model, turn_system, think, channel, channel_thought, channel_end */
void ref_tok_specials(const void *mp, int *out) {
    const Tok *tk = &((const Model *)mp)->tok;
    const int v[13] = {tk->bos, tk->eos, tk->eot, tk->add_space_prefix, tk->turn_start, tk->turn_end, tk->turn_user,
                       tk->turn_model, tk->turn_system, tk->think, tk->channel, tk->channel_thought, tk->channel_end};
    memcpy(out, v, sizeof v);
}
float ref_tok_score(const void *mp, int id) { return ((const Model *)mp)->tok.scores[id]; }
int ref_tok_lookup(void *mp, const char *s, int len) { return tok_lookup(&((Model *)mp)->tok, s, len); }
/* gemma_bpe_encode of raw bytes; returns the count */
int ref_bpe_encode(void *mp, const char *text, int len, int *out) {
    int n = 0;
    int *t = gemma_bpe_encode(&((Model *)mp)->tok, text, len, &n);
    memcpy(out, t, (size_t)n * sizeof(int));
    free(t);
    return n;
}
/* append_gemma_text (line split, escape, BPE); returns the count */
int ref_gemma_text(void *mp, const char *text, int *out) {
    int n = 0;
    append_gemma_text(&((Model *)mp)->tok, out, &n, text);
    return n;
}
/* chat_encode of one user prompt (with the thinking system turn if asked) */
int ref_chat_encode(void *mp, const char *prompt, int thinking, int *out) {
    int n = 0;
    int *t = chat_encode(&((Model *)mp)->tok, prompt, thinking, &n);
    memcpy(out, t, (size_t)n * sizeof(int));
    free(t);
    return n;
}

/* ---- fingerprints, main.c:1811-1836 ----------------------------------------- */
void ref_hidden_stats(const float *v, int n, float *sum, float *l2, float *amax) { hidden_stats(v, n, sum, l2, amax); }
size_t ref_kv_cache_offset(int layer, int pos, int max_seq) { return kv_cache_offset(layer, pos, 0, max_seq); }

/* the tokenizer alone: parse_gguf + init_tokenizer (no weights needed) */
void *ref_tok_open(const void *data, size_t size) {
    Model *m = (Model *)calloc(1, sizeof(Model));
    m->fdata = (uint8_t *)data;
    m->fsz = size;
    m->fd = -1;
    char **merges = NULL;
    int n_merges = 0;
    parse_gguf(m, &merges, &n_merges);
    init_tokenizer(&m->tok, merges, n_merges);
    return m;
}
/* chat_encode_history over texts[i] with roles[i] (0 user, 1 model) */
int ref_chat_encode_history(void *mp, const char *const *texts, const int *roles, int n, int thinking, int *out,
                            int max_toks) {
    ChatHistory h;
    chat_history_init(&h);
    for (int i = 0; i < n; i++) chat_history_push(&h, roles[i] ? CHAT_ASSISTANT : CHAT_USER, texts[i]);
    const int r = chat_encode_history(&((Model *)mp)->tok, &h, thinking, out, max_toks);
    chat_history_free(&h);
    return r;
}
/* tokens_to_text into out (cap bytes); returns the length */
int ref_tokens_to_text(void *mp, const int *tokens, int start, int end, char *out, int cap) {
    char *s = tokens_to_text(&((Model *)mp)->tok, tokens, start, end);
    const int n = (int)strlen(s);
    if (n < cap) memcpy(out, s, (size_t)n + 1);
    free(s);
    return n;
}
/* parse_response: (thinking, answer) texts, or thinking absent (-1 length) */
void ref_parse_response(void *mp, const int *tokens, int n, char *think, int *think_len, char *answer, int *ans_len,
                        int cap) {
    char *t = NULL, *a = NULL;
    parse_response(&((Model *)mp)->tok, tokens, n, &t, &a);
    *think_len = t ? (int)strlen(t) : -1;
    *ans_len = a ? (int)strlen(a) : -1;
    if (t && *think_len < cap) memcpy(think, t, (size_t)*think_len + 1);
    if (a && *ans_len < cap) memcpy(answer, a, (size_t)*ans_len + 1);
    free(t);
    free(a);
}
int ref_is_special(void *mp, int id) { return is_special(&((Model *)mp)->tok, id); }
