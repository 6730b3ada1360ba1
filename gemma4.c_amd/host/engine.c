/*
 * engine.c -- C11 host engine over libg4hip.so (see engine.h).
 *
 * Structure follows thamada/Gemma4.c gemma4-4b/cpu-blas/main.c: the GGUF
 * reader and metadata defaults of parse_gguf (main.c:841-966), the tensor
 * names of load_weights (main.c:1328-1400), the layer routing helpers
 * (main.c:716-746), forward() (main.c:1838-2029) and the greedy branch of
 * generate() (main.c:2335-2488).  Arithmetic is done only by the HIP library.
 */
#define _POSIX_C_SOURCE 200809L
#include "engine.h"

#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include "../../include/g4hip.h"

#define E_N_LAYER_KV 24      /* main.c:77: layers 0..23 store KV; the tail reads 22/23 */
#define E_MAX_LAYERS 256

enum { GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };

static char g_err[512];

const char *g4e_last_error(void) { return g_err; }

static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

/* a failed g4_* call: keep the library's message */
static int lib_fail(int rc, const char *what) {
    snprintf(g_err, sizeof g_err, "%s: %s", what, g4_last_error());
    return rc;
}
#define CK(call)                                   \
    do {                                           \
        int rc_ = (call);                          \
        if (rc_) return lib_fail(rc_, #call);      \
    } while (0)

typedef struct {
    void *p;     /* device */
    int type, n, d;
} Tensor;

typedef struct {
    int dim, hidden, n_layers, n_heads, n_kv, vocab, max_seq, ple_dim, window;
    int swa_pattern, hd_swa, hd_full, rot_swa, rot_full, eos;
    float theta, theta_swa, eps, softcap;
    int swa[E_MAX_LAYERS];
    int has_swa_list;
} Config;

struct g4e_model {
    Config c;
    /* weights (HBM) */
    Tensor embd, ple_tok, ple_proj;
    float *ple_proj_norm, *rope_freqs, *norm_out;
    float *attn_norm[E_MAX_LAYERS], *post_attn_norm[E_MAX_LAYERS], *ffn_norm[E_MAX_LAYERS];
    float *post_ffw_norm[E_MAX_LAYERS], *q_norm[E_MAX_LAYERS], *k_norm[E_MAX_LAYERS];
    float *post_norm[E_MAX_LAYERS], *out_scale[E_MAX_LAYERS];
    Tensor wq[E_MAX_LAYERS], wk[E_MAX_LAYERS], wv[E_MAX_LAYERS], wo[E_MAX_LAYERS];
    Tensor gate[E_MAX_LAYERS], up[E_MAX_LAYERS], down[E_MAX_LAYERS];
    Tensor inp_gate[E_MAX_LAYERS], proj[E_MAX_LAYERS];
    /* state (HBM) */
    float *x, *xb2, *hb, *q, *k, *v, *q_out, *ple, *ple_ctx, *ple_gate, *logits;
    float *x_alt;            /* second residual-stream buffer (fused prologues write the other one) */
    float *ybuf;             /* PLE projection output, read by the next residual step */
    float *x_last;           /* buffer holding the residual stream after the last step */
    void *q8;
    float *kc[E_N_LAYER_KV], *vc[E_N_LAYER_KV];
    int kv_ring[E_N_LAYER_KV];
    float *attn_part;
    float *rope_tab;         /* (cos, sin) per pair: [rot_swa/2] then [rot_full/2] */
    int G_swa, G_full;
    int *dstep;              /* [0] token, [1] pos, [2] argmax result */
    void *argmax_part;
    int *hstep;              /* pinned host mirror of dstep */
    void *stream;
    void *graph;             /* captured greedy decode step */
    /* prompt chunks (allocated on first use for pf_cap tokens; rows of the
     * chunk are contiguous) */
    int pf_cap, pf_Gmax;
    int pf_chunk;            /* tokens per prompt chunk; 0: generate prefills token by token */
    int *pf_tok;
    float *pf_x, *pf_xb2, *pf_q, *pf_k, *pf_v, *pf_ao, *pf_o, *pf_g, *pf_u, *pf_h, *pf_d, *pf_ig, *pf_pg, *pf_y;
    float *pf_ple, *pf_ctx, *pf_tab_swa, *pf_tab_full, *pf_part;
    void *pf_q8, *pf_q8a, *pf_q8p;
    float *pf_kch[3], *pf_vch[3];   /* chunk K/V: [0] scratch, [1] donor 22, [2] donor 23 */
    /* host */
    int trace;
    float *layer_x;
    void *allocs[4096];
    int n_allocs;
    int poison;              /* fill byte of new device buffers (G4E_POISON), -1: none */
};

/* ---- routing, main.c:716-746 ------------------------------------------------ */
static int is_swa(const Config *c, int l) {
    if (c->has_swa_list) return c->swa[l];
    if (c->swa_pattern <= 0) return 0;
    return (l % c->swa_pattern) < (c->swa_pattern - 1);
}
static int layer_hd(const Config *c, int l) { return is_swa(c, l) ? c->hd_swa : c->hd_full; }
static int layer_has_kv(int l) { return l < E_N_LAYER_KV; }
static int kv_source(const Config *c, int l) { return layer_has_kv(l) ? l : (is_swa(c, l) ? 22 : 23); }
static int is_q8_type(int t) { return t == G4_Q4_K || t == G4_Q5_K; }

/* ---- GGUF reader (main.c:782-966) ------------------------------------------ */
typedef struct { const uint8_t *d; uint64_t p, n; int bad; } Rd;

static int need(Rd *r, uint64_t k) {
    if (r->bad || r->p + k > r->n) { r->bad = 1; return 0; }
    return 1;
}
static uint32_t ru32(Rd *r) { uint32_t v = 0; if (need(r, 4)) memcpy(&v, r->d + r->p, 4); r->p += 4; return v; }
static uint64_t ru64(Rd *r) { uint64_t v = 0; if (need(r, 8)) memcpy(&v, r->d + r->p, 8); r->p += 8; return v; }
static float rf32(Rd *r) { float v = 0; if (need(r, 4)) memcpy(&v, r->d + r->p, 4); r->p += 4; return v; }
static const char *rstr(Rd *r, uint64_t *len) {
    uint64_t n = ru64(r);
    const char *s = (const char *)r->d + r->p;
    if (!need(r, n)) n = 0;
    r->p += n;
    *len = n;
    return s;
}
static void skip(Rd *r, uint32_t t, int depth) {
    if (r->bad || depth > 4) { r->bad = 1; return; }
    switch (t) {
    case GV_U8: case GV_I8: case GV_BOOL: r->p += 1; break;
    case GV_U16: case GV_I16: r->p += 2; break;
    case GV_U32: case GV_I32: case GV_F32: r->p += 4; break;
    case GV_U64: case GV_I64: case GV_F64: r->p += 8; break;
    case GV_STR: { uint64_t n = ru64(r); r->p += n; break; }
    case GV_ARR: {
        uint32_t at = ru32(r);
        uint64_t al = ru64(r);
        if (at == GV_STR || at == GV_ARR) {
            for (uint64_t i = 0; i < al && !r->bad; i++) skip(r, at, depth + 1);
        } else {
            static const int sz[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
            if (at > GV_F64) { r->bad = 1; break; }
            r->p += al * (uint64_t)sz[at];
        }
        break;
    }
    default: r->bad = 1;
    }
    if (r->p > r->n) r->bad = 1;
}
static int64_t rint_val(Rd *r, uint32_t t) {
    int64_t v = 0;
    switch (t) {
    case GV_U8: case GV_BOOL: if (need(r, 1)) v = r->d[r->p]; r->p += 1; break;
    case GV_I8: if (need(r, 1)) v = (int8_t)r->d[r->p]; r->p += 1; break;
    case GV_U16: { uint16_t x = 0; if (need(r, 2)) memcpy(&x, r->d + r->p, 2); r->p += 2; v = x; break; }
    case GV_I16: { int16_t x = 0; if (need(r, 2)) memcpy(&x, r->d + r->p, 2); r->p += 2; v = x; break; }
    case GV_U32: v = ru32(r); break;
    case GV_I32: v = (int32_t)ru32(r); break;
    case GV_U64: v = (int64_t)ru64(r); break;
    case GV_I64: v = (int64_t)ru64(r); break;
    case GV_F32: v = (int64_t)rf32(r); break;
    case GV_F64: { double x = 0; if (need(r, 8)) memcpy(&x, r->d + r->p, 8); r->p += 8; v = (int64_t)x; break; }
    default: skip(r, t, 0);
    }
    return v;
}
static float rfloat_val(Rd *r, uint32_t t) {
    switch (t) {
    case GV_F32: return rf32(r);
    case GV_F64: { double x = 0; if (need(r, 8)) memcpy(&x, r->d + r->p, 8); r->p += 8; return (float)x; }
    case GV_U32: return (float)ru32(r);
    case GV_I32: return (float)(int32_t)ru32(r);
    case GV_U64: return (float)ru64(r);
    case GV_I64: return (float)(int64_t)ru64(r);
    default: skip(r, t, 0); return 0.0f;
    }
}
static int key_is(const char *k, uint64_t kl, const char *lit) { return kl == strlen(lit) && !memcmp(k, lit, kl); }

typedef struct {
    const char *name;
    uint64_t nlen, off;
    uint64_t ne[4];
    int n_dims, type;
} TInfo;

/* ---- device allocation bookkeeping ----------------------------------------- */
static int dalloc(g4e_model *m, void **p, size_t bytes) {
    if (m->n_allocs >= (int)(sizeof m->allocs / sizeof m->allocs[0])) return fail(G4_ERR_NOMEM, "too many allocations");
    CK(g4_malloc(p, bytes ? bytes : 1));
    m->allocs[m->n_allocs++] = *p;
    if (m->poison >= 0) CK(g4_memset(*p, m->poison, bytes ? bytes : 1));
    return 0;
}

static size_t tensor_bytes(int type, uint64_t n, uint64_t d) {
    return g4_tensor_bytes(type, (int)n, (int)d);
}

static const TInfo *find_t(const TInfo *ti, int nt, const char *name) {
    const size_t L = strlen(name);
    for (int i = 0; i < nt; i++)
        if (ti[i].nlen == L && !memcmp(ti[i].name, name, L)) return &ti[i];
    return NULL;
}

/* upload one tensor; matrices [ne1 rows x ne0] of K-quant types go through the
 * planar layout, everything else is copied verbatim. */
static int upload(g4e_model *m, const uint8_t *base, const TInfo *t, Tensor *out) {
    const uint64_t n = t->ne[0], d = t->n_dims > 1 ? t->ne[1] : 1;
    if (t->n_dims > 2 || n == 0 || d == 0 || n > 0x7fffffff || d > 0x7fffffff)
        return fail(G4_ERR_FORMAT, "tensor %.*s: unsupported shape", (int)t->nlen, t->name);
    const size_t bytes = tensor_bytes(t->type, n, d);
    if (!bytes) return fail(G4_ERR_TYPE, "tensor %.*s: unsupported type %d or shape", (int)t->nlen, t->name, t->type);
    int rc = dalloc(m, &out->p, bytes);
    if (rc) return rc;
    out->type = t->type;
    out->n = (int)n;
    out->d = (int)d;
    const uint8_t *src = base + t->off;
    if (t->type == G4_Q4_K || t->type == G4_Q5_K || t->type == G4_Q6_K) CK(g4_upload_quant(out->p, src, t->type, (int)n, (int)d));
    else CK(g4_memcpy_h2d(out->p, src, bytes));
    return 0;
}

/* parse_gguf (main.c:841-966): metadata with the reference's defaults, the
 * tensor table, and the data offset.  Host only. */
typedef struct {
    TInfo *ti;
    uint64_t nt;
    const uint8_t *base;
} Image;

static int parse(const uint8_t *data, size_t size, int max_seq, Config *c, Image *img) {
    Rd r = {data, 0, size, 0};
    memset(c, 0, sizeof *c);
    img->ti = NULL;
    if (size < 24 || ru32(&r) != 0x46554747u) return fail(G4_ERR_FORMAT, "Error: invalid GGUF magic");
    (void)ru32(&r);
    const uint64_t n_tensors = ru64(&r), n_kv = ru64(&r);
    /* defaults, main.c:854-871 */
    c->theta = 1e6f; c->theta_swa = 10000.0f; c->eps = 1e-6f; c->max_seq = 8192; c->swa_pattern = 6;
    c->hd_swa = 256; c->hd_full = 512; c->rot_swa = 256; c->rot_full = 512; c->ple_dim = 256;
    c->window = 512; c->softcap = 30.0f; c->eos = 106;
    uint32_t alignment = 32;
    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        uint64_t kl;
        const char *k = rstr(&r, &kl);
        const uint32_t vt = ru32(&r);
#define KI(lit, field) else if (key_is(k, kl, lit)) field = (int)rint_val(&r, vt)
#define KF(lit, field) else if (key_is(k, kl, lit)) field = rfloat_val(&r, vt)
        if (key_is(k, kl, "general.alignment")) alignment = (uint32_t)rint_val(&r, vt);
        KI("gemma4.embedding_length", c->dim);
        KI("gemma4.feed_forward_length", c->hidden);
        KI("gemma4.block_count", c->n_layers);
        KI("gemma4.attention.head_count", c->n_heads);
        KI("gemma4.attention.head_count_kv", c->n_kv);
        KI("gemma4.attention.key_length_swa", c->hd_swa);
        KI("gemma4.attention.key_length", c->hd_full);
        KI("gemma4.rope.dimension_count_swa", c->rot_swa);
        KI("gemma4.rope.dimension_count", c->rot_full);
        KF("gemma4.attention.layer_norm_rms_epsilon", c->eps);
        KF("gemma4.rope.freq_base", c->theta);
        KF("gemma4.rope.freq_base_swa", c->theta_swa);
        KI("gemma4.attention.sliding_window", c->window);
        KI("gemma4.embedding_length_per_layer_input", c->ple_dim);
        KF("gemma4.final_logit_softcapping", c->softcap);
        KI("gemma4.context_length", c->max_seq);
        KI("tokenizer.ggml.eos_token_id", c->eos);
        else if (key_is(k, kl, "gemma4.attention.sliding_window_pattern") && vt == GV_ARR) {
            const uint32_t et = ru32(&r);
            const uint64_t n = ru64(&r);
            if (n > 0 && n <= E_MAX_LAYERS && et != GV_STR && et != GV_ARR) {
                for (uint64_t j = 0; j < n; j++) c->swa[j] = rint_val(&r, et) ? 1 : 0;
                c->has_swa_list = 1;
            } else {
                for (uint64_t j = 0; j < n && !r.bad; j++) skip(&r, et, 1);
            }
        } else if (key_is(k, kl, "tokenizer.ggml.tokens") && vt == GV_ARR) {
            /* vocab_size = the length of the token list (main.c:922-931) */
            (void)ru32(&r);
            const uint64_t n = ru64(&r);
            c->vocab = (int)n;
            for (uint64_t j = 0; j < n && !r.bad; j++) { uint64_t sl; (void)rstr(&r, &sl); }
        } else {
            skip(&r, vt, 0);
        }
#undef KI
#undef KF
    }
    if (r.bad) return fail(G4_ERR_FORMAT, "truncated GGUF metadata");
    if (n_tensors > 100000) return fail(G4_ERR_FORMAT, "implausible tensor count %llu", (unsigned long long)n_tensors);
    TInfo *ti = (TInfo *)calloc(n_tensors ? n_tensors : 1, sizeof(TInfo));
    if (!ti) return fail(G4_ERR_NOMEM, "out of host memory");
    for (uint64_t i = 0; i < n_tensors && !r.bad; i++) {
        ti[i].name = rstr(&r, &ti[i].nlen);
        ti[i].n_dims = (int)ru32(&r);
        if (ti[i].n_dims < 1 || ti[i].n_dims > 4) { r.bad = 1; break; }
        for (int dd = 0; dd < ti[i].n_dims; dd++) ti[i].ne[dd] = ru64(&r);
        ti[i].type = (int)ru32(&r);
        ti[i].off = ru64(&r);
    }
    if (r.bad || alignment == 0) { free(ti); return fail(G4_ERR_FORMAT, "truncated GGUF tensor table"); }
    const uint64_t doff = (r.p + (alignment - 1)) & ~(uint64_t)(alignment - 1);
    for (uint64_t i = 0; i < n_tensors; i++) {
        const uint64_t n = ti[i].ne[0], d = ti[i].n_dims > 1 ? ti[i].ne[1] : 1;
        size_t b = tensor_bytes(ti[i].type, n, d);
        if (b == 0) b = (size_t)n * d;    /* unknown types are rejected only if used */
        if (doff + ti[i].off + b > size) { free(ti); return fail(G4_ERR_FORMAT, "tensor data past the end of the file"); }
    }
    if (max_seq > 0) c->max_seq = max_seq;
    if (c->n_layers <= 0 || c->n_layers > E_MAX_LAYERS || c->dim <= 0 || c->hidden <= 0 || c->n_heads <= 0 ||
        c->n_kv <= 0 || c->vocab <= 0 || c->max_seq <= 0 || c->n_heads % c->n_kv || c->ple_dim <= 0) {
        free(ti);
        return fail(G4_ERR_FORMAT, "bad model config (layers %d dim %d heads %d kv %d vocab %d)", c->n_layers, c->dim,
                    c->n_heads, c->n_kv, c->vocab);
    }
    img->ti = ti;
    img->nt = n_tensors;
    img->base = data + doff;
    return 0;
}

/* shape/type checks of everything load_weights binds (main.c:1328-1400);
 * the reference trusts the file, the device kernels do not. */
static int check_t(const Image *im, const char *name, const int *types, int ntypes, uint64_t n, uint64_t d,
                   int optional) {
    const TInfo *t = find_t(im->ti, (int)im->nt, name);
    if (!t) return optional ? 0 : fail(G4_ERR_FORMAT, "Error: missing tensor %s", name);
    int ok = 0;
    for (int i = 0; i < ntypes; i++) ok |= t->type == types[i];
    if (!ok) return fail(G4_ERR_TYPE, "Unsupported tensor type %d for %s", t->type, name);
    const uint64_t tn = t->ne[0], td = t->n_dims > 1 ? t->ne[1] : 1;
    if (t->n_dims > 2 || tn != n || td != d)
        return fail(G4_ERR_FORMAT, "%s: shape [%llu x %llu], expected [%llu x %llu]", name, (unsigned long long)tn,
                    (unsigned long long)td, (unsigned long long)n, (unsigned long long)d);
    if ((t->type == G4_Q4_K || t->type == G4_Q5_K || t->type == G4_Q6_K) && n % 256)
        return fail(G4_ERR_FORMAT, "%s: row length %llu not a multiple of 256", name, (unsigned long long)n);
    return 0;
}

static int validate(const Config *c, const Image *im) {
    static const int F32T[] = {G4_F32};
    static const int MAT[] = {G4_Q4_K, G4_Q5_K, G4_Q6_K};
    static const int Q45[] = {G4_Q4_K, G4_Q5_K};
    static const int Q6[] = {G4_Q6_K};
    static const int PROJ[] = {G4_BF16};
    const int L = c->n_layers;
    char name[128];
    int rc;
    if (c->hd_swa != 256 && c->hd_swa != 512) return fail(G4_ERR_FORMAT, "head_dim_swa %d unsupported", c->hd_swa);
    if (c->hd_full != 256 && c->hd_full != 512) return fail(G4_ERR_FORMAT, "head_dim %d unsupported", c->hd_full);
    if (c->n_heads / c->n_kv > 8) return fail(G4_ERR_FORMAT, "n_heads/n_kv > 8 unsupported");
    if (c->dim % 256 || c->ple_dim % 256) return fail(G4_ERR_FORMAT, "dim/ple_dim must be multiples of 256");
    if (c->n_layers > E_N_LAYER_KV && c->n_layers < 24) return fail(G4_ERR_FORMAT, "layer count");
    if (c->n_layers > E_N_LAYER_KV && (is_swa(c, 22) != 1 || is_swa(c, 23) != 0))
        return fail(G4_ERR_FORMAT, "shared-KV donors 22/23 must be sliding/full layers (main.c:743-746)");
    if ((rc = check_t(im, "token_embd.weight", Q6, 1, c->dim, c->vocab, 0)) ||
        (rc = check_t(im, "per_layer_token_embd.weight", MAT, 3, (uint64_t)c->ple_dim * L, c->vocab, 0)) ||
        (rc = check_t(im, "per_layer_model_proj.weight", PROJ, 1, c->dim, (uint64_t)c->ple_dim * L, 0)) ||
        (rc = check_t(im, "per_layer_proj_norm.weight", F32T, 1, c->ple_dim, 1, 0)) ||
        (rc = check_t(im, "output_norm.weight", F32T, 1, c->dim, 1, 0)) ||
        (rc = check_t(im, "rope_freqs.weight", F32T, 1, c->rot_full / 2, 1, 1)))
        return rc;
    for (int l = 0; l < L; l++) {
        const uint64_t hd = layer_hd(c, l), qd = c->n_heads * hd, kvd = c->n_kv * hd;
#define CT(suffix, types, nt_, n_, d_, opt)                                        \
        snprintf(name, sizeof name, "blk.%d." suffix, l);                          \
        if ((rc = check_t(im, name, types, nt_, n_, d_, opt))) return rc;
        CT("attn_norm.weight", F32T, 1, c->dim, 1, 0);
        CT("post_attention_norm.weight", F32T, 1, c->dim, 1, 0);
        CT("attn_q_norm.weight", F32T, 1, hd, 1, 0);
        CT("attn_k_norm.weight", F32T, 1, hd, 1, 0);
        CT("attn_q.weight", MAT, 3, c->dim, qd, 0);
        if (layer_has_kv(l)) {
            CT("attn_k.weight", MAT, 3, c->dim, kvd, 0);
            CT("attn_v.weight", MAT, 3, c->dim, kvd, 0);
        }
        CT("attn_output.weight", MAT, 3, qd, c->dim, 0);
        CT("ffn_norm.weight", F32T, 1, c->dim, 1, 0);
        CT("post_ffw_norm.weight", F32T, 1, c->dim, 1, 0);
        CT("ffn_gate.weight", Q45, 2, c->dim, c->hidden, 0);
        CT("ffn_up.weight", Q45, 2, c->dim, c->hidden, 0);
        CT("ffn_down.weight", MAT, 3, c->hidden, c->dim, 0);
        CT("inp_gate.weight", MAT, 3, c->dim, c->ple_dim, 0);
        CT("proj.weight", MAT, 3, c->ple_dim, c->dim, 0);
        CT("post_norm.weight", F32T, 1, c->dim, 1, 0);
        CT("layer_output_scale.weight", F32T, 1, 1, 1, 1);
#undef CT
        snprintf(name, sizeof name, "blk.%d.ffn_gate.weight", l);
        const TInfo *g = find_t(im->ti, (int)im->nt, name);
        snprintf(name, sizeof name, "blk.%d.ffn_up.weight", l);
        const TInfo *u = find_t(im->ti, (int)im->nt, name);
        if (g->type != u->type) return fail(G4_ERR_TYPE, "blk.%d: ffn_gate and ffn_up types differ", l);
    }
    return 0;
}

int g4e_check_image(const void *data, size_t size, int max_seq, int out[9]) {
    Config c;
    Image im;
    if (!data) return fail(G4_ERR_ARG, "g4e_check_image: null pointer");
    int rc = parse((const uint8_t *)data, size, max_seq, &c, &im);
    if (rc) return rc;
    rc = validate(&c, &im);
    free(im.ti);
    if (rc == 0 && out) {
        const int v[9] = {c.dim, c.hidden, c.n_layers, c.n_heads, c.n_kv, c.vocab, c.max_seq, c.ple_dim, c.window};
        memcpy(out, v, sizeof v);
    }
    return rc;
}

/* time chunks of the decode attention for a window capacity: about 32
 * positions per workgroup at full capacity, 1..128 chunks (more only if a
 * chunk would exceed 1024 positions) */
static int attn_chunks(int cap) {
    int G = (cap + 31) / 32;
    if (G < 1) G = 1;
    if (G > 128) G = 128;
    while ((cap + G - 1) / G > 1024) G++;
    return G;
}

/* load_weights (upload to HBM) + alloc_state (main.c:1328-1423) */
static int load(g4e_model *m, const Image *im) {
    const Config *c = &m->c;
    const int L = c->n_layers;
    char name[128];
    int rc;
#define UP(nm, dst)                                                                       \
    do {                                                                                  \
        const TInfo *t_ = find_t(im->ti, (int)im->nt, nm);                                \
        if (t_ && (rc = upload(m, im->base, t_, &(dst)))) return rc;                      \
    } while (0)
#define UPF(nm, dst)                                                                      \
    do {                                                                                  \
        Tensor tt_ = {0};                                                                 \
        UP(nm, tt_);                                                                      \
        dst = (float *)tt_.p;                                                             \
    } while (0)
    UP("token_embd.weight", m->embd);
    UP("per_layer_token_embd.weight", m->ple_tok);
    UP("per_layer_model_proj.weight", m->ple_proj);
    UPF("per_layer_proj_norm.weight", m->ple_proj_norm);
    UPF("output_norm.weight", m->norm_out);
    UPF("rope_freqs.weight", m->rope_freqs);
    for (int l = 0; l < L; l++) {
#define LT(suffix, dst) snprintf(name, sizeof name, "blk.%d." suffix, l); UP(name, dst);
#define LF(suffix, dst) snprintf(name, sizeof name, "blk.%d." suffix, l); UPF(name, dst);
        LF("attn_norm.weight", m->attn_norm[l]);
        LF("post_attention_norm.weight", m->post_attn_norm[l]);
        LF("attn_q_norm.weight", m->q_norm[l]);
        LF("attn_k_norm.weight", m->k_norm[l]);
        LT("attn_q.weight", m->wq[l]);
        if (layer_has_kv(l)) {
            LT("attn_k.weight", m->wk[l]);
            LT("attn_v.weight", m->wv[l]);
        }
        LT("attn_output.weight", m->wo[l]);
        LF("ffn_norm.weight", m->ffn_norm[l]);
        LF("post_ffw_norm.weight", m->post_ffw_norm[l]);
        LT("ffn_gate.weight", m->gate[l]);
        LT("ffn_up.weight", m->up[l]);
        LT("ffn_down.weight", m->down[l]);
        LT("inp_gate.weight", m->inp_gate[l]);
        LT("proj.weight", m->proj[l]);
        LF("post_norm.weight", m->post_norm[l]);
        LF("layer_output_scale.weight", m->out_scale[l]);
#undef LT
#undef LF
    }
#undef UP
#undef UPF

    /* alloc_state, in HBM */
    const int hdmax = c->hd_full > c->hd_swa ? c->hd_full : c->hd_swa;
    const int qmax = c->n_heads * hdmax, kvmax = c->n_kv * hdmax;
    int q8n = c->hidden > qmax ? c->hidden : qmax;
    if (c->dim > q8n) q8n = c->dim;
    q8n = (q8n + 255) / 256 * 256;
    void *p;
#define DA(field, bytes) if ((rc = dalloc(m, &p, (size_t)(bytes)))) return rc; field = p;
    DA(m->x, (size_t)c->dim * 4);
    DA(m->x_alt, (size_t)c->dim * 4);
    DA(m->ybuf, (size_t)c->dim * 4);
    m->x_last = m->x;
    DA(m->xb2, (size_t)c->dim * 4);
    DA(m->hb, (size_t)c->hidden * 4);
    DA(m->q, (size_t)qmax * 4);
    DA(m->k, (size_t)kvmax * 4);
    DA(m->v, (size_t)kvmax * 4);
    DA(m->q_out, (size_t)qmax * 4);
    DA(m->ple, (size_t)c->ple_dim * L * 4);
    DA(m->ple_ctx, (size_t)c->ple_dim * L * 4);
    DA(m->ple_gate, (size_t)c->ple_dim * 4);
    DA(m->logits, (size_t)c->vocab * 4);
    DA(m->q8, g4_q8K_bytes(q8n));
    DA(m->dstep, 64);
    DA(m->argmax_part, g4_argmax_part_bytes(c->vocab));
    /* KV: sliding-window layers keep a ring of `window` slots, full layers
     * max_seq slots; row stride = n_kv * head_dim of the layer */
    for (int l = 0; l < L && l < E_N_LAYER_KV; l++) {
        const int kvd = c->n_kv * layer_hd(c, l);
        int slots = c->max_seq, ring = 0;
        if (is_swa(c, l) && c->window > 0 && c->window < c->max_seq) { slots = c->window; ring = c->window; }
        DA(m->kc[l], (size_t)slots * kvd * 4);
        DA(m->vc[l], (size_t)slots * kvd * 4);
        m->kv_ring[l] = ring;
    }
    /* attention partials: chunk counts fixed from capacity (<= 1024 positions
     * per chunk) so that one captured graph serves every position */
    const int cap_swa = c->window > 0 && c->window < c->max_seq ? c->window : c->max_seq;
    m->G_swa = attn_chunks(cap_swa);
    m->G_full = attn_chunks(c->max_seq);
    const int Gmax = m->G_full > m->G_swa ? m->G_full : m->G_swa;
    DA(m->attn_part, g4_attn_part_bytes(c->n_heads, hdmax, Gmax));
#undef DA
    if ((rc = dalloc(m, &p, (size_t)(c->rot_swa / 2 + c->rot_full / 2) * 8))) return rc;
    m->rope_tab = p;
    CK(g4_host_alloc((void **)&m->hstep, 64));
    memset(m->hstep, 0, 64);
    return 0;
}

static int open_image(const uint8_t *data, size_t size, int max_seq, g4e_model *m) {
    Image im;
    int rc = parse(data, size, max_seq, &m->c, &im);
    if (rc) return rc;
    rc = validate(&m->c, &im);
    if (rc == 0) rc = load(m, &im);
    free(im.ti);
    return rc;
}

int g4e_open_image(const void *data, size_t size, int max_seq, int device, g4e_model **out) {
    if (!data || !out) return fail(G4_ERR_ARG, "g4e_open_image: null pointer");
    *out = NULL;
    CK(g4_init(device));
    g4e_model *m = (g4e_model *)calloc(1, sizeof *m);
    if (!m) return fail(G4_ERR_NOMEM, "out of host memory");
    int rc = g4_stream_create(&m->stream);
    if (rc) { free(m); return lib_fail(rc, "g4_stream_create"); }
    g4_set_stream(m->stream);
    /* G4E_POISON=<byte>: fill every device buffer with that byte when it is
     * allocated (0xff: NaN floats), so that a read of memory no kernel has
     * written shows in the results */
    const char *poison = getenv("G4E_POISON");
    m->poison = poison && *poison ? (int)(strtol(poison, NULL, 0) & 0xff) : -1;
    m->pf_chunk = G4E_PREFILL_CHUNK;
    rc = open_image((const uint8_t *)data, size, max_seq, m);
    if (rc == 0) rc = g4_sync() ? lib_fail(G4_ERR_HIP, "g4_sync") : 0;
    if (rc) { g4e_close(m); return rc; }
    *out = m;
    return 0;
}

int g4e_open_file(const char *path, int max_seq, int device, g4e_model **out) {
    if (!path || !out) return fail(G4_ERR_ARG, "g4e_open_file: null pointer");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(G4_ERR_ARG, "Error: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return fail(G4_ERR_ARG, "Error: cannot stat %s", path); }
    void *p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return fail(G4_ERR_NOMEM, "Error: mmap failed");
    const int rc = g4e_open_image(p, (size_t)st.st_size, max_seq, device, out);
    munmap(p, (size_t)st.st_size);
    return rc;
}

void g4e_close(g4e_model *m) {
    if (!m) return;
    g4_set_stream(m->stream);
    g4_sync();
    if (m->graph) g4_graph_destroy(m->graph);
    for (int i = 0; i < m->n_allocs; i++) g4_free(m->allocs[i]);
    if (m->hstep) g4_host_free(m->hstep);
    g4_set_stream(NULL);
    if (m->stream) g4_stream_destroy(m->stream);
    free(m->layer_x);
    free(m);
}

void g4e_config(const g4e_model *m, int out[9]) {
    const Config *c = &m->c;
    const int v[9] = {c->dim, c->hidden, c->n_layers, c->n_heads, c->n_kv, c->vocab, c->max_seq, c->ple_dim, c->window};
    memcpy(out, v, sizeof v);
}

/* ---- the step, main.c:1838-2029 ------------------------------------------ */

/* mm(o, x, w, n, d, type, q8, q8_ready), main.c:1669-1694 */
static int mm(g4e_model *m, float *o, const float *x, const Tensor *w, int q8_ready) {
    CK(g4_mm(o, x, w->p, w->n, w->d, w->type, m->q8, q8_ready));
    return 0;
}

/* Enqueue one forward step; token and position are read from m->dstep, so the
 * same sequence of launches is valid for every position (graph capture). */
/* a Q4_K/Q5_K GEMV that can take the residual step + norm + Q8_K as its
 * prologue (g4_mm_residual_q8) */
static int pro_ok(const Config *c, const Tensor *w) {
    const int nb = c->dim / 256;
    return is_q8_type(w->type) && c->dim % 256 == 0 && (nb == 8 || nb == 10 || nb == 16);
}

/* Enqueue one forward step; token and position are read from m->dstep, so the
 * same sequence of launches is valid for every position (graph capture).
 * The residual stream lives in two buffers: a GEMV whose prologue performs
 * a residual step reads one and writes the other (its workgroups run
 * concurrently); single-workgroup steps update it in place. */
static int enqueue_step(g4e_model *m, int lm_mode) {
    const Config *c = &m->c;
    const int dim = c->dim, L = c->n_layers, pd = c->ple_dim;
    const int *dtok = m->dstep, *dpos = m->dstep + 1;
    float *x = m->x, *xo = m->x_alt;
    /* emb_lookup * sqrt(dim) (main.c:1849-1854) and build_ple (main.c:1747-1778) */
    CK(g4_emb_lookup_dev(x, m->embd.p, m->embd.type, m->embd.d, dtok, dim, sqrtf((float)dim)));
    CK(g4_mm(m->ple_ctx, x, m->ple_proj.p, m->ple_proj.n, m->ple_proj.d, m->ple_proj.type, m->q8, 0));
    CK(g4_ple_finish(m->ple, m->ple_ctx, m->ple_tok.p, m->ple_tok.type, m->ple_tok.d, m->ple_proj_norm, dtok, 0, pd, L,
                     sqrtf((float)pd), 1.0f / sqrtf((float)dim), 1.0f / sqrtf(2.0f), c->eps));
    /* RoPE angles of this position for both layer types (main.c:1725-1742) */
    float *tab_swa = m->rope_tab, *tab_full = m->rope_tab + c->rot_swa;
    CK(g4_rope_table(tab_swa, dpos, 0, c->rot_swa, c->theta_swa, 1.0f, NULL));
    CK(g4_rope_table(tab_full, dpos, 0, c->rot_full, c->theta, 1.0f, m->rope_freqs));
    if (m->trace) CK(g4_memcpy_d2h(m->layer_x, x, (size_t)dim * 4));
    for (int l = 0; l < L; l++) {
        const int hd = layer_hd(c, l), swa = is_swa(c, l);
        const int n_rot = swa ? c->rot_swa : c->rot_full;
        const int q8_att = is_q8_type(m->wq[l].type);
        /* the previous layer's post_norm + residual + out_scale (main.c:1995-2003;
         * none before layer 0), this layer's attn_norm + Q8_K (main.c:1878-1884),
         * then Q, K, V on that one Q8_K of xb2 (main.c:1883-1892) */
        const float *y = l ? m->ybuf : NULL, *w_post = l ? m->post_norm[l - 1] : NULL;
        const float *osc = l ? m->out_scale[l - 1] : NULL;
        int rc;
        const int src = kv_source(c, l), has_kv = layer_has_kv(l);
        /* K rides in the Q launch when it has Q's type, and V with them when it
         * is Q6_K (fp32 path on the normed vector) */
        const int k_pair = has_kv && pro_ok(c, &m->wq[l]) && m->wk[l].type == m->wq[l].type;
        const int v_too = k_pair && m->wv[l].type == G4_Q6_K;
        if (v_too) {
            CK(g4_mm_residual_q8_qkv(m->q, m->wq[l].p, m->wq[l].d, m->k, m->wk[l].p, m->wk[l].d, m->v, m->wv[l].p,
                                     m->wv[l].d, m->wv[l].type, m->wq[l].n, m->wq[l].type, x, y ? xo : x, y, w_post, osc,
                                     m->attn_norm[l], m->xb2, m->q8, c->eps));
            if (y) { float *t = x; x = xo; xo = t; }
        } else if (k_pair) {
            CK(g4_mm_residual_q8_pair(m->q, m->wq[l].p, m->wq[l].d, m->k, m->wk[l].p, m->wk[l].d, m->wq[l].n,
                                      m->wq[l].type, x, y ? xo : x, y, w_post, osc, m->attn_norm[l], m->xb2, m->q8, 0,
                                      c->eps));
            if (y) { float *t = x; x = xo; xo = t; }
        } else if (pro_ok(c, &m->wq[l])) {
            CK(g4_mm_residual_q8(m->q, m->wq[l].p, NULL, m->wq[l].n, m->wq[l].d, m->wq[l].type, NULL, x, y ? xo : x, y,
                                 w_post, osc, m->attn_norm[l], m->xb2, m->q8, 0, c->eps));
            if (y) { float *t = x; x = xo; xo = t; }
        } else {
            CK(g4_residual_norm(x, y, w_post, osc, m->attn_norm[l], m->xb2, q8_att ? m->q8 : NULL, 0, dim, c->eps));
            if ((rc = mm(m, m->q, m->xb2, &m->wq[l], q8_att))) return rc;
        }
        if (m->trace && l > 0) CK(g4_memcpy_d2h(m->layer_x + (size_t)l * dim, x, (size_t)dim * 4));
        if (has_kv) {
            if (is_q8_type(m->wk[l].type) != q8_att && is_q8_type(m->wk[l].type))
                CK(g4_quantize_row_q8_K(m->xb2, m->q8, dim));
            if (!k_pair && (rc = mm(m, m->k, m->xb2, &m->wk[l], 1))) return rc;
            if (!v_too && (rc = mm(m, m->v, m->xb2, &m->wv[l], 1))) return rc;
        }
        /* q_norm + RoPE, K/V norm + RoPE + append (main.c:1886-1904) and the
         * attention over the source layer's cache (main.c:1909-1950, attn_scale
         * 1.0) in one launch pair */
        const int o_q8 = is_q8_type(m->wo[l].type);
        CK(g4_attn_decode_fused(m->q, m->q_norm[l], has_kv ? m->k : NULL, has_kv ? m->v : NULL,
                                has_kv ? m->k_norm[l] : NULL, has_kv ? m->kc[l] : NULL, has_kv ? m->vc[l] : NULL,
                                m->kc[src], m->vc[src], c->n_kv * layer_hd(c, src), m->kv_ring[src], dpos,
                                swa ? c->window : 0, c->n_heads, c->n_kv, hd, n_rot, swa ? tab_swa : tab_full, c->eps,
                                1.0f, swa ? m->G_swa : m->G_full, m->attn_part, m->q_out, o_q8 ? m->q8 : NULL));
        if ((rc = mm(m, m->xb2, m->q_out, &m->wo[l], o_q8))) return rc;
        /* post_attention_norm + residual, then ffn_norm + Q8_K (main.c:1960-1975),
         * in place (one workgroup), then gelu(gate) * up (main.c:1976-1980).  As
         * the prologue of every workgroup of the gate|up GEMV (g4_mm_residual_q8
         * with both matrices) the step costs as much as this launch: 14.5 us
         * against 5.0 + 9.5 us at the E4B shape */
        const int q8_ffn = is_q8_type(m->gate[l].type);
        CK(g4_residual_norm(x, m->xb2, m->post_attn_norm[l], NULL, m->ffn_norm[l], m->xb2, q8_ffn ? m->q8 : NULL, 0, dim,
                            c->eps));
        CK(g4_mm_gate_up_gelu(m->hb, m->gate[l].p, m->up[l].p, dim, c->hidden, m->gate[l].type, m->q8));
        /* down (main.c:1981) */
        if ((rc = mm(m, m->xb2, m->hb, &m->down[l], 0))) return rc;
        /* post_ffw_norm + residual, Q8_K of x (main.c:1982-1988) and the
         * inp_gate GEMV with gelu * ple[l] in its epilogue (main.c:1988-1993) */
        if (pro_ok(c, &m->inp_gate[l])) {
            CK(g4_mm_residual_q8(m->ple_gate, m->inp_gate[l].p, NULL, dim, pd, m->inp_gate[l].type, m->ple + (size_t)l * pd, x,
                                 xo, m->xb2, m->post_ffw_norm[l], NULL, NULL, NULL, NULL, 1, c->eps));
            float *t = x; x = xo; xo = t;
        } else {
            const int q8_ig = is_q8_type(m->inp_gate[l].type);
            CK(g4_residual_norm(x, m->xb2, m->post_ffw_norm[l], NULL, NULL, NULL, q8_ig ? m->q8 : NULL, 1, dim, c->eps));
            if (q8_ig) {
                CK(g4_mm_quant_dot_rows_gelu_mul(m->ple_gate, m->inp_gate[l].p, dim, pd, m->inp_gate[l].type, m->q8,
                                                 m->ple + (size_t)l * pd));
            } else {
                if ((rc = mm(m, m->ple_gate, x, &m->inp_gate[l], 0))) return rc;
                CK(g4_gelu_mul_quant(m->ple_gate, m->ple + (size_t)l * pd, pd, NULL));
            }
        }
        /* proj (main.c:1994): mm() quantizes its 256-wide input inside the GEMV;
         * its residual step runs in the next layer's Q launch */
        if ((rc = mm(m, m->ybuf, m->ple_gate, &m->proj[l], 0))) return rc;
    }
    /* the last layer's post_norm + residual + out_scale and the final norm
     * (main.c:1995-2003, 2021) */
    CK(g4_residual_norm(x, m->ybuf, m->post_norm[L - 1], m->out_scale[L - 1], lm_mode ? m->norm_out : NULL,
                        lm_mode ? m->xb2 : NULL, NULL, 0, dim, c->eps));
    if (m->trace) CK(g4_memcpy_d2h(m->layer_x + (size_t)L * dim, x, (size_t)dim * 4));
    m->x_last = x;
    if (lm_mode == 0) return 0;
    /* logits_tied (main.c:1780-1796): Q6_K rows times the final-normed hidden
     * (kept in xb2), soft-cap */
    CK(g4_mm_quant_rows_softcap(m->logits, m->xb2, m->embd.p, dim, c->vocab, m->embd.type, c->softcap));
    return 0;
}

/* ---------------------------------------------------------------------------
 * Prompt chunks: the forward() of m consecutive prompt tokens with lm_mode 0
 * (main.c:2366-2384 runs them one at a time), layer by layer over all m
 * tokens: the Q4_K/Q5_K projections through the batched GEMM (bit-identical
 * per token to the decode GEMV), norms and residual steps through the rows
 * forms of the decode step's kernels (same thread layout, so the same bits
 * per row), attention over m query rows.  A sliding-window ring cannot hold
 * every query's window while the chunk's own positions are appended, so each
 * storing layer writes its chunk's K/V to a chunk buffer, the attention reads
 * positions >= p0 from there and earlier ones from the cache, and the chunk
 * is appended to the cache afterwards (for the shared-KV donors 22 and 23
 * after the last layer, when their readers are done).  Only the KV caches
 * carry over to the next token, as in the reference.
 * ------------------------------------------------------------------------- */
static int pf_alloc(g4e_model *m, int cap) {
    const Config *c = &m->c;
    const int L = c->n_layers, pd = c->ple_dim;
    const int hdmax = c->hd_full > c->hd_swa ? c->hd_full : c->hd_swa;
    const int qmax = c->n_heads * hdmax, kvmax = c->n_kv * hdmax;
    int q8n = c->hidden > qmax ? c->hidden : qmax;
    if (c->dim > q8n) q8n = c->dim;
    q8n = (q8n + 255) / 256 * 256;
    const size_t M = (size_t)cap;
    int rc;
    void *p;
    m->pf_Gmax = (c->max_seq + 1023) / 1024;
    if (m->pf_Gmax < 16) m->pf_Gmax = 16;
#define PA(field, bytes) if ((rc = dalloc(m, &p, (size_t)(bytes)))) return rc; field = p;
    PA(m->pf_tok, M * 4);
    PA(m->pf_x, M * c->dim * 4);
    PA(m->pf_xb2, M * c->dim * 4);
    PA(m->pf_q, M * qmax * 4);
    PA(m->pf_k, M * kvmax * 4);
    PA(m->pf_v, M * kvmax * 4);
    PA(m->pf_ao, M * qmax * 4);
    PA(m->pf_o, M * c->dim * 4);
    PA(m->pf_g, M * c->hidden * 4);
    PA(m->pf_u, M * c->hidden * 4);
    PA(m->pf_h, M * c->hidden * 4);
    PA(m->pf_d, M * c->dim * 4);
    PA(m->pf_ig, M * pd * 4);
    PA(m->pf_pg, M * pd * 4);
    PA(m->pf_y, M * c->dim * 4);
    PA(m->pf_ple, M * L * pd * 4);
    PA(m->pf_ctx, M * L * pd * 4);
    PA(m->pf_tab_swa, M * (size_t)(c->rot_swa / 2) * 8);
    PA(m->pf_tab_full, M * (size_t)(c->rot_full / 2) * 8);
    PA(m->pf_part, M * g4_attn_part_bytes(c->n_heads, hdmax, m->pf_Gmax));
    PA(m->pf_q8, M * g4_q8K_row_stride(q8n));
    PA(m->pf_q8a, M * g4_q8K_row_stride((qmax + 255) / 256 * 256));
    PA(m->pf_q8p, M * g4_q8K_row_stride((pd + 255) / 256 * 256));
    for (int i = 0; i < 3; i++) {
        PA(m->pf_kch[i], M * kvmax * 4);
        PA(m->pf_vch[i], M * kvmax * 4);
    }
#undef PA
    m->pf_cap = cap;
    return 0;
}

/* chunk K/V buffer of layer l (storing layers) */
static int pf_slot(int l) { return l == 22 ? 1 : l == 23 ? 2 : 0; }

/* mm over the chunk's rows: K-quant through the batched GEMM on the Q8_K rows
 * (q8_ready: already quantized by the preceding residual step), the other
 * types per token */
static int mm_rows(g4e_model *m, float *o, const float *x, const Tensor *w, int M, int q8_ready) {
    if (is_q8_type(w->type) && q8_ready) return g4_mm_batch_q8(o, w->p, m->pf_q8, w->n, w->d, M, w->type) ? lib_fail(G4_ERR_HIP, "g4_mm_batch_q8") : 0;
    return g4_mm_batch(o, x, w->p, w->n, w->d, M, w->type, m->pf_q8) ? lib_fail(G4_ERR_HIP, "g4_mm_batch") : 0;
}

/* One prompt chunk of M tokens at positions p0..p0+M-1, layer by layer.
 * trace (optional, host): each layer's input rows go to trace[(l*ntot + t0 +
 * z)*dim] and the last layer's output to l = n_layers; ntot is the whole
 * prompt's length and t0 this chunk's first row. */
static int enqueue_prefill_chunk(g4e_model *m, int p0, int M, float *trace, int ntot, int t0) {
    const Config *c = &m->c;
    const int dim = c->dim, L = c->n_layers, pd = c->ple_dim;
    int rc;
    CK(g4_emb_lookup_rows(m->pf_x, m->embd.p, m->embd.type, m->embd.d, m->pf_tok, M, dim, sqrtf((float)dim)));
    if ((rc = mm_rows(m, m->pf_ctx, m->pf_x, &m->ple_proj, M, 0))) return rc;
    CK(g4_ple_finish_rows(m->pf_ple, m->pf_ctx, m->ple_tok.p, m->ple_tok.type, m->ple_tok.d, m->ple_proj_norm,
                          m->pf_tok, M, pd, L, sqrtf((float)pd), 1.0f / sqrtf((float)dim), 1.0f / sqrtf(2.0f), c->eps));
    CK(g4_rope_table_rows(m->pf_tab_swa, p0, M, c->rot_swa, c->theta_swa, 1.0f, NULL));
    CK(g4_rope_table_rows(m->pf_tab_full, p0, M, c->rot_full, c->theta, 1.0f, m->rope_freqs));
    for (int l = 0; l < L; l++) {
        const int hd = layer_hd(c, l), swa = is_swa(c, l);
        const int n_rot = swa ? c->rot_swa : c->rot_full;
        const int src = kv_source(c, l), has_kv = layer_has_kv(l);
        const int kvd = c->n_kv * hd, kvd_src = c->n_kv * layer_hd(c, src);
        const int q8_att = is_q8_type(m->wq[l].type);
        /* residual step of the previous layer + attn_norm (+ Q8_K rows) */
        CK(g4_residual_norm_rows(m->pf_x, l ? m->pf_y : NULL, l ? m->post_norm[l - 1] : NULL,
                                 l ? m->out_scale[l - 1] : NULL, m->attn_norm[l], m->pf_xb2, q8_att ? m->pf_q8 : NULL, 0,
                                 dim, c->eps, M, pro_ok(c, &m->wq[l])));
        if (trace) CK(g4_memcpy_d2h(trace + ((size_t)l * ntot + t0) * dim, m->pf_x, (size_t)M * dim * 4));
        if ((rc = mm_rows(m, m->pf_q, m->pf_xb2, &m->wq[l], M, q8_att))) return rc;
        float *kch = NULL, *vch = NULL;
        if (has_kv) {
            const int q8k = is_q8_type(m->wk[l].type) && q8_att, q8v = is_q8_type(m->wv[l].type) && q8_att;
            if ((rc = mm_rows(m, m->pf_k, m->pf_xb2, &m->wk[l], M, q8k))) return rc;
            if ((rc = mm_rows(m, m->pf_v, m->pf_xb2, &m->wv[l], M, q8v))) return rc;
            kch = m->pf_kch[pf_slot(l)];
            vch = m->pf_vch[pf_slot(l)];
        }
        CK(g4_qkv_post_rows(m->pf_q, m->q_norm[l], has_kv ? m->pf_k : NULL, has_kv ? m->pf_v : NULL,
                            has_kv ? m->k_norm[l] : NULL, kch, vch, kvd, swa ? m->pf_tab_swa : m->pf_tab_full, M,
                            c->n_heads, c->n_kv, hd, n_rot, c->eps));
        /* attention over the query rows; chunks of <= 128 positions */
        const int window = swa ? c->window : 0;
        const int nmax = window > 0 && window < p0 + M ? window : p0 + M;
        int G = (nmax + 127) / 128;
        if (G > m->pf_Gmax) G = m->pf_Gmax;
        const int o_q8 = is_q8_type(m->wo[l].type);
        CK(g4_attn_decode_rows(m->pf_q, m->kc[src], m->vc[src], m->pf_kch[pf_slot(src)], m->pf_vch[pf_slot(src)],
                               kvd_src, m->kv_ring[src], p0, M, window, c->n_heads, c->n_kv, hd, 1.0f, G, m->pf_part,
                               m->pf_ao, o_q8 ? m->pf_q8a : NULL));
        if (has_kv && pf_slot(l) == 0) CK(g4_kv_store_rows(m->kc[l], m->vc[l], kch, vch, kvd, m->kv_ring[l], p0, M, kvd));
        if (o_q8) {
            CK(g4_mm_batch_q8(m->pf_o, m->wo[l].p, m->pf_q8a, m->wo[l].n, m->wo[l].d, M, m->wo[l].type));
        } else if ((rc = mm_rows(m, m->pf_o, m->pf_ao, &m->wo[l], M, 0))) {
            return rc;
        }
        /* post_attention_norm + residual, ffn_norm + Q8_K rows; gelu(gate) * up; down */
        const int q8_ffn = is_q8_type(m->gate[l].type);
        CK(g4_residual_norm_rows(m->pf_x, m->pf_o, m->post_attn_norm[l], NULL, m->ffn_norm[l], m->pf_xb2,
                                 q8_ffn ? m->pf_q8 : NULL, 0, dim, c->eps, M, 0));
        if ((rc = mm_rows(m, m->pf_g, m->pf_xb2, &m->gate[l], M, q8_ffn))) return rc;
        if ((rc = mm_rows(m, m->pf_u, m->pf_xb2, &m->up[l], M, q8_ffn && is_q8_type(m->up[l].type)))) return rc;
        CK(g4_gelu_mul_rows(m->pf_h, m->pf_g, m->pf_u, c->hidden, M, c->hidden));
        if ((rc = mm_rows(m, m->pf_d, m->pf_h, &m->down[l], M, 0))) return rc;
        /* post_ffw_norm + residual, Q8_K rows of x; PLE gate and projection */
        const int q8_ig = is_q8_type(m->inp_gate[l].type);
        CK(g4_residual_norm_rows(m->pf_x, m->pf_d, m->post_ffw_norm[l], NULL, NULL, NULL, q8_ig ? m->pf_q8 : NULL, 1,
                                 dim, c->eps, M, pro_ok(c, &m->inp_gate[l])));
        if ((rc = mm_rows(m, m->pf_ig, m->pf_x, &m->inp_gate[l], M, q8_ig))) return rc;
        CK(g4_gelu_mul_rows(m->pf_pg, m->pf_ig, m->pf_ple + (size_t)l * pd, pd, M, L * pd));
        if (is_q8_type(m->proj[l].type)) {
            CK(g4_quantize_rows_q8_K(m->pf_pg, m->pf_q8p, pd, M));
            CK(g4_mm_batch_q8(m->pf_y, m->proj[l].p, m->pf_q8p, pd, dim, M, m->proj[l].type));
        } else if ((rc = mm_rows(m, m->pf_y, m->pf_pg, &m->proj[l], M, 0))) {
            return rc;
        }
    }
    if (trace) {
        CK(g4_residual_norm_rows(m->pf_x, m->pf_y, m->post_norm[L - 1], m->out_scale[L - 1], NULL, NULL, NULL, 0, dim,
                                 c->eps, M, 0));
        CK(g4_memcpy_d2h(trace + ((size_t)L * ntot + t0) * dim, m->pf_x, (size_t)M * dim * 4));
    }
    /* the shared-KV donors' chunks, now that their readers are done */
    for (int l = 22; l <= 23 && l < L; l++)
        if (layer_has_kv(l)) {
            const int kvd = c->n_kv * layer_hd(c, l);
            CK(g4_kv_store_rows(m->kc[l], m->vc[l], m->pf_kch[pf_slot(l)], m->pf_vch[pf_slot(l)], kvd, m->kv_ring[l],
                                p0, M, kvd));
        }
    return 0;
}

int g4e_prefill_trace(g4e_model *m, const int *tokens, int n, int pos0, float *trace) {
    if (!m || !tokens || n < 0 || pos0 < 0) return fail(G4_ERR_ARG, "g4e_prefill: bad arguments");
    if (pos0 + n > m->c.max_seq) return fail(G4_ERR_ARG, "g4e_prefill: positions past max_seq");
    g4_set_stream(m->stream);
    int rc;
    /* chunk buffers: sized by the first call, up to 512 tokens; longer
     * prompts run in chunks of that size */
    const int want = m->pf_chunk > 0 ? m->pf_chunk : G4E_PREFILL_CHUNK;
    if (m->pf_cap == 0 && n > 0 && (rc = pf_alloc(m, want < m->c.max_seq ? want : m->c.max_seq))) return rc;
    const int chunk = want < m->pf_cap ? want : m->pf_cap;
    for (int t0 = 0; t0 < n; t0 += chunk) {
        const int M = n - t0 < chunk ? n - t0 : chunk;
        CK(g4_memcpy_h2d(m->pf_tok, tokens + t0, (size_t)M * 4));
        if ((rc = enqueue_prefill_chunk(m, pos0 + t0, M, trace, n, t0))) return rc;
    }
    CK(g4_sync());
    return 0;
}

int g4e_prefill(g4e_model *m, const int *tokens, int n, int pos0) { return g4e_prefill_trace(m, tokens, n, pos0, NULL); }

int g4e_kv_info(const g4e_model *m, int layer, int out[2]) {
    if (!m || !out || layer < 0 || layer >= m->c.n_layers || !layer_has_kv(layer))
        return fail(G4_ERR_ARG, "g4e_kv_info: layer %d stores no KV", layer);
    const int ring = m->kv_ring[layer];
    out[0] = m->c.n_kv * layer_hd(&m->c, layer);
    out[1] = ring > 0 ? ring : m->c.max_seq;
    return 0;
}

int g4e_read_kv(g4e_model *m, int layer, int slot0, int nslots, float *k, float *v) {
    int info[2], rc;
    if ((rc = g4e_kv_info(m, layer, info))) return rc;
    if (slot0 < 0 || nslots < 0 || slot0 + nslots > info[1] || !k || !v) return fail(G4_ERR_ARG, "g4e_read_kv: bad range");
    g4_set_stream(m->stream);
    CK(g4_sync());
    CK(g4_memcpy_d2h(k, m->kc[layer] + (size_t)slot0 * info[0], (size_t)nslots * info[0] * 4));
    CK(g4_memcpy_d2h(v, m->vc[layer] + (size_t)slot0 * info[0], (size_t)nslots * info[0] * 4));
    return 0;
}

int g4e_set_prefill_chunk(g4e_model *m, int tokens) {
    if (!m || tokens < 0 || tokens > G4E_PREFILL_CHUNK)
        return fail(G4_ERR_ARG, "g4e_set_prefill_chunk: %d tokens (0..%d)", tokens, G4E_PREFILL_CHUNK);
    if (m->pf_cap > 0 && tokens > m->pf_cap)
        return fail(G4_ERR_STATE, "g4e_set_prefill_chunk: chunk buffers hold %d tokens", m->pf_cap);
    m->pf_chunk = tokens;
    return 0;
}

static int set_step(g4e_model *m, int token, int pos) {
    const Config *c = &m->c;
    if (token < 0 || token >= c->vocab) return fail(G4_ERR_ARG, "token %d out of range", token);
    if (pos < 0 || pos >= c->max_seq) return fail(G4_ERR_ARG, "pos %d out of range (max_seq %d)", pos, c->max_seq);
    CK(g4_store_i32x2(m->dstep, token, pos));
    return 0;
}

int g4e_forward(g4e_model *m, int token, int pos, int lm_mode) {
    if (!m) return fail(G4_ERR_ARG, "null model");
    g4_set_stream(m->stream);
    int rc = set_step(m, token, pos);
    if (rc) return rc;
    rc = enqueue_step(m, lm_mode);
    if (rc) return rc;
    CK(g4_sync());
    return 0;
}

int g4e_read_logits(g4e_model *m, float *host) {
    g4_set_stream(m->stream);
    CK(g4_memcpy_d2h(host, m->logits, (size_t)m->c.vocab * 4));
    return 0;
}

int g4e_read_x(g4e_model *m, float *host) {
    g4_set_stream(m->stream);
    CK(g4_memcpy_d2h(host, m->x_last, (size_t)m->c.dim * 4));
    return 0;
}

int g4e_argmax(g4e_model *m, int *tok) {
    g4_set_stream(m->stream);
    CK(g4_argmax(m->logits, m->c.vocab, m->dstep + 2, m->argmax_part, NULL, NULL));
    CK(g4_memcpy_d2h(tok, m->dstep + 2, 4));
    return 0;
}

int g4e_set_trace(g4e_model *m, int on) {
    if (on && !m->layer_x) {
        m->layer_x = (float *)calloc((size_t)(m->c.n_layers + 1) * m->c.dim, sizeof(float));
        if (!m->layer_x) return fail(G4_ERR_NOMEM, "out of host memory");
    }
    m->trace = on;
    return 0;
}

const float *g4e_layer_x(const g4e_model *m) { return m->layer_x; }

/* One greedy decode step as launches: forward with logits, then argmax,
 * which also stores the token as the next input and advances the position. */
static int enqueue_greedy_step(g4e_model *m) {
    int rc = enqueue_step(m, 1);
    if (rc) return rc;
    CK(g4_argmax(m->logits, m->c.vocab, m->dstep + 2, m->argmax_part, m->dstep, m->dstep + 1));
    return 0;
}

static int ensure_graph(g4e_model *m) {
    if (m->graph) return 0;
    if (m->trace) return fail(G4_ERR_STATE, "graph capture with trace on");
    CK(g4_graph_begin());
    int rc = enqueue_greedy_step(m);
    void *g = NULL;
    const int rc2 = g4_graph_end(&g);
    if (rc) return rc;
    if (rc2) return lib_fail(rc2, "g4_graph_end");
    m->graph = g;
    return 0;
}

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + (double)t.tv_nsec * 1e-9;
}

int g4e_decode_steps(g4e_model *m, int token, int pos0, int steps, int use_graph, int *out, double *sec) {
    if (!m || steps < 0) return fail(G4_ERR_ARG, "g4e_decode_steps: bad arguments");
    if (pos0 + steps > m->c.max_seq) return fail(G4_ERR_ARG, "decode past max_seq");
    g4_set_stream(m->stream);
    int rc = set_step(m, token, pos0);
    if (rc) return rc;
    if (use_graph && (rc = ensure_graph(m))) return rc;
    CK(g4_sync());
    const double t0 = now_s();
    for (int s = 0; s < steps; s++) {
        if (use_graph) CK(g4_graph_launch(m->graph));
        else if ((rc = enqueue_greedy_step(m))) return rc;
        if (out) {
            CK(g4_memcpy_d2h_async(&m->hstep[2], m->dstep + 2, 4));
            CK(g4_sync());
            out[s] = m->hstep[2];
        }
    }
    CK(g4_sync());
    if (sec) *sec = now_s() - t0;
    return 0;
}

int g4e_generate_greedy(g4e_model *m, const int *prompt, int n_prompt, int max_new, int *out_tokens,
                        double *prefill_sec, double *decode_sec, int use_graph) {
    if (!m || !prompt || n_prompt <= 0 || max_new < 0) return -fail(G4_ERR_ARG, "g4e_generate_greedy: bad arguments");
    g4_set_stream(m->stream);
    const double t0 = now_s();
    int gen = 0, rc;
    /* prefill: lm_mode 0 except for the last prompt token (main.c:2366-2384),
     * in prompt chunks or token by token */
    if (m->pf_chunk > 0) {
        const int np = n_prompt - 1 < m->c.max_seq ? n_prompt - 1 : m->c.max_seq;
        if (np > 0 && (rc = g4e_prefill(m, prompt, np, 0))) return -rc;
    } else {
        for (int pos = 0; pos < n_prompt - 1; pos++) {
            if (pos >= m->c.max_seq) return gen;
            if ((rc = set_step(m, prompt[pos], pos)) || (rc = enqueue_step(m, 0))) return -rc;
        }
    }
    const int last = n_prompt - 1;
    if (last >= m->c.max_seq) return gen;
    if ((rc = set_step(m, prompt[last], last))) return -rc;
    if (use_graph && (rc = ensure_graph(m))) return -rc;
    if (g4_sync()) return -lib_fail(G4_ERR_HIP, "g4_sync");
    const double t1 = now_s();
    if (prefill_sec) *prefill_sec = t1 - t0;
    /* decode: each step computes the logits of the current token and its argmax
     * becomes the next input (main.c:2426-2435) */
    for (int pos = last; pos < n_prompt + max_new - 1 && pos < m->c.max_seq; pos++) {
        if (use_graph) rc = g4_graph_launch(m->graph) ? lib_fail(G4_ERR_HIP, "g4_graph_launch") : 0;
        else rc = enqueue_greedy_step(m);
        if (rc) return -rc;
        if (g4_memcpy_d2h_async(&m->hstep[2], m->dstep + 2, 4) || g4_sync()) return -lib_fail(G4_ERR_HIP, "readback");
        const int next = m->hstep[2];
        if (next == m->c.eos) break;
        out_tokens[gen++] = next;
    }
    if (decode_sec) *decode_sec = now_s() - t1;
    return gen;
}
