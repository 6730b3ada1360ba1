/*
 * text.c -- host text path (see text.h).  Vocabulary lookups go through an
 * open-addressing table keyed by the piece bytes; BPE keeps the score of
 * every adjacent pair and recomputes only the two pairs a merge touches, so
 * a line of n characters costs O(n^2) instead of a fresh lookup of every
 * pair after each merge, with the same result: the highest-scoring pair,
 * leftmost among equals, merged until no pair forms a token
 * (bpe_merge, main.c:1084-1110).
 */
#define _POSIX_C_SOURCE 200809L
#include "text.h"

#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define SP "\xe2\x96\x81"          /* U+2581, the escaped space (main.c:78) */
#define PAIR_MAX 65536             /* pairs this long or longer never merge (main.c:1085) */

static char g_err[256];
const char *g4t_last_error(void) { return g_err; }
static int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

struct g4t_vocab {
    int n;
    char **piece;
    int *len;
    float *score;
    int *slot;                    /* hash table of ids, -1 empty; capacity mask + 1 */
    uint32_t mask;
    int sp[13];                   /* g4t_specials order */
};

enum { S_BOS, S_EOS, S_EOT, S_PREFIX, S_TURN_START, S_TURN_END, S_TURN_USER, S_TURN_MODEL, S_TURN_SYSTEM, S_THINK,
       S_CHANNEL, S_CHANNEL_THOUGHT, S_CHANNEL_END };

static uint32_t hash(const char *s, int n) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (int i = 0; i < n; i++) h = (h ^ (uint8_t)s[i]) * 0x100000001b3ull;
    return (uint32_t)(h ^ (h >> 29));
}

int g4t_lookup(const g4t_vocab *v, const char *s, int len) {
    if (!v || len < 0) return -1;
    for (uint32_t h = hash(s, len) & v->mask;; h = (h + 1) & v->mask) {
        const int id = v->slot[h];
        if (id < 0) return -1;
        if (v->len[id] == len && !memcmp(v->piece[id], s, (size_t)len)) return id;
    }
}

/* tok_find_special (main.c:1002-1008): the highest id whose piece is name */
static int find_special(const g4t_vocab *v, const char *name) {
    const int n = (int)strlen(name);
    for (int i = v->n - 1; i >= 0; i--)
        if (v->len[i] == n && !memcmp(v->piece[i], name, (size_t)n)) return i;
    return -1;
}

/* ---- GGUF metadata (main.c:841-966) -------------------------------------- */
enum { GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };
typedef struct { const uint8_t *d; uint64_t p, n; int bad; } Rd;

static int need(Rd *r, uint64_t k) {
    if (r->bad || k > r->n - r->p) { r->bad = 1; return 0; }
    return 1;
}
static uint64_t rdu(Rd *r, int bytes) {
    uint64_t v = 0;
    if (!need(r, (uint64_t)bytes)) return 0;
    memcpy(&v, r->d + r->p, (size_t)bytes);
    r->p += (uint64_t)bytes;
    return v;
}
static const char *rdstr(Rd *r, uint64_t *len) {
    *len = rdu(r, 8);
    if (!need(r, *len)) return NULL;
    const char *s = (const char *)r->d + r->p;
    r->p += *len;
    return s;
}
static const int elem_bytes[13] = {1, 1, 2, 2, 4, 4, 4, 1, -1, -1, 8, 8, 8};
static void skip(Rd *r, uint32_t t, int depth) {
    if (t > GV_F64 || depth > 2) { r->bad = 1; return; }
    if (t == GV_STR) { uint64_t l; rdstr(r, &l); return; }
    if (t == GV_ARR) {
        const uint32_t et = (uint32_t)rdu(r, 4);
        const uint64_t n = rdu(r, 8);
        if (et <= GV_F64 && elem_bytes[et] > 0) {
            if (n > (r->n - r->p) / (uint64_t)elem_bytes[et]) { r->bad = 1; return; }
            r->p += n * (uint64_t)elem_bytes[et];
        } else {
            for (uint64_t i = 0; i < n && !r->bad; i++) skip(r, et, depth + 1);
        }
        return;
    }
    need(r, (uint64_t)elem_bytes[t]);
    if (!r->bad) r->p += (uint64_t)elem_bytes[t];
}
/* read_int_val (main.c:813-826) */
static int64_t rdint(Rd *r, uint32_t t) {
    switch (t) {
    case GV_U8: case GV_BOOL: return (int64_t)(uint8_t)rdu(r, 1);
    case GV_I8: return (int64_t)(int8_t)rdu(r, 1);
    case GV_U16: return (int64_t)(uint16_t)rdu(r, 2);
    case GV_I16: return (int64_t)(int16_t)rdu(r, 2);
    case GV_U32: return (int64_t)(uint32_t)rdu(r, 4);
    case GV_I32: return (int64_t)(int32_t)rdu(r, 4);
    case GV_U64: return (int64_t)rdu(r, 8);
    case GV_I64: return (int64_t)rdu(r, 8);
    case GV_F32: { uint32_t u = (uint32_t)rdu(r, 4); float f; memcpy(&f, &u, 4); return (int64_t)f; }
    case GV_F64: { uint64_t u = rdu(r, 8); double f; memcpy(&f, &u, 8); return (int64_t)f; }
    default: skip(r, t, 0); return 0;
    }
}
static int key_is(const char *k, uint64_t kl, const char *s) { return kl == strlen(s) && !memcmp(k, s, kl); }

void g4t_close(g4t_vocab *v) {
    if (!v) return;
    if (v->piece)
        for (int i = 0; i < v->n; i++) free(v->piece[i]);
    free(v->piece);
    free(v->len);
    free(v->score);
    free(v->slot);
    free(v);
}

int g4t_open_image(const void *data, size_t size, g4t_vocab **out) {
    if (!data || !out) return fail(G4T_ERR_ARG, "g4t_open_image: null pointer");
    *out = NULL;
    Rd r = {(const uint8_t *)data, 0, size, 0};
    if (rdu(&r, 4) != 0x46554747u) return fail(G4T_ERR_FORMAT, "invalid GGUF magic");
    rdu(&r, 4);
    rdu(&r, 8);
    const uint64_t n_kv = rdu(&r, 8);
    g4t_vocab *v = (g4t_vocab *)calloc(1, sizeof *v);
    if (!v) return fail(G4T_ERR_NOMEM, "out of host memory");
    int bos = 2, eos = 106, prefix = 1;           /* defaults, main.c:868-871 */
    const float *scores = NULL;                   /* into the image */
    uint64_t n_scores = 0;
    Rd merges = {0};
    uint64_t n_merges = 0;
    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        uint64_t kl;
        const char *k = rdstr(&r, &kl);
        const uint32_t t = (uint32_t)rdu(&r, 4);
        if (r.bad) break;
        if (key_is(k, kl, "tokenizer.ggml.bos_token_id")) bos = (int)rdint(&r, t);
        else if (key_is(k, kl, "tokenizer.ggml.eos_token_id")) eos = (int)rdint(&r, t);
        else if (key_is(k, kl, "tokenizer.ggml.add_space_prefix")) prefix = (int)rdint(&r, t);
        else if (key_is(k, kl, "tokenizer.ggml.tokens") && t == GV_ARR) {
            rdu(&r, 4);
            const uint64_t n = rdu(&r, 8);
            if (n > (r.n - r.p) / 8 || n > (1u << 28)) { r.bad = 1; break; }
            v->n = (int)n;
            v->piece = (char **)calloc(n ? n : 1, sizeof(char *));
            v->len = (int *)calloc(n ? n : 1, sizeof(int));
            if (!v->piece || !v->len) { g4t_close(v); return fail(G4T_ERR_NOMEM, "out of host memory"); }
            for (uint64_t j = 0; j < n && !r.bad; j++) {
                uint64_t l;
                const char *s = rdstr(&r, &l);
                if (r.bad || l > (1u << 20)) { r.bad = 1; break; }
                v->piece[j] = (char *)malloc(l + 1);
                if (!v->piece[j]) { g4t_close(v); return fail(G4T_ERR_NOMEM, "out of host memory"); }
                memcpy(v->piece[j], s, l);
                v->piece[j][l] = 0;
                v->len[j] = (int)l;
            }
        } else if (key_is(k, kl, "tokenizer.ggml.scores") && t == GV_ARR) {
            const uint32_t et = (uint32_t)rdu(&r, 4);
            const uint64_t n = rdu(&r, 8);
            /* n is the file's 64-bit count: bound it before n * 4 can wrap */
            if (et == GV_F32 && !r.bad && n <= (r.n - r.p) / 4 && need(&r, n * 4)) {
                scores = (const float *)(r.d + r.p);
                n_scores = n;
                r.p += n * 4;
            } else {
                r.p -= 12;
                skip(&r, t, 0);
            }
        } else if (key_is(k, kl, "tokenizer.ggml.merges") && t == GV_ARR) {
            rdu(&r, 4);
            n_merges = rdu(&r, 8);
            merges = r;                           /* walked again once the vocabulary is known */
            for (uint64_t j = 0; j < n_merges && !r.bad; j++) { uint64_t l; rdstr(&r, &l); }
        } else {
            skip(&r, t, 0);
        }
    }
    if (r.bad) { g4t_close(v); return fail(G4T_ERR_FORMAT, "truncated or malformed GGUF metadata"); }
    if (v->n <= 0) { g4t_close(v); return fail(G4T_ERR_FORMAT, "GGUF has no tokenizer.ggml.tokens"); }
    v->score = (float *)calloc((size_t)v->n, sizeof(float));
    uint32_t cap = 16;
    while (cap < 2u * (uint32_t)v->n) cap <<= 1;
    v->slot = (int *)malloc(cap * sizeof(int));
    if (!v->score || !v->slot) { g4t_close(v); return fail(G4T_ERR_NOMEM, "out of host memory"); }
    v->mask = cap - 1;
    for (uint32_t i = 0; i < cap; i++) v->slot[i] = -1;
    for (int id = 0; id < v->n; id++) {
        if (g4t_lookup(v, v->piece[id], v->len[id]) >= 0) continue;     /* duplicates: the lowest id */
        uint32_t h = hash(v->piece[id], v->len[id]) & v->mask;
        while (v->slot[h] >= 0) h = (h + 1) & v->mask;
        v->slot[h] = id;
    }
    for (uint64_t i = 0; i < n_scores && i < (uint64_t)v->n; i++) memcpy(&v->score[i], &scores[i], 4);
    /* init_tokenizer (main.c:1010-1031): merge i ("a b") scores token a+b
     * with n_merges - i */
    for (uint64_t i = 0; i < n_merges; i++) {
        uint64_t l;
        const char *s = rdstr(&merges, &l);
        const char *sp = memchr(s, ' ', l);
        const char *nul = memchr(s, 0, l);      /* the reference sees C strings */
        if (nul) l = (uint64_t)(nul - s);
        if (!sp || sp >= s + l) continue;
        const size_t la = (size_t)(sp - s), lb = (size_t)(s + l - sp - 1);
        char *buf = (char *)malloc(la + lb + 1);
        if (!buf) { g4t_close(v); return fail(G4T_ERR_NOMEM, "out of host memory"); }
        memcpy(buf, s, la);
        memcpy(buf + la, sp + 1, lb);
        const int id = g4t_lookup(v, buf, (int)(la + lb));
        if (id >= 0) v->score[id] = (float)(n_merges - i);
        free(buf);
    }
    v->sp[S_BOS] = bos;
    v->sp[S_EOS] = eos;
    v->sp[S_EOT] = eos;
    v->sp[S_PREFIX] = prefix;
    v->sp[S_TURN_START] = find_special(v, "<|turn>");
    v->sp[S_TURN_END] = find_special(v, "<turn|>");
    v->sp[S_TURN_USER] = find_special(v, "<|turn>user\n");
    v->sp[S_TURN_MODEL] = find_special(v, "<|turn>model\n");
    v->sp[S_TURN_SYSTEM] = find_special(v, "<|turn>system\n");
    v->sp[S_THINK] = find_special(v, "<|think|>");
    v->sp[S_CHANNEL] = find_special(v, "<|channel>");
    v->sp[S_CHANNEL_THOUGHT] = find_special(v, "<|channel>thought\n");
    if (v->sp[S_CHANNEL_THOUGHT] < 0) v->sp[S_CHANNEL_THOUGHT] = find_special(v, "<|channel>thought");
    v->sp[S_CHANNEL_END] = find_special(v, "<channel|>");
    *out = v;
    return 0;
}

int g4t_open_file(const char *path, g4t_vocab **out) {
    if (!path || !out) return fail(G4T_ERR_ARG, "g4t_open_file: null pointer");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(G4T_ERR_ARG, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return fail(G4T_ERR_ARG, "cannot stat %s", path); }
    void *p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return fail(G4T_ERR_NOMEM, "mmap failed");
    const int rc = g4t_open_image(p, (size_t)st.st_size, out);
    munmap(p, (size_t)st.st_size);
    return rc;
}

int g4t_size(const g4t_vocab *v) { return v ? v->n : 0; }
void g4t_specials(const g4t_vocab *v, int out[13]) { memcpy(out, v->sp, sizeof v->sp); }
float g4t_score(const g4t_vocab *v, int id) { return id >= 0 && id < v->n ? v->score[id] : 0.0f; }
const char *g4t_piece(const g4t_vocab *v, int id, int *len) {
    if (id < 0 || id >= v->n) { if (len) *len = 0; return NULL; }
    if (len) *len = v->len[id];
    return v->piece[id];
}

/* ---- encoding ------------------------------------------------------------- */
typedef struct { int *t; int n, cap, full; } Out;
static void push(Out *o, int id) {
    if (o->n >= o->cap) { o->full = 1; return; }
    o->t[o->n++] = id;
}

/* utf8_char_len (main.c:1047-1053) */
static int u8len(unsigned char c) {
    if ((c & 0x80) == 0) return 1;
    if ((c & 0xE0) == 0xC0) return 2;
    if ((c & 0xF0) == 0xE0) return 3;
    if ((c & 0xF8) == 0xF0) return 4;
    return 1;
}

/* the token of pieces a and b joined, or -1 */
static int pair_id(const g4t_vocab *v, int a, int b, char **buf, size_t *cap) {
    const size_t la = (size_t)v->len[a], lb = (size_t)v->len[b];
    if (la + lb >= PAIR_MAX) return -1;
    if (la + lb > *cap) {
        char *nb = (char *)realloc(*buf, la + lb);
        if (!nb) return -1;
        *buf = nb;
        *cap = la + lb;
    }
    memcpy(*buf, v->piece[a], la);
    memcpy(*buf + la, v->piece[b], lb);
    return g4t_lookup(v, *buf, (int)(la + lb));
}

/* gemma_bpe_encode + bpe_merge (main.c:1084-1133) */
static int bpe(const g4t_vocab *v, const char *s, int len, Out *o) {
    int *t = (int *)malloc(((size_t)len + 1) * sizeof(int));
    int *pid = (int *)malloc(((size_t)len + 1) * sizeof(int));
    if (!t || !pid) { free(t); free(pid); return fail(G4T_ERR_NOMEM, "out of host memory"); }
    int n = 0;
    for (int i = 0; i < len;) {
        int cl = u8len((unsigned char)s[i]);
        if (i + cl > len) cl = len - i;
        const int id = g4t_lookup(v, s + i, cl);
        if (id < 0) fprintf(stderr, "Warning: unknown token bytes at offset %d\n", i);
        else t[n++] = id;
        i += cl;
    }
    char *buf = NULL;
    size_t bcap = 0;
    for (int i = 0; i + 1 < n; i++) pid[i] = pair_id(v, t[i], t[i + 1], &buf, &bcap);
    while (n > 1) {
        float best = -1e20f;
        int bi = -1;
        for (int i = 0; i + 1 < n; i++)
            if (pid[i] >= 0 && v->score[pid[i]] > best) { best = v->score[pid[i]]; bi = i; }
        if (bi < 0) break;
        t[bi] = pid[bi];
        memmove(t + bi + 1, t + bi + 2, (size_t)(n - bi - 2) * sizeof(int));
        memmove(pid + bi, pid + bi + 1, (size_t)(n - bi - 2) * sizeof(int));
        n--;
        if (bi > 0) pid[bi - 1] = pair_id(v, t[bi - 1], t[bi], &buf, &bcap);
        if (bi + 1 < n) pid[bi] = pair_id(v, t[bi], t[bi + 1], &buf, &bcap);
    }
    for (int i = 0; i < n; i++) push(o, t[i]);
    free(buf);
    free(t);
    free(pid);
    return 0;
}

int g4t_encode_raw(const g4t_vocab *v, const char *bytes, int len, int *out, int cap) {
    if (!v || (!bytes && len) || len < 0 || !out || cap < 0) return fail(G4T_ERR_ARG, "g4t_encode_raw: bad arguments");
    Out o = {out, 0, cap, 0};
    const int rc = bpe(v, bytes, len, &o);
    if (rc) return rc;
    return o.full ? fail(G4T_ERR_FULL, "more than %d tokens", cap) : o.n;
}

/* append_str_tok (main.c:1139-1162) */
static int str_tok(const g4t_vocab *v, const char *s, Out *o) {
    const int sid = find_special(v, s);
    if (sid >= 0) { push(o, sid); return 0; }
    const int n = (int)strlen(s);
    int all_nl = n > 0;
    for (int i = 0; i < n && all_nl; i++) all_nl = s[i] == '\n';
    if (all_nl) {
        const int id = g4t_lookup(v, s, n);
        if (id >= 0) { push(o, id); return 0; }
    }
    return bpe(v, s, n, o);
}

/* one line: gemma_escape_line (main.c:1055-1082) then BPE */
static int line(const g4t_vocab *v, const char *s, int n, Out *o) {
    char *e = (char *)malloc((size_t)n * 4 + 4);
    if (!e) return fail(G4T_ERR_NOMEM, "out of host memory");
    int k = 0;
    if (v->sp[S_PREFIX] && n > 0) { memcpy(e, SP, 3); k = 3; }
    for (int i = 0; i < n;) {
        if (s[i] == ' ') {
            memcpy(e + k, SP, 3);
            k += 3;
            i++;
        } else {
            int cl = u8len((unsigned char)s[i]);
            if (i + cl > n) cl = n - i;
            memcpy(e + k, s + i, (size_t)cl);
            k += cl;
            i += cl;
        }
    }
    const int rc = bpe(v, e, k, o);
    free(e);
    return rc;
}

/* append_gemma_text (main.c:1164-1196) */
static int gemma_text(const g4t_vocab *v, const char *text, Out *o) {
    const char *p = text, *ln = text;
    int rc;
    for (; *p; p++) {
        if (*p != '\n') continue;
        if (p > ln && (rc = line(v, ln, (int)(p - ln), o))) return rc;
        if ((rc = str_tok(v, "\n", o))) return rc;
        ln = p + 1;
    }
    if (p > ln && (rc = line(v, ln, (int)(p - ln), o))) return rc;
    return 0;
}

int g4t_encode_text(const g4t_vocab *v, const char *text, int *out, int cap) {
    if (!v || !text || !out || cap < 0) return fail(G4T_ERR_ARG, "g4t_encode_text: bad arguments");
    Out o = {out, 0, cap, 0};
    const int rc = gemma_text(v, text, &o);
    if (rc) return rc;
    return o.full ? fail(G4T_ERR_FULL, "more than %d tokens", cap) : o.n;
}

/* append_turn_end / append_turn_role (main.c:1198-1221) */
static int turn_end(const g4t_vocab *v, Out *o) {
    if (v->sp[S_TURN_END] >= 0) {
        push(o, v->sp[S_TURN_END]);
        return str_tok(v, "\n", o);
    }
    return str_tok(v, "<turn|>\n", o);
}
static int turn_role(const g4t_vocab *v, int combined, const char *role, Out *o) {
    int rc;
    if (combined >= 0) { push(o, combined); return 0; }
    if (v->sp[S_TURN_START] >= 0) push(o, v->sp[S_TURN_START]);
    else if ((rc = str_tok(v, "<|turn>", o))) return rc;
    if ((rc = str_tok(v, role, o))) return rc;
    return str_tok(v, "\n", o);
}

int g4t_chat_encode(const g4t_vocab *v, const char *const *texts, const int *roles, int n_msgs, int thinking,
                    int *out, int cap) {
    if (!v || n_msgs < 0 || (n_msgs && (!texts || !roles)) || !out || cap < 0)
        return fail(G4T_ERR_ARG, "g4t_chat_encode: bad arguments");
    Out o = {out, 0, cap, 0};
    int rc;
#define FULL_AFTER_TURN() if (o.full || o.n >= cap) return fail(G4T_ERR_FULL, "prompt too long (max %d tokens)", cap)
    if (cap <= 0) return fail(G4T_ERR_FULL, "prompt too long (max %d tokens)", cap);
    push(&o, v->sp[S_BOS]);
    if (thinking) {            /* append_system_think_turn (main.c:1233-1243) */
        if ((rc = turn_role(v, v->sp[S_TURN_SYSTEM], "system", &o))) return rc;
        if (v->sp[S_THINK] >= 0) push(&o, v->sp[S_THINK]);
        else if ((rc = str_tok(v, "<|think|>", &o))) return rc;
        if ((rc = str_tok(v, "\n", &o)) || (rc = turn_end(v, &o))) return rc;
        FULL_AFTER_TURN();
    }
    for (int i = 0; i < n_msgs; i++) {
        if (!texts[i]) return fail(G4T_ERR_ARG, "g4t_chat_encode: message %d is null", i);
        const int model = roles[i] != 0;
        if ((rc = turn_role(v, model ? v->sp[S_TURN_MODEL] : v->sp[S_TURN_USER], model ? "model" : "user", &o)) ||
            (rc = gemma_text(v, texts[i], &o)) || (rc = turn_end(v, &o)))
            return rc;
        FULL_AFTER_TURN();
    }
    if ((rc = turn_role(v, v->sp[S_TURN_MODEL], "model", &o))) return rc;
    FULL_AFTER_TURN();
#undef FULL_AFTER_TURN
    return o.n;
}

/* ---- decoding --------------------------------------------------------------- */
int g4t_is_special(const g4t_vocab *v, int id) {
    static const int which[12] = {S_BOS, S_EOS, S_EOT, S_TURN_START, S_TURN_END, S_TURN_USER, S_TURN_MODEL,
                                  S_TURN_SYSTEM, S_THINK, S_CHANNEL, S_CHANNEL_THOUGHT, S_CHANNEL_END};
    for (int i = 0; i < 12; i++)
        if (id == v->sp[which[i]]) return 1;
    return 0;
}

/* a token's printable text: empty for specials and ids out of range, U+2581
 * as a space (print_tok, main.c:2216-2231) */
static size_t piece_text(const g4t_vocab *v, int id, char *dst, size_t room) {
    if (id < 0 || id >= v->n || g4t_is_special(v, id)) return 0;
    const char *s = v->piece[id];
    const int n = v->len[id];
    size_t k = 0;
    for (int j = 0; j < n;) {
        char c;
        if (j + 3 <= n && !memcmp(s + j, SP, 3)) { c = ' '; j += 3; }
        else c = s[j++];
        if (k < room) dst[k] = c;
        k++;
    }
    return k;
}

int g4t_decode(const g4t_vocab *v, const int *tokens, int start, int end, char *out, size_t cap) {
    if (!v || !out || cap == 0 || start < 0 || (end > start && !tokens)) return fail(G4T_ERR_ARG, "g4t_decode: bad arguments");
    size_t k = 0;
    for (int i = start; i < end; i++) {
        const size_t room = k < cap - 1 ? cap - 1 - k : 0;
        const size_t w = piece_text(v, tokens[i], out + k, room);
        if (w > room) { out[k] = 0; return fail(G4T_ERR_FULL, "decoded text exceeds %zu bytes", cap); }
        k += w;
    }
    out[k] = 0;
    return (int)k;
}

static int has_newline(const g4t_vocab *v, int id) {
    return id >= 0 && id < v->n && memchr(v->piece[id], '\n', (size_t)v->len[id]) != NULL;
}
static int thought_opener(const g4t_vocab *v, int id) {
    return id == v->sp[S_CHANNEL_THOUGHT] || id == v->sp[S_CHANNEL];
}

/* parse_response + skip_channel_label (main.c:2182-2214) */
void g4t_split_response(const g4t_vocab *v, const int *tokens, int n, int *ts, int *te, int *as) {
    int s = -1, e = -1;
    for (int i = 0; i < n; i++) {
        if (thought_opener(v, tokens[i]) && s < 0) {
            s = i + 1;
            if (tokens[s - 1] == v->sp[S_CHANNEL])
                while (s < n)
                    if (has_newline(v, tokens[s++])) break;
        } else if (tokens[i] == v->sp[S_CHANNEL_END]) {
            e = i;
        }
    }
    if (s >= 0 && e > s) {
        *ts = s;
        *te = e;
        *as = e + 1;
    } else {
        *ts = *te = -1;
        *as = 0;
    }
}

/* ---- the thinking state machine of generate() (main.c:2406-2470) ---------- */
void g4t_stream_init(g4t_stream *s, const g4t_vocab *v, int enable_thinking, int show_thinking, int budget) {
    memset(s, 0, sizeof *s);
    s->v = v;
    s->thinking = enable_thinking != 0;
    s->show = show_thinking != 0;
    s->budget = budget;
    s->mode = s->thinking ? 0 : 2;
}

int g4t_stream_force(const g4t_stream *s) {
    const int ce = s->v->sp[S_CHANNEL_END];
    if (s->thinking && s->saw_thought && !s->saw_answer && s->budget >= 0 && s->thinking_tokens >= s->budget && ce >= 0)
        return ce;
    return -1;
}

int g4t_stream_push(g4t_stream *s, int tok, char *out, size_t cap) {
    const g4t_vocab *v = s->v;
    if (s->thinking) {
        if (!s->saw_thought && thought_opener(v, tok)) {
            s->saw_thought = 1;
            s->mode = 0;
            s->skipping_label = tok == v->sp[S_CHANNEL];
        } else if (tok == v->sp[S_CHANNEL_END]) {
            s->skipping_label = 0;
            if (s->saw_thought && !s->saw_answer) {
                s->mode = 2;
                s->saw_answer = 1;
            }
        } else if (s->skipping_label) {
            if (has_newline(v, tok)) {
                s->skipping_label = 0;
                s->mode = s->show ? 1 : 0;
            }
        } else if (s->saw_thought && !s->saw_answer) {
            s->thinking_tokens++;
        }
    }
    if (!out || cap == 0) return 0;
    size_t k = 0;
    if (s->mode != 0) {
        k = piece_text(v, tok, out, cap - 1);
        if (k > cap - 1) k = cap - 1;
    }
    out[k] = 0;
    return (int)k;
}
