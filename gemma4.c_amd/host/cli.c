/*
 * cli.c -- g4run, the command line of the engine: the options, single-shot
 * and interactive chat of thamada/Gemma4.c gemma4-4b/cpu-blas/main.c
 * (main 2577-2826, run_single_shot 2544-2575, run_interactive 2577-2620,
 * run_chat_turn 2508-2542, generate 2335-2488), with the forward pass, the
 * repetition penalty and sample_token on the GPU (libg4engine.so) and the
 * text path on the host (host/text.h).
 *
 *   g4run <model.gguf> [-p prompt] [-n tokens] [-t temp] [-k topp] [-r penalty]
 *         [-N window] [-s seed] [-l max_seq] [-i] [--think] [--show-thinking]
 *         [--thinking-budget n] [--dump-prompt] [--dump-gen] [--dump-logits-at n]
 *         [--dump-hidden-at pos] [--force-gen ids] [--f32-matmul] [--eager]
 */
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "engine.h"
#include "text.h"

#define TOP_K 40                  /* DEFAULT_TOP_K, main.c:71 */
#define PENALTY_LAST_N 64         /* main.c:72 */
#define THINKING_BUDGET 256       /* main.c:73 */
#define MAX_TURNS 128             /* MAX_CHAT_TURNS, main.c:69 */

typedef struct {
    int max_new, last_n, thinking, show, budget, dump_prompt, dump_gen, dump_logits_at, dump_hidden_at, graph;
    float temp, topp, penalty;
    uint64_t seed;
    int *force;
    int n_force;
} Opts;

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + (double)t.tv_nsec * 1e-9;
}

/* parse_token_list (main.c:2296-2316) */
static int *token_list(const char *s, int *n_out) {
    int cap = 64, n = 0;
    int *t = (int *)malloc((size_t)cap * sizeof(int));
    while (t && *s) {
        while (*s == ' ' || *s == ',') s++;
        if (!*s) break;
        char *end = NULL;
        const long v = strtol(s, &end, 10);
        if (end == s) break;
        if (n >= cap) {
            cap *= 2;
            int *nt = (int *)realloc(t, (size_t)cap * sizeof(int));
            if (!nt) { free(t); return NULL; }
            t = nt;
        }
        t[n++] = (int)v;
        s = end;
    }
    *n_out = n;
    return t;
}

/* dump_logits_top (main.c:2318-2333): the k largest logits in descending
 * order (equal values by index; the reference's exchange sort may order
 * exact ties otherwise) */
static void dump_top(const float *lg, int n, int k) {
    if (k > n) k = n;
    int *idx = (int *)malloc((size_t)(k > 0 ? k : 1) * sizeof(int));
    int m = 0;
    for (int i = 0; i < n && idx; i++) {
        if (m == k && !(lg[i] > lg[idx[k - 1]])) continue;
        int j = m < k ? m++ : k - 1;
        while (j > 0 && lg[i] > lg[idx[j - 1]]) { idx[j] = idx[j - 1]; j--; }
        idx[j] = i;
    }
    fprintf(stderr, "  top-%d logits:", m);
    for (int i = 0; i < m; i++) fprintf(stderr, " %d=%.4f", idx[i], lg[idx[i]]);
    fputc('\n', stderr);
    free(idx);
}

static void hidden_dump(g4e_model *m, int pos) {
    int cfg[9];
    g4e_config(m, cfg);
    const int L = cfg[2];
    /* dump_kv_fingerprint lines of layer 0 (main.c:1829-1836) */
    static const char *tags[G4E_FP_TAGS] = {"attn_norm", "K_pre_norm", "K_pre_rope", "K_store", "K_read0", "K_readN",
                                            "q_out"};
    float fp[G4E_FP_TAGS * 7];
    int have[G4E_FP_TAGS];
    if (!g4e_kv_fingerprint(m, fp, have)) {
        for (int t = 0; t < G4E_FP_Q_OUT; t++) {
            if (!have[t]) continue;
            const float *f = fp + 7 * t;
            fprintf(stderr, "[kv L0 P%d] %s sum=%.4f l2=%.4f max=%.4f v0=%.6f v1=%.6f v2=%.6f v3=%.6f\n",
                    t == G4E_FP_K_READ0 ? 0 : pos, tags[t], f[0], f[1], f[2], f[3], f[4], f[5], f[6]);
        }
        if (have[G4E_FP_Q_OUT]) {
            const float *f = fp + 7 * G4E_FP_Q_OUT;
            fprintf(stderr, "[hidden pos %d] layer %2d q_out sum=%.4f l2=%.4f max=%.4f\n", pos, 0, f[0], f[1], f[2]);
        }
    }
    float *st = (float *)malloc((size_t)(2 * L + 1) * 3 * sizeof(float));
    if (!st || g4e_hidden_stats(m, st)) { free(st); return; }
    fprintf(stderr, "[hidden pos %d] after_emb sum=%.4f l2=%.4f max=%.4f\n", pos, st[0], st[1], st[2]);
    for (int l = 0; l < L; l++) {
        const float *a = st + 3 * (1 + 2 * l), *b = st + 3 * (2 + 2 * l);
        fprintf(stderr, "[hidden pos %d] layer %2d attn_out sum=%.4f l2=%.4f max=%.4f\n", pos, l, a[0], a[1], a[2]);
        fprintf(stderr, "[hidden pos %d] layer %2d sum=%.4f l2=%.4f max=%.4f\n", pos, l, b[0], b[1], b[2]);
    }
    free(st);
}

/* generate (main.c:2335-2488); the generated tokens go to gen (cap max_new) */
static int generate(g4e_model *m, const g4t_vocab *v, const int *prompt, int n_prompt, const Opts *o, int *gen,
                    int *n_gen) {
    int cfg[9], sp[13];
    g4e_config(m, cfg);
    g4t_specials(v, sp);
    const int vocab = cfg[5], max_seq = cfg[6], eos = sp[1], eot = sp[2];
    float *logits = o->dump_logits_at >= 0 ? (float *)malloc((size_t)vocab * sizeof(float)) : NULL;
    g4t_stream st;
    g4t_stream_init(&st, v, o->thinking, o->show, o->budget);
    *n_gen = 0;
    const double t0 = now_s();
    int np = n_prompt - 1 < max_seq ? n_prompt - 1 : max_seq;
    if (o->dump_hidden_at >= 0) g4e_set_dump_hidden_at(m, o->dump_hidden_at);
    if (np > 0 && g4e_prefill(m, prompt, np, 0)) {
        fprintf(stderr, "Error: %s\n", g4e_last_error());
        free(logits);
        return -1;
    }
    if (o->dump_hidden_at >= 0 && o->dump_hidden_at < np) hidden_dump(m, o->dump_hidden_at);
    const double t_pf = now_s() - t0;
    if (n_prompt > 0)
        fprintf(stderr, "Prefill complete: %d tokens in %.2fs (%.2f tok/s)\n", n_prompt, t_pf,
                t_pf > 0 ? n_prompt / t_pf : 0.0);
    if (g4e_gen_begin(m, o->seed)) { fprintf(stderr, "Error: %s\n", g4e_last_error()); free(logits); return -1; }
    const double t1 = now_s();
    int token = prompt[n_prompt - 1], warned = 0, rc = 0;
    char text[4096];
    for (int pos = n_prompt - 1; pos < n_prompt + o->max_new - 1; pos++) {
        if (pos >= max_seq) {
            fprintf(stderr, "\n[max sequence length %d reached]\n", max_seq);
            break;
        }
        int forced = g4t_stream_force(&st);
        if (forced >= 0 && !warned) {
            fprintf(stderr, "\n[thinking budget %d tokens reached; forcing <channel|>]\n", o->budget);
            warned = 1;
        }
        if (forced < 0 && o->force && *n_gen < o->n_force) forced = o->force[*n_gen];
        int next;
        if (g4e_gen_step(m, token, pos, o->temp, o->topp, TOP_K, o->penalty, o->last_n, forced, o->graph, &next)) {
            fprintf(stderr, "Error: %s\n", g4e_last_error());
            rc = -1;
            break;
        }
        if (pos == o->dump_hidden_at) hidden_dump(m, pos);
        if (logits && *n_gen == o->dump_logits_at && !g4e_read_logits(m, logits)) {
            fprintf(stderr, "[logits at gen step %d, pos %d]\n", *n_gen, pos);
            dump_top(logits, vocab, 8);
        }
        if (next == eos || next == eot) break;
        const int saw_thought = st.saw_thought, saw_answer = st.saw_answer;
        g4t_stream_push(&st, next, text, sizeof text);
        if (o->show && !saw_thought && st.saw_thought) fputs("\n--- Thinking ---\n", stderr);
        if (o->show && !saw_answer && st.saw_answer) fputs("\n--- Answer ---\n", stderr);
        fputs(text, stdout);
        fflush(stdout);
        gen[(*n_gen)++] = next;
        token = next;
    }
    const double t2 = now_s();
    free(logits);
    const double dec = t2 - t1, total = t2 - t0;
    fputc('\n', stdout);
    fprintf(stderr, "\nDecode complete: %d tokens in %.2fs (%.2f tok/s)\n", *n_gen, dec, dec > 0 ? *n_gen / dec : 0.0);
    printf("\n\n--- %d prompt tokens + %d generated tokens ---\n", n_prompt, *n_gen);
    printf("--- %.1fs total ---\n", total);
    /* throughput_summary (main.c:2283-2294) */
    fprintf(stderr, "--- throughput ---\n");
    fprintf(stderr, "  prefill: %.2f tok/s\n", t_pf > 0 ? n_prompt / t_pf : 0.0);
    fprintf(stderr, "  decode:  %.2f tok/s\n", dec > 0 ? *n_gen / dec : 0.0);
    fprintf(stderr, "  total:   %.2f tok/s\n", total > 0 ? (n_prompt + *n_gen) / total : 0.0);
    return rc;
}

static void usage(const char *argv0) {
    fprintf(stderr, "Usage: %s <model.gguf> [options]\n", argv0);
    fprintf(stderr, "Options:\n"
                    "  -p <prompt>       User prompt (default: Hello, how are you?)\n"
                    "  -n <tokens>       Max tokens to generate per turn (default: 256)\n"
                    "  -t <temp>         Temperature (default: 0.6)\n"
                    "  -k <topp>         Top-p sampling (default: 0.9)\n"
                    "  -r <penalty>      Repetition penalty (default: 1.0)\n"
                    "  -N <n>            Repetition penalty window (default: 64, 0 = all tokens)\n"
                    "  -s <seed>         Random seed (default: time)\n"
                    "  -l <len>          Max sequence length (default: 8192)\n"
                    "  -i                Interactive multi-turn mode\n"
                    "  --think           Enable thinking mode\n"
                    "  --show-thinking   Show reasoning trace (implies --think)\n"
                    "  --thinking-budget <n>  Max thinking tokens before forcing <channel|> (default: %d with --think)\n"
                    "  --dump-prompt     Print prompt token IDs to stderr\n"
                    "  --dump-gen        Print generated token IDs to stderr\n"
                    "  --dump-logits-at <n>   Dump top logits at generation step n\n"
                    "  --dump-hidden-at <pos> Dump hidden stats per layer at sequence pos\n"
                    "  --force-gen <ids> Force the generated token IDs (comma-separated)\n"
                    "  --f32-matmul      Q4_K/Q5_K through dequantized fp32 weights\n"
                    "  --eager           Launch every decode step's kernels instead of replaying a graph\n",
            THINKING_BUDGET);
}

int main(int argc, char **argv) {
    setvbuf(stdout, NULL, _IOLBF, 0);
    if (argc < 2) { usage(argv[0]); return 1; }
    const char *path = argv[1], *prompt = "Hello, how are you?";
    Opts o = {256, PENALTY_LAST_N, 0, 0, -1, 0, 0, -1, -1, 1, 0.6f, 0.9f, 1.0f, (uint64_t)time(NULL), NULL, 0};
    int max_seq = 8192, interactive = 0, budget_set = 0, f32 = 0;
    for (int i = 2; i < argc; i++) {
        const char *a = argv[i];
        if (!strcmp(a, "-i") || !strcmp(a, "--interactive")) { interactive = 1; continue; }
        if (!strcmp(a, "--think")) { o.thinking = 1; continue; }
        if (!strcmp(a, "--show-thinking")) { o.thinking = o.show = 1; continue; }
        if (!strcmp(a, "--dump-prompt")) { o.dump_prompt = 1; continue; }
        if (!strcmp(a, "--dump-gen")) { o.dump_gen = 1; continue; }
        if (!strcmp(a, "--f32-matmul")) { f32 = 1; continue; }
        if (!strcmp(a, "--eager")) { o.graph = 0; continue; }
        if (i + 1 >= argc) { fprintf(stderr, "Error: option %s requires a value\n", a); return 1; }
        const char *val = argv[++i];
        if (!strcmp(a, "--thinking-budget")) { o.budget = atoi(val); budget_set = 1; }
        else if (!strcmp(a, "--force-gen")) { free(o.force); o.force = token_list(val, &o.n_force); }
        else if (!strcmp(a, "--dump-logits-at")) o.dump_logits_at = atoi(val);
        else if (!strcmp(a, "--dump-hidden-at")) o.dump_hidden_at = atoi(val);
        else if (!strcmp(a, "-p")) prompt = val;
        else if (!strcmp(a, "-n")) o.max_new = atoi(val);
        else if (!strcmp(a, "-t")) o.temp = (float)atof(val);
        else if (!strcmp(a, "-k")) o.topp = (float)atof(val);
        else if (!strcmp(a, "-r")) o.penalty = (float)atof(val);
        else if (!strcmp(a, "-N")) o.last_n = atoi(val);
        else if (!strcmp(a, "-s")) o.seed = (uint64_t)strtoull(val, NULL, 10);
        else if (!strcmp(a, "-l")) max_seq = atoi(val);
        else { fprintf(stderr, "Error: unknown option %s\n", a); return 1; }
    }
    if (o.thinking && !budget_set) o.budget = THINKING_BUDGET;
    if (o.max_new < 0) o.max_new = 0;
    printf("Loading %s ...\n", path);
    g4t_vocab *v = NULL;
    if (g4t_open_file(path, &v)) { fprintf(stderr, "Error: %s\n", g4t_last_error()); return 1; }
    g4e_model *m = NULL;
    if (g4e_open_file(path, max_seq, 0, &m)) {
        fprintf(stderr, "Error: %s\n", g4e_last_error());
        g4t_close(v);
        return 1;
    }
    int cfg[9];
    g4e_config(m, cfg);
    printf("Model: dim=%d hidden=%d layers=%d heads=%d kv_heads=%d vocab=%d\n", cfg[0], cfg[1], cfg[2], cfg[3], cfg[4],
           cfg[5]);
    if (f32) g4e_set_f32_matmul(m, 1);
    int *prompt_toks = (int *)malloc(G4T_MAX_PROMPT_TOKS * sizeof(int));
    int *gen = (int *)malloc(((size_t)o.max_new + 1) * sizeof(int));
    int rc = prompt_toks && gen ? 0 : 1;
    const char *texts[MAX_TURNS];
    int roles[MAX_TURNS], n_hist = 0;
    char *owned[MAX_TURNS] = {0};
    char *line = NULL;
    size_t line_cap = 0;
    if (interactive) {
        fprintf(stderr, "Interactive mode ( /quit to exit )\n");
        if (o.thinking) {
            fprintf(stderr, "Thinking mode: ON%s", o.show ? " (showing trace)" : " (answer only)");
            if (o.budget >= 0) fprintf(stderr, " [budget=%d tokens]", o.budget);
            fputc('\n', stderr);
        }
    }
    int first = 1;
    while (rc == 0) {
        /* the next user message: the -p prompt first, then stdin when interactive */
        const char *msg = NULL;
        if (first && (!interactive || (prompt && prompt[0]))) {
            msg = prompt;
        } else if (interactive) {
            fprintf(stderr, "You: ");
            fflush(stderr);
            ssize_t n = getline(&line, &line_cap, stdin);
            if (n < 0) break;
            while (n > 0 && (line[n - 1] == '\n' || line[n - 1] == '\r')) line[--n] = 0;
            if (n == 0 || !strcmp(line, "/quit") || !strcmp(line, "/exit")) break;
            msg = line;
        } else {
            break;
        }
        first = 0;
        if (n_hist >= MAX_TURNS) { fprintf(stderr, "Error: max %d turns reached\n", MAX_TURNS); rc = 1; break; }
        owned[n_hist] = strdup(msg);
        texts[n_hist] = owned[n_hist];
        roles[n_hist++] = 0;
        const int n_prompt = g4t_chat_encode(v, texts, roles, n_hist, o.thinking, prompt_toks, G4T_MAX_PROMPT_TOKS);
        if (n_prompt < 0) {
            fprintf(stderr, "Error: %s\n", g4t_last_error());
            rc = 1;
            break;
        }
        if (!interactive) {
            printf("Prompt: \"%s\" (%d tokens)%s\n\n", msg, n_prompt, o.thinking ? " [thinking]" : "");
            if (o.dump_prompt) {
                fprintf(stderr, "Prompt token IDs:");
                for (int i = 0; i < n_prompt; i++) fprintf(stderr, " %d", prompt_toks[i]);
                fputc('\n', stderr);
            }
        } else {
            fputs("Model: ", stdout);
            fflush(stdout);
        }
        int n_gen = 0;
        if (generate(m, v, prompt_toks, n_prompt, &o, gen, &n_gen)) { rc = 1; break; }
        if (o.dump_gen) {
            fprintf(stderr, "Generated token IDs:");
            for (int i = 0; i < n_gen; i++) fprintf(stderr, " %d", gen[i]);
            fputc('\n', stderr);
        }
        if (!interactive) break;
        /* run_chat_turn: the answer (thinking stripped) joins the history */
        int ts, te, as;
        g4t_split_response(v, gen, n_gen, &ts, &te, &as);
        size_t cap = 1 << 20;
        char *ans = (char *)malloc(cap);
        if (!ans || g4t_decode(v, gen, as, n_gen, ans, cap) < 0) { free(ans); rc = 1; break; }
        if (!ans[0]) {
            fprintf(stderr, "Warning: empty model response\n");
            free(ans);
            continue;
        }
        if (n_hist >= MAX_TURNS) { free(ans); fprintf(stderr, "Error: max %d turns reached\n", MAX_TURNS); rc = 1; break; }
        owned[n_hist] = ans;
        texts[n_hist] = ans;
        roles[n_hist++] = 1;
    }
    if (interactive) fprintf(stderr, "\nBye.\n");
    for (int i = 0; i < n_hist; i++) free(owned[i]);
    free(line);
    free(prompt_toks);
    free(gen);
    free(o.force);
    g4e_close(m);
    g4t_close(v);
    return rc;
}
