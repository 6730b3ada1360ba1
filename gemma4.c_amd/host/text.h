/*
 * text.h -- host text path of the engine: the Gemma 4 vocabulary of a GGUF,
 * the BPE tokenizer and chat template, detokenization and the thinking /
 * answer split of generated tokens.
 *
 * Behaviour follows thamada/Gemma4.c gemma4-4b/cpu-blas/main.c: vocabulary
 * and merges from the GGUF metadata (parse_gguf, main.c:841-966;
 * init_tokenizer, 1010-1045), Gemma line escaping and greedy BPE (1047-1133),
 * special tokens and the chat template (1135-1312), detokenization and
 * special-token filtering (2127-2180, 2216-2231), response parsing
 * (2182-2214) and the thinking state machine of generate() (2406-2470).
 * All functions return 0 / a count on success and a negative G4T_ERR_* on
 * failure (the reference prints and exits instead); g4t_last_error() holds
 * the message.
 */
#ifndef G4_TEXT_H
#define G4_TEXT_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { G4T_ERR_ARG = -1, G4T_ERR_FORMAT = -2, G4T_ERR_NOMEM = -3, G4T_ERR_FULL = -4 };

/* longest prompt the template encodes (MAX_PROMPT_TOKS, main.c:67) */
#define G4T_MAX_PROMPT_TOKS 8192

typedef struct g4t_vocab g4t_vocab;

const char *g4t_last_error(void);

/* the tokenizer metadata of a GGUF image (tokenizer.ggml.tokens, .scores,
 * .merges, .bos_token_id, .eos_token_id, .add_space_prefix); the image is
 * only read during the call */
int  g4t_open_image(const void *data, size_t size, g4t_vocab **out);
int  g4t_open_file(const char *path, g4t_vocab **out);
void g4t_close(g4t_vocab *v);

int g4t_size(const g4t_vocab *v);
/* out[13]: bos, eos, eot, add_space_prefix, turn_start, turn_end,
 * turn_user, turn_model, turn_system, think, channel, channel_thought,
 * channel_end (-1 where the vocabulary has no such token) */
void g4t_specials(const g4t_vocab *v, int out[13]);
/* merge score of a token (its rank from the end of the merge list, or the
 * GGUF score; 0 if neither) */
float g4t_score(const g4t_vocab *v, int id);
/* the token whose text is exactly s[0..len) (lowest id on duplicates), or -1 */
int g4t_lookup(const g4t_vocab *v, const char *s, int len);
/* a token's raw text (not NUL-terminated) and its length */
const char *g4t_piece(const g4t_vocab *v, int id, int *len);

/* gemma_bpe_encode: UTF-8 characters looked up one by one (unknown ones
 * skipped), then greedy merging of the best-scoring adjacent pair */
int g4t_encode_raw(const g4t_vocab *v, const char *bytes, int len, int *out, int cap);
/* append_gemma_text: lines split at '\n', spaces escaped as U+2581 (and a
 * leading one when add_space_prefix), BPE per line, the newline token */
int g4t_encode_text(const g4t_vocab *v, const char *text, int *out, int cap);

/* chat_encode_history (main.c:1276-1298): bos, the thinking system turn if
 * asked, each message as a user (role 0) or model (role 1) turn, then the
 * model prefix.  G4T_ERR_FULL past cap tokens. */
int g4t_chat_encode(const g4t_vocab *v, const char *const *texts, const int *roles, int n_msgs, int thinking,
                    int *out, int cap);

/* 1 for the special tokens tokens_to_text and print_tok drop (main.c:2127) */
int g4t_is_special(const g4t_vocab *v, int id);
/* tokens_to_text: the pieces of tokens[start..end) without specials, U+2581
 * as a space; writes a NUL-terminated string of at most cap bytes and
 * returns its length (or G4T_ERR_FULL) */
int g4t_decode(const g4t_vocab *v, const int *tokens, int start, int end, char *out, size_t cap);
/* parse_response: the thinking channel's token range and the answer's
 * (thinking [ts, te), answer [as, n)); ts = te = -1 when there is no
 * closed thinking channel (then the answer is all of it) */
void g4t_split_response(const g4t_vocab *v, const int *tokens, int n, int *ts, int *te, int *as);

/* The thinking state machine of generate() over the generated tokens.
 * g4t_stream_next tells whether the next token must be the channel end
 * (the thinking budget is spent); g4t_stream_push takes the token that was
 * generated and writes what is to be printed (NUL-terminated, nothing when
 * hidden) into out. */
typedef struct {
    const g4t_vocab *v;
    int thinking, show, budget;          /* budget < 0: unlimited */
    int mode;                            /* 0 hidden, 1 thinking, 2 answer */
    int saw_thought, saw_answer, skipping_label, thinking_tokens, budget_hit;
} g4t_stream;
void g4t_stream_init(g4t_stream *s, const g4t_vocab *v, int enable_thinking, int show_thinking, int budget);
int  g4t_stream_force(const g4t_stream *s);          /* token to force next, or -1 */
/* returns the bytes written to out (at most cap - 1) */
int  g4t_stream_push(g4t_stream *s, int token, char *out, size_t cap);

#ifdef __cplusplus
}
#endif
#endif
