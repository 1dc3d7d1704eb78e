/* TEST INFRASTRUCTURE ONLY: the C restatement of the reference int8 step (cpu/ygg.cpp:222-459) used as the checker.
   Not part of the product; see ygg_oracle.c. */
#ifndef YGG_ORACLE_H
#define YGG_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { YO_OK = 0, YO_ERR_IO = 1, YO_ERR_FORMAT = 2, YO_ERR_LIMITS = 3, YO_ERR_NOMEM = 4, YO_ERR_ARG = 5,
       YO_ERR_TOKEN = 6 };

/* Per-stream digest of every (layer, leaf, int8 state) in token order:
   d = d * MUL + (leaf * LEAF + sum_i (u8(q_i) + 1) * ((2 i + 1) * COORD) + l)  (mod 2^64), starting from INIT. */
#define YO_DIGEST_INIT 0xCBF29CE484222325ull
#define YO_DIGEST_MUL 0x100000001B3ull
#define YO_DIGEST_LEAF 0xD6E8FEB86659FD93ull
#define YO_DIGEST_COORD 0x9E3779B97F4A7C15ull

typedef struct yo_model yo_model;

int yo_load(const char *path, yo_model **out, char *err, int errlen);
void yo_free(yo_model *m);
/* n_layers, n, block, vocab, depth, R, R2, input_rank, shift, E, VP, factored */
int yo_info(const yo_model *m, int32_t *out12);
/* tokens (B, T); state (B, L, n) int8 in/out; optional: logits (B, T, V), leaves (B, T, L), states (B, T, L, n),
   digest (B) in/out (seed with yo_digest_init()) */
int yo_run(const yo_model *m, const int32_t *tokens, int B, int T, int8_t *state, float *logits, int32_t *leaves,
           int8_t *states, uint64_t *digest, int threads, char *err, int errlen);
/* Full-size checks: the digest (as yo_run) and lgsum (B) in/out, += the f32 bit patterns (as uint32) of every logit of
   the stream's tokens, mod 2^64; no per-token outputs are kept. */
int yo_run_sums(const yo_model *m, const int32_t *tokens, int B, int T, int8_t *state, uint64_t *digest,
                uint64_t *lgsum, int threads, char *err, int errlen);
uint64_t yo_digest_init(void);
/* The f32 softmax of the reference's `time` mode (cpu/ygg.cpp:44-72) over rows of V logits: probabilities into
   probs (rows, V) and the log-sum-exp of each row into lse (rows). */
void yo_softmax(const float *logits, long rows, int V, float *probs, float *lse);

#ifdef __cplusplus
}
#endif
#endif
