/* Greedy selection and the generation loop that drives the runtime.
 * Same contract as the reference include/generation.h:9-71 (names, limits,
 * stop precedence, atomic result, lowest-id ties, NaN/Inf rejection), so the
 * reference's callers link against it unchanged. */
#ifndef LUNELETTE_GENERATION_H
#define LUNELETTE_GENERATION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LUNELETTE_VOCAB_SIZE 131072
#define LUNELETTE_CONTEXT_LIMIT 256
#define LUNELETTE_LONG_CONTEXT_LIMIT 4352
#define LUNELETTE_BLOCK_LIMIT 256
#define LUNELETTE_GENERATION_LIMIT 256

/* include/generation.h:11-16. */
typedef struct {
    size_t max_new_tokens; /* 0..256 */
    int64_t eos_token;     /* 0..131071 */
} lunelette_generation_config;

#define LUNELETTE_GENERATION_DEFAULT {32, 2}

/* include/generation.h:18-28. */
typedef enum {
    LUNELETTE_STOP_LIMIT,
    LUNELETTE_STOP_EOS,
    LUNELETTE_STOP_CONTEXT
} lunelette_stop_reason;

typedef struct {
    int64_t tokens[LUNELETTE_GENERATION_LIMIT];
    size_t count;
    lunelette_stop_reason stop;
} lunelette_generation_result;

/* include/generation.h:35-36. Writes all 131072 last-token logits. */
typedef int (*lunelette_logits_fn)(void *context, const int64_t *ids, size_t count,
    float *logits, char *error, size_t capacity);

/* include/generation.h:38-45 (src/generation.c:8-34): strict '>' over all
 * 131072 logits, lowest id on ties (-0 == +0), any NaN/Inf rejects; token is
 * unchanged on failure; clears error on success. */
int lunelette_select_greedy(const float *logits, int64_t *token, char *error, size_t capacity);

/* include/generation.h:47-62 (src/generation.c:130-136). */
int lunelette_generate_with_logits(lunelette_logits_fn next, void *context,
    const int64_t *prompt, size_t count, const lunelette_generation_config *config,
    lunelette_generation_result *result, char *error, size_t capacity);

/* include/generation.h:64-71 (src/generation.c:36-128): context_limit is
 * exactly 256 or 4352; EOS beats budget beats context. */
int lunelette_generate_with_logits_capacity(lunelette_logits_fn next, void *context,
    const int64_t *prompt, size_t count, size_t context_limit,
    const lunelette_generation_config *config, lunelette_generation_result *result,
    char *error, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif
