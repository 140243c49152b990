/* Greedy selection and the full-prefix generation loop (contract of the
 * reference include/generation.h:38-71, behaviour of src/generation.c:8-136). */
#include "lunelette_generation.h"
#include "lh_scan.h"

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static void say(char *error, size_t capacity, const char *text)
{
    if (error && capacity) {
        snprintf(error, capacity, "%s", text);
    }
}

/* The reference's forward scan with a strict > keeps the first index of the
 * maximum (-0.0 and +0.0 compare equal) and fails at the first nonfinite
 * logit; lh_argmax_all_finite gives the same index in one vectorized pass,
 * and only on failure a second pass names the first nonfinite logit. */
int lunelette_select_greedy(const float *logits, int64_t *token, char *error, size_t capacity)
{
    if (!logits || !token) {
        say(error, capacity, "selection: require logits and token");
        return -1;
    }
    size_t best;
    if (!lh_argmax_all_finite(logits, LUNELETTE_VOCAB_SIZE, &best)) {
        if (error && capacity) {
            snprintf(error, capacity, "selection: nonfinite logit at token %zu",
                lh_first_nonfinite(logits, LUNELETTE_VOCAB_SIZE));
        }
        return -1;
    }
    *token = (int64_t)best;
    if (error && capacity) {
        error[0] = '\0';
    }
    return 0;
}

int lunelette_generate_with_logits_capacity(lunelette_logits_fn next, void *context,
    const int64_t *prompt, size_t count, size_t context_limit,
    const lunelette_generation_config *config, lunelette_generation_result *result,
    char *error, size_t capacity)
{
    say(error, capacity, context_limit == LUNELETTE_CONTEXT_LIMIT ?
        "generation: require callback, prompt 1..256, config budget 0..256, valid EOS, result" :
        "generation: require callback, context 256 or 4352, prompt within context, "
        "config budget 0..256, valid EOS, result");
    if (!next || !prompt || !config || !result || !count || count > context_limit ||
        (context_limit != LUNELETTE_CONTEXT_LIMIT &&
            context_limit != LUNELETTE_LONG_CONTEXT_LIMIT) ||
        config->max_new_tokens > LUNELETTE_GENERATION_LIMIT || config->eos_token < 0 ||
        config->eos_token >= LUNELETTE_VOCAB_SIZE) {
        return -1;
    }
    for (size_t i = 0; i < count; i++) {
        if (prompt[i] < 0 || prompt[i] >= LUNELETTE_VOCAB_SIZE) {
            if (error && capacity) {
                snprintf(error, capacity, "generation: invalid prompt token at %zu", i);
            }
            return -1;
        }
    }
    int64_t *ids = malloc(context_limit * sizeof *ids);
    float *logits = NULL;
    if (!ids) {
        say(error, capacity, "generation: prefix allocation failed");
        return -1;
    }
    memcpy(ids, prompt, count * sizeof *ids);
    if (config->max_new_tokens && count < context_limit) {
        logits = malloc(LUNELETTE_VOCAB_SIZE * sizeof(float));
        if (!logits) {
            say(error, capacity, "generation: logits allocation failed");
            free(ids);
            return -1;
        }
    }
    lunelette_generation_result pending;
    memset(&pending, 0, sizeof pending);
    pending.stop = LUNELETTE_STOP_LIMIT;
    int status = 0;
    while (pending.count < config->max_new_tokens) {
        if (count == context_limit) {
            pending.stop = LUNELETTE_STOP_CONTEXT;
            break;
        }
        if (error && capacity) {
            snprintf(error, capacity, "generation: logits callback failed at step %zu",
                pending.count);
        }
        int64_t best;
        if (next(context, ids, count, logits, error, capacity) ||
            lunelette_select_greedy(logits, &best, error, capacity)) {
            status = -1;
            break;
        }
        ids[count++] = best;
        pending.tokens[pending.count++] = best;
        if (best == config->eos_token) {
            pending.stop = LUNELETTE_STOP_EOS;
            break;
        }
    }
    free(ids);
    free(logits);
    if (status) {
        return -1;
    }
    *result = pending;
    if (error && capacity) {
        error[0] = '\0';
    }
    return 0;
}

int lunelette_generate_with_logits(lunelette_logits_fn next, void *context,
    const int64_t *prompt, size_t count, const lunelette_generation_config *config,
    lunelette_generation_result *result, char *error, size_t capacity)
{
    return lunelette_generate_with_logits_capacity(next, context, prompt, count,
        LUNELETTE_CONTEXT_LIMIT, config, result, error, capacity);
}
