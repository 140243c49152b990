/* Greedy selection and the full-prefix generation loop, to the contract of
 * the reference's include/generation.h:38-71. */
#include "lunelette_generation.h"
#include "lh_scan.h"
#include "lh_host_alloc.h"

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

/* Request checks of include/generation.h:47-71, all made before any callback
 * (every prompt id, even for a zero budget). Returns the diagnostic of the
 * first problem, or NULL; *at names a bad prompt position. */
static const char *request_problem(lunelette_logits_fn next, const int64_t *prompt, size_t count,
    size_t limit, const lunelette_generation_config *config,
    const lunelette_generation_result *result, size_t *at)
{
    if (limit != LUNELETTE_CONTEXT_LIMIT && limit != LUNELETTE_LONG_CONTEXT_LIMIT) {
        return "generation: context limit must be 256 or 4352";
    }
    if (!next || !prompt || !config || !result) {
        return "generation: callback, prompt, config and result are required";
    }
    if (!count || count > limit) {
        return "generation: prompt length must be 1..context limit";
    }
    if (config->max_new_tokens > LUNELETTE_GENERATION_LIMIT) {
        return "generation: budget above 256 new tokens";
    }
    if (config->eos_token < 0 || config->eos_token >= LUNELETTE_VOCAB_SIZE) {
        return "generation: EOS id outside the vocabulary";
    }
    for (size_t i = 0; i < count; i++) {
        if (prompt[i] < 0 || prompt[i] >= LUNELETTE_VOCAB_SIZE) {
            *at = i;
            return "generation: prompt id at position %zu outside the vocabulary";
        }
    }
    return NULL;
}

/* Stop rule after `produced` new tokens with the sequence `length` long:
 * the last token being EOS wins over an exhausted budget, which wins over a
 * full context (the prompt's own ids never count as EOS). -1: continue. */
static int stop_rule(int64_t last, size_t produced, size_t length, size_t limit,
    const lunelette_generation_config *config)
{
    if (produced && last == config->eos_token) {
        return LUNELETTE_STOP_EOS;
    }
    if (produced == config->max_new_tokens) {
        return LUNELETTE_STOP_LIMIT;
    }
    if (length == limit) {
        return LUNELETTE_STOP_CONTEXT;
    }
    return -1;
}

/* The full prefix (prompt then generated ids) is handed to the callback on
 * every step; the caller's result is written only after the last step
 * succeeded, so a failure leaves it exactly as it was. */
int lunelette_generate_with_logits_capacity(lunelette_logits_fn next, void *context,
    const int64_t *prompt, size_t count, size_t context_limit,
    const lunelette_generation_config *config, lunelette_generation_result *result,
    char *error, size_t capacity)
{
    size_t at = 0;
    const char *problem = request_problem(next, prompt, count, context_limit, config, result,
        &at);
    if (problem) {
        if (error && capacity) {
            snprintf(error, capacity, problem, at);
        }
        return -1;
    }
    lunelette_generation_result staged = {.count = 0, .stop = LUNELETTE_STOP_LIMIT};
    size_t length = count;
    int64_t last = -1;
    int stop = stop_rule(last, 0, length, context_limit, config);
    int64_t *prefix = NULL;
    float *scratch = NULL;
    if (stop < 0) {
        prefix = lh_malloc(context_limit * sizeof *prefix);
        scratch = lh_malloc(LUNELETTE_VOCAB_SIZE * sizeof *scratch);
        if (!prefix || !scratch) {
            say(error, capacity, "generation: scratch allocation failed");
            lh_free(prefix);
            lh_free(scratch);
            return -1;
        }
        memcpy(prefix, prompt, count * sizeof *prefix);
    }
    while (stop < 0) {
        if (error && capacity) {
            error[0] = '\0';
        }
        if (next(context, prefix, length, scratch, error, capacity)) {
            if (error && capacity && !error[0]) {
                snprintf(error, capacity, "generation: the logits callback failed on new token "
                    "%zu", staged.count);
            }
            break;
        }
        if (lunelette_select_greedy(scratch, &last, error, capacity)) {
            break;
        }
        prefix[length++] = last;
        staged.tokens[staged.count++] = last;
        stop = stop_rule(last, staged.count, length, context_limit, config);
    }
    lh_free(prefix);
    lh_free(scratch);
    if (stop < 0) {
        return -1;
    }
    staged.stop = (lunelette_stop_reason)stop;
    *result = staged;
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
