/* Chat framing of one turn, to the contract of the reference's include/chat.h:
 * BOS, then [SYSTEM_PROMPT] system [/SYSTEM_PROMPT] when a system text is
 * given, then [INST] prompt [/INST]; raw framing is BOS + prompt and takes no
 * system text. Texts are encoded as ordinary text, so a literal control
 * spelling inside them stays text.
 *
 * The frame is planned as a list of segments (a control id, or the encoding
 * of one text), measured, and written to the caller's array only when it fits
 * the 256-id context, so a failure leaves ids and count untouched. */
#include "lunelette_chat.h"
#include "lh_host_alloc.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    int64_t control;       /* id of a control segment, or -1 for text */
    const char *text;      /* text to encode (control == -1) */
    uint32_t *ids;         /* encoded text, owned */
    size_t n;
} segment;

static void fail(char *error, size_t error_size, const char *message)
{
    if (error && error_size) {
        snprintf(error, error_size, "%s", message);
    }
}

int lunelette_chat_prompt(const lunelette_tokenizer *tokenizer, const char *prompt,
    const char *system, int raw, int64_t ids[LUNELETTE_CONTEXT_LIMIT], size_t *count,
    char *error, size_t error_size)
{
    if (!tokenizer || !prompt || !ids || !count) {
        fail(error, error_size, "chat: tokenizer, prompt and output are required");
        return -1;
    }
    if (raw && system) {
        fail(error, error_size, "chat: raw framing takes no system text");
        return -1;
    }
    segment plan[7];
    size_t segments = 0;
    plan[segments++] = (segment){LUNELETTE_TOKEN_BOS, NULL, NULL, 0};
    if (system) {
        plan[segments++] = (segment){LUNELETTE_TOKEN_SYSTEM, NULL, NULL, 0};
        plan[segments++] = (segment){-1, system, NULL, 0};
        plan[segments++] = (segment){LUNELETTE_TOKEN_END_SYSTEM, NULL, NULL, 0};
    }
    if (!raw) {
        plan[segments++] = (segment){LUNELETTE_TOKEN_INST, NULL, NULL, 0};
    }
    plan[segments++] = (segment){-1, prompt, NULL, 0};
    if (!raw) {
        plan[segments++] = (segment){LUNELETTE_TOKEN_END_INST, NULL, NULL, 0};
    }

    int status = -1;
    size_t total = 0;
    for (size_t i = 0; i < segments; i++) {
        segment *s = &plan[i];
        if (s->control >= 0) {
            total += 1;
            continue;
        }
        if (!lunelette_tokenizer_encode(tokenizer, (const unsigned char *)s->text,
                strlen(s->text), &s->ids, &s->n, error, error_size)) {
            goto release;
        }
        total += s->n;
    }
    if (total > LUNELETTE_CONTEXT_LIMIT) {
        if (error && error_size) {
            snprintf(error, error_size, "chat: the framed turn needs %zu ids, over the 256-id "
                "context", total);
        }
        goto release;
    }
    size_t at = 0;
    for (size_t i = 0; i < segments; i++) {
        if (plan[i].control >= 0) {
            ids[at++] = plan[i].control;
        } else {
            for (size_t j = 0; j < plan[i].n; j++) {
                ids[at++] = plan[i].ids[j];
            }
        }
    }
    *count = at;
    status = 0;
release:
    for (size_t i = 0; i < segments; i++) {
        lh_free(plan[i].ids);
    }
    return status;
}
