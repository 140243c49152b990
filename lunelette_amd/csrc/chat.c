/* Chat framing of one turn (behaviour of the reference's src/chat.c:6-59):
 * BOS, [SYSTEM_PROMPT] system [/SYSTEM_PROMPT] when given, [INST] prompt
 * [/INST] unless raw. Texts are encoded as ordinary text; the output is
 * written only when the whole frame fits the 256-token context. */
#include "lunelette_chat.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int lunelette_chat_prompt(const lunelette_tokenizer *tokenizer, const char *prompt,
    const char *system, int raw, int64_t ids[LUNELETTE_CONTEXT_LIMIT], size_t *count,
    char *error, size_t error_size)
{
    if (!tokenizer || !prompt || !ids || !count || (raw && system)) {
        if (error && error_size) {
            snprintf(error, error_size, "Invalid prompt arguments (raw forbids system)");
        }
        return -1;
    }
    uint32_t *user = NULL, *sys = NULL;
    size_t user_n = 0, sys_n = 0;
    int status = -1;
    if (!lunelette_tokenizer_encode(tokenizer, (const unsigned char *)prompt, strlen(prompt),
            &user, &user_n, error, error_size) ||
        (system && !lunelette_tokenizer_encode(tokenizer, (const unsigned char *)system,
            strlen(system), &sys, &sys_n, error, error_size))) {
        goto done;
    }
    const size_t framing = 1 + (raw ? 0 : 2) + (system ? 2 : 0);
    const size_t total = framing + user_n + sys_n;
    if (total > LUNELETTE_CONTEXT_LIMIT) {
        if (error && error_size) {
            snprintf(error, error_size, "Prompt exceeds 256-token context (%zu tokens)", total);
        }
        goto done;
    }
    size_t n = 0;
    ids[n++] = LUNELETTE_TOKEN_BOS;
    if (system) {
        ids[n++] = LUNELETTE_TOKEN_SYSTEM;
        for (size_t i = 0; i < sys_n; i++) {
            ids[n++] = sys[i];
        }
        ids[n++] = LUNELETTE_TOKEN_END_SYSTEM;
    }
    if (!raw) {
        ids[n++] = LUNELETTE_TOKEN_INST;
    }
    for (size_t i = 0; i < user_n; i++) {
        ids[n++] = user[i];
    }
    if (!raw) {
        ids[n++] = LUNELETTE_TOKEN_END_INST;
    }
    *count = n;
    status = 0;
done:
    free(user);
    free(sys);
    return status;
}
