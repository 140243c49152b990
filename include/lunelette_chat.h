/* Chat framing of one turn: the reference's include/chat.h:1-15 and
 * src/chat.c:1-59. BOS, then [SYSTEM_PROMPT] system [/SYSTEM_PROMPT] when a
 * system text is given, then [INST] prompt [/INST] (raw: the prompt alone,
 * and a system text is refused). Each text is encoded as ordinary text. At
 * most 256 ids (the runtime's short context); 0 on success, -1 on failure with
 * ids and count untouched. */
#ifndef LUNELETTE_CHAT_H
#define LUNELETTE_CHAT_H

#include <stddef.h>
#include <stdint.h>

#include "lunelette_generation.h"
#include "lunelette_tokenizer.h"

#ifdef __cplusplus
extern "C" {
#endif

int lunelette_chat_prompt(const lunelette_tokenizer *tokenizer, const char *prompt,
    const char *system, int raw, int64_t ids[LUNELETTE_CONTEXT_LIMIT], size_t *count,
    char *error, size_t error_size);

#ifdef __cplusplus
}
#endif

#endif
