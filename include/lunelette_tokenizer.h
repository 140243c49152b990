/* Tekken 13 byte-level BPE tokenizer, the text side of the runtime's callers.
 *
 * Same contract as the reference's include/tokenizer.h:1-59 (names, limits,
 * ownership, the 1/0 return convention) and the behaviour of
 * src/tokenizer.c:131-608: loads exactly the supported Tekken13 JSON schema
 * (config v13 with the canonical pre-tokenizer pattern, 130072 ordinary ranks
 * with canonical base64 bytes covering every single byte, 1000 specials with
 * the framing spellings at 1, 2, 3, 4, 17, 18), splits text with that
 * pattern and merges each piece by lowest rank, leftmost on ties. Ordinary
 * ids are rank + 1000. Text is strict UTF-8; literal special spellings are
 * ordinary text.
 */
#ifndef LUNELETTE_TOKENIZER_H
#define LUNELETTE_TOKENIZER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LUNELETTE_TOKENIZER_MAX_INPUT 4096u
#define LUNELETTE_TOKENIZER_LONG_INPUT 32768u
#define LUNELETTE_TOKENIZER_VOCAB_SIZE 131072u
#define LUNELETTE_TOKENIZER_SPECIAL_COUNT 1000u

/* include/tokenizer.h:13-20. */
enum lunelette_special_token {
    LUNELETTE_TOKEN_BOS = 1,
    LUNELETTE_TOKEN_EOS = 2,
    LUNELETTE_TOKEN_INST = 3,
    LUNELETTE_TOKEN_END_INST = 4,
    LUNELETTE_TOKEN_SYSTEM = 17,
    LUNELETTE_TOKEN_END_SYSTEM = 18
};

typedef struct lunelette_tokenizer lunelette_tokenizer;

/* include/tokenizer.h:24-32. 1 on success; on failure *out is NULL. */
int lunelette_tokenizer_open(const char *path, lunelette_tokenizer **out,
    char *error, size_t error_size);
void lunelette_tokenizer_close(lunelette_tokenizer *tokenizer);

/* include/tokenizer.h:34-39: at most MAX_INPUT bytes; caller frees *ids; on
 * error *ids = NULL, *count = 0. */
int lunelette_tokenizer_encode(const lunelette_tokenizer *tokenizer,
    const unsigned char *text, size_t length, uint32_t **ids, size_t *count,
    char *error, size_t error_size);

/* include/tokenizer.h:41-47: input_limit is MAX_INPUT or LONG_INPUT. */
int lunelette_tokenizer_encode_with_limit(const lunelette_tokenizer *tokenizer,
    const unsigned char *text, size_t length, size_t input_limit,
    uint32_t **ids, size_t *count, char *error, size_t error_size);

/* include/tokenizer.h:49-57: raw bytes of ordinary ids (specials 0..999 and
 * ids >= 131072 fail), at most MAX_INPUT ids and 4 MiB; *bytes gets an extra
 * NUL not counted in *length. */
int lunelette_tokenizer_decode(const lunelette_tokenizer *tokenizer,
    const uint32_t *ids, size_t count, unsigned char **bytes, size_t *length,
    char *error, size_t error_size);

/* Additive: the pre-tokenizer's piece boundaries of a strict UTF-8 text of at
 * most LONG_INPUT bytes, as byte offsets: ends[k] is the end of piece k
 * (pieces are contiguous from 0). Returns the number of pieces, or -1 (invalid
 * UTF-8, arguments, or more pieces than capacity). No tokenizer file needed. */
long lunelette_tokenizer_split(const unsigned char *text, size_t length, size_t *ends,
    size_t capacity);

#ifdef __cplusplus
}
#endif

#endif
