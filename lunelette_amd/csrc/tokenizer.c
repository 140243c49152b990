/* Tekken 13 tokenizer (behaviour of the reference's src/tokenizer.c:131-608
 * and its bounded JSON reader src/tokenizer_json.c:1-417).
 *
 * JSON: a strict reader into a node array; strings are decoded in place
 * (escapes, surrogate pairs, validated UTF-8). Limits as in the reference:
 * 32 MiB file, depth 32, 1 500 000 nodes, decoded strings <= 4096 bytes,
 * objects <= 64 members without duplicate keys, arrays <= 131072 elements,
 * number and literal tokens <= 128 bytes.
 *
 * Vocabulary: token bytes of every ordinary rank in one arena (rank order),
 * indexed by an open-addressing table (64-bit FNV-1a, 2^18 slots).
 *
 * Encoding: strict UTF-8 decode with a class mask per code point
 * (lh_unicode_classes.h), split by the pre-tokenizer pattern (its seven
 * alternatives in order, with the backtracking each one needs), then each
 * piece is one token when its bytes are, else merged from single bytes by
 * lowest-rank adjacent pair, leftmost on equal ranks (a min-heap of
 * (rank, position) with lazily dropped stale entries). */
#define _POSIX_C_SOURCE 200809L
#include "lunelette_tokenizer.h"
#include "lh_unicode_classes.h"
#include "lh_host_alloc.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define TK_ORDINARY 130072u
#define TK_SPECIALS 1000u
#define TK_MAX_TOKEN 1024u
#define TK_MAX_DECODE (4u << 20)
#define TK_MAX_VOCAB_BYTES (16u << 20)
#define TK_SLOTS (1u << 18)
#define TK_NONE 0xffffffffu

/* The supported pattern, byte for byte as the file's config stores it. */
static const char tk_pattern[] =
    "[^\\r\\n\\p{L}\\p{N}]?[\\p{Lu}\\p{Lt}\\p{Lm}\\p{Lo}\\p{M}]*"
    "[\\p{Ll}\\p{Lm}\\p{Lo}\\p{M}]+|"
    "[^\\r\\n\\p{L}\\p{N}]?[\\p{Lu}\\p{Lt}\\p{Lm}\\p{Lo}\\p{M}]+"
    "[\\p{Ll}\\p{Lm}\\p{Lo}\\p{M}]*|\\p{N}| ?[^\\s\\p{L}\\p{N}]+"
    "[\\r\\n/]*|\\s*[\\r\\n]+|\\s+(?!\\S)|\\s+";

static int fail(char *error, size_t size, const char *format, ...)
{
    if (error && size) {
        va_list args;
        va_start(args, format);
        vsnprintf(error, size, format, args);
        va_end(args);
    }
    return 0;
}

/* ---- strict UTF-8 ---- */

/* One scalar value at s (n bytes left): shortest form, no surrogates, at most
 * U+10FFFF. Returns its width, 0 when invalid. */
static size_t utf8_scalar(const unsigned char *s, size_t n, unsigned *cp)
{
    if (!n) {
        return 0;
    }
    const unsigned lead = s[0];
    if (lead < 0x80) {
        *cp = lead;
        return 1;
    }
    size_t width;
    unsigned value, minimum;
    if (lead >= 0xc2 && lead <= 0xdf) {
        width = 2, value = lead & 0x1f, minimum = 0x80;
    } else if (lead >= 0xe0 && lead <= 0xef) {
        width = 3, value = lead & 0x0f, minimum = 0x800;
    } else if (lead >= 0xf0 && lead <= 0xf4) {
        width = 4, value = lead & 0x07, minimum = 0x10000;
    } else {
        return 0;
    }
    if (n < width) {
        return 0;
    }
    for (size_t i = 1; i < width; i++) {
        if ((s[i] & 0xc0) != 0x80) {
            return 0;
        }
        value = value << 6 | (s[i] & 0x3f);
    }
    if (value < minimum || value > 0x10ffff || (value >= 0xd800 && value <= 0xdfff)) {
        return 0;
    }
    *cp = value;
    return width;
}

/* ---- bounded JSON ---- */

enum { J_MAX_FILE = 32u << 20, J_MAX_DEPTH = 32, J_MAX_NODES = 1500000u, J_MAX_STRING = 4096,
       J_MAX_MEMBERS = 64, J_MAX_ELEMENTS = 131072, J_MAX_SCALAR = 128 };

typedef struct {
    unsigned char *text;       /* decoded string, or the raw number/literal */
    uint32_t length;
    uint32_t child;            /* first element / first key (0: none) */
    uint32_t next;             /* next element / next key of the parent */
    uint32_t value;            /* for a key: its value */
    char kind;                 /* '{' '[' '"' '0' 't' 'f' 'n' */
} jnode;

typedef struct {
    unsigned char *data;
    size_t length, at;
    jnode *node;               /* node 0 is the missing-node sentinel */
    uint32_t count, capacity;
    int out_of_memory;         /* a node array could not grow */
} jdoc;

static void j_space(jdoc *d)
{
    while (d->at < d->length) {
        const unsigned char c = d->data[d->at];
        if (c != ' ' && c != '\t' && c != '\r' && c != '\n') {
            return;
        }
        d->at++;
    }
}

static uint32_t j_new(jdoc *d, char kind)
{
    if (d->count == J_MAX_NODES) {
        return 0;
    }
    if (d->count == d->capacity) {
        uint32_t capacity = d->capacity ? 2 * d->capacity : 4096;
        if (capacity > J_MAX_NODES) {
            capacity = J_MAX_NODES;
        }
        jnode *grown = lh_realloc(d->node, (size_t)capacity * sizeof(*grown));
        if (!grown) {
            d->out_of_memory = 1;
            return 0;
        }
        d->node = grown;
        d->capacity = capacity;
    }
    const uint32_t i = d->count++;
    memset(&d->node[i], 0, sizeof(d->node[i]));
    d->node[i].kind = kind;
    return i;
}

static int j_hex4(jdoc *d, unsigned *out)
{
    if (d->length - d->at < 4) {
        return 0;
    }
    unsigned v = 0;
    for (int i = 0; i < 4; i++) {
        const unsigned c = d->data[d->at++];
        const int digit = c >= '0' && c <= '9' ? (int)(c - '0') :
            c >= 'a' && c <= 'f' ? (int)(c - 'a' + 10) :
            c >= 'A' && c <= 'F' ? (int)(c - 'A' + 10) : -1;
        if (digit < 0) {
            return 0;
        }
        v = v << 4 | (unsigned)digit;
    }
    *out = v;
    return 1;
}

static size_t put_utf8(unsigned char *out, unsigned cp)
{
    if (cp < 0x80) {
        out[0] = (unsigned char)cp;
        return 1;
    }
    if (cp < 0x800) {
        out[0] = (unsigned char)(0xc0 | cp >> 6);
        out[1] = (unsigned char)(0x80 | (cp & 0x3f));
        return 2;
    }
    if (cp < 0x10000) {
        out[0] = (unsigned char)(0xe0 | cp >> 12);
        out[1] = (unsigned char)(0x80 | (cp >> 6 & 0x3f));
        out[2] = (unsigned char)(0x80 | (cp & 0x3f));
        return 3;
    }
    out[0] = (unsigned char)(0xf0 | cp >> 18);
    out[1] = (unsigned char)(0x80 | (cp >> 12 & 0x3f));
    out[2] = (unsigned char)(0x80 | (cp >> 6 & 0x3f));
    out[3] = (unsigned char)(0x80 | (cp & 0x3f));
    return 4;
}

/* A string at d->at (the opening quote), decoded in place: the decoded bytes
 * never outrun the source position. */
static int j_string(jdoc *d, uint32_t node)
{
    const size_t start = ++d->at;
    size_t out = start;
    for (;;) {
        if (out - start > J_MAX_STRING || d->at == d->length) {
            return 0;
        }
        unsigned c = d->data[d->at];
        if (c == '"') {
            d->at++;
            d->node[node].text = d->data + start;
            d->node[node].length = (uint32_t)(out - start);
            return 1;
        }
        if (c < 0x20) {
            return 0;
        }
        if (c >= 0x80) {
            unsigned cp;
            const size_t width = utf8_scalar(d->data + d->at, d->length - d->at, &cp);
            if (!width) {
                return 0;
            }
            memmove(d->data + out, d->data + d->at, width);
            out += width;
            d->at += width;
            continue;
        }
        d->at++;
        if (c != '\\') {
            d->data[out++] = (unsigned char)c;
            continue;
        }
        if (d->at == d->length) {
            return 0;
        }
        c = d->data[d->at++];
        static const char plain[] = "\"\\/bfnrt", decoded[] = "\"\\/\b\f\n\r\t";
        const char *hit = c ? strchr(plain, (int)c) : NULL;
        if (hit) {
            d->data[out++] = (unsigned char)decoded[hit - plain];
            continue;
        }
        if (c != 'u' || !j_hex4(d, &c)) {
            return 0;
        }
        if (c >= 0xdc00 && c <= 0xdfff) {
            return 0;
        }
        if (c >= 0xd800 && c <= 0xdbff) {
            unsigned low;
            if (d->length - d->at < 2 || d->data[d->at] != '\\' || d->data[d->at + 1] != 'u') {
                return 0;
            }
            d->at += 2;
            if (!j_hex4(d, &low) || low < 0xdc00 || low > 0xdfff) {
                return 0;
            }
            c = 0x10000 + ((c - 0xd800) << 10) + (low - 0xdc00);
        }
        out += put_utf8(d->data + out, c);
    }
}

static int j_digits(jdoc *d)
{
    const size_t first = d->at;
    while (d->at < d->length && d->data[d->at] >= '0' && d->data[d->at] <= '9') {
        d->at++;
    }
    return d->at > first;
}

/* A number (JSON grammar) or true/false/null at d->at. */
static int j_scalar(jdoc *d, uint32_t node)
{
    const size_t start = d->at;
    const unsigned char c = d->data[d->at];
    if (c == '-' || (c >= '0' && c <= '9')) {
        if (c == '-') {
            d->at++;
        }
        if (d->at == d->length || d->data[d->at] < '0' || d->data[d->at] > '9') {
            return 0;
        }
        if (d->data[d->at] == '0') {
            d->at++;
        } else {
            j_digits(d);
        }
        if (d->at < d->length && d->data[d->at] == '.') {
            d->at++;
            if (!j_digits(d)) {
                return 0;
            }
        }
        if (d->at < d->length && (d->data[d->at] == 'e' || d->data[d->at] == 'E')) {
            d->at++;
            if (d->at < d->length && (d->data[d->at] == '+' || d->data[d->at] == '-')) {
                d->at++;
            }
            if (!j_digits(d)) {
                return 0;
            }
        }
        d->node[node].kind = '0';
    } else {
        const char *word = c == 't' ? "true" : c == 'f' ? "false" : c == 'n' ? "null" : NULL;
        const size_t n = word ? strlen(word) : 0;
        if (!word || d->length - d->at < n || memcmp(d->data + d->at, word, n)) {
            return 0;
        }
        d->at += n;
    }
    if (d->at - start > J_MAX_SCALAR) {
        return 0;
    }
    d->node[node].text = d->data + start;
    d->node[node].length = (uint32_t)(d->at - start);
    return 1;
}

static uint32_t j_value(jdoc *d, int depth);

/* Members or elements of the container node up to its closing bracket. */
static int j_container(jdoc *d, uint32_t node, int depth)
{
    const int object = d->node[node].kind == '{';
    const unsigned char close = object ? '}' : ']';
    d->at++;
    j_space(d);
    if (d->at < d->length && d->data[d->at] == close) {
        d->at++;
        return 1;
    }
    uint32_t last = 0, members = 0;
    for (;;) {
        if (++members > (object ? J_MAX_MEMBERS : J_MAX_ELEMENTS)) {
            return 0;
        }
        uint32_t item = j_value(d, depth + 1);
        if (!item) {
            return 0;
        }
        if (object) {
            if (d->node[item].kind != '"') {
                return 0;
            }
            for (uint32_t k = d->node[node].child; k; k = d->node[k].next) {
                if (d->node[k].length == d->node[item].length &&
                    !memcmp(d->node[k].text, d->node[item].text, d->node[k].length)) {
                    return 0;
                }
            }
            j_space(d);
            if (d->at == d->length || d->data[d->at] != ':') {
                return 0;
            }
            d->at++;
            const uint32_t value = j_value(d, depth + 1);
            if (!value) {
                return 0;
            }
            d->node[item].value = value;
        }
        if (last) {
            d->node[last].next = item;
        } else {
            d->node[node].child = item;
        }
        last = item;
        j_space(d);
        if (d->at == d->length) {
            return 0;
        }
        const unsigned char c = d->data[d->at++];
        if (c == close) {
            return 1;
        }
        if (c != ',') {
            return 0;
        }
    }
}

static uint32_t j_value(jdoc *d, int depth)
{
    if (depth > J_MAX_DEPTH) {
        return 0;
    }
    j_space(d);
    if (d->at == d->length) {
        return 0;
    }
    const char c = (char)d->data[d->at];
    const uint32_t node = j_new(d, c);
    if (!node) {
        return 0;
    }
    const int ok = c == '"' ? j_string(d, node) :
        (c == '{' || c == '[') ? j_container(d, node, depth) : j_scalar(d, node);
    return ok ? node : 0;
}

static void j_free(jdoc *d)
{
    lh_free(d->data);
    lh_free(d->node);
    memset(d, 0, sizeof(*d));
}

/* Reads a whole file of at most 32 MiB holding exactly one value: 1, or 0
 * (unreadable, not JSON, past a limit), or -1 when memory ran out. */
static int j_parse(const char *path, jdoc *d);

static int j_read(const char *path, jdoc *d)
{
    const int ok = j_parse(path, d);
    if (ok) {
        return 1;
    }
    const int out_of_memory = d->out_of_memory;
    j_free(d);
    return out_of_memory ? -1 : 0;
}

static int j_parse(const char *path, jdoc *d)
{
    memset(d, 0, sizeof(*d));
    FILE *f = fopen(path, "rb");
    if (!f) {
        return 0;
    }
    long size = -1;
    if (!fseek(f, 0, SEEK_END)) {
        size = ftell(f);
    }
    if (size < 0 || (unsigned long)size > J_MAX_FILE || fseek(f, 0, SEEK_SET)) {
        fclose(f);
        return 0;
    }
    d->length = (size_t)size;
    d->data = lh_malloc(d->length + 1);
    d->out_of_memory = !d->data;
    const int read_ok = d->data && fread(d->data, 1, d->length, f) == d->length && !ferror(f);
    fclose(f);
    if (read_ok) {
        j_new(d, 0);                       /* the sentinel, node 0 */
    }
    if (!read_ok || d->count != 1 || j_value(d, 0) != 1) {
        return 0;
    }
    j_space(d);
    return d->at == d->length;
}

/* Value of key in the object node (0 when absent or not an object). */
static uint32_t j_field(const jdoc *d, uint32_t object, const char *key)
{
    if (!object || d->node[object].kind != '{') {
        return 0;
    }
    const size_t n = strlen(key);
    for (uint32_t k = d->node[object].child; k; k = d->node[k].next) {
        if (d->node[k].length == n && !memcmp(d->node[k].text, key, n)) {
            return d->node[k].value;
        }
    }
    return 0;
}

/* A number node of plain decimal digits that fits 32 bits. */
static int j_u32(const jdoc *d, uint32_t node, unsigned *out)
{
    if (!node || d->node[node].kind != '0' || !d->node[node].length) {
        return 0;
    }
    unsigned long long v = 0;
    for (uint32_t i = 0; i < d->node[node].length; i++) {
        const unsigned char c = d->node[node].text[i];
        if (c < '0' || c > '9') {
            return 0;
        }
        v = v * 10 + (unsigned)(c - '0');
        if (v > 0xffffffffull) {
            return 0;
        }
    }
    *out = (unsigned)v;
    return 1;
}

static int j_is_string(const jdoc *d, uint32_t node, const char *text)
{
    const size_t n = strlen(text);
    return node && d->node[node].kind == '"' && d->node[node].length == n &&
        !memcmp(d->node[node].text, text, n);
}

static int j_is_u32(const jdoc *d, uint32_t object, const char *key, unsigned want)
{
    unsigned v;
    return j_u32(d, j_field(d, object, key), &v) && v == want;
}

/* ---- vocabulary ---- */

struct lunelette_tokenizer {
    unsigned char *arena;               /* ordinary token bytes in rank order */
    uint32_t start[TK_ORDINARY + 1];    /* rank r: arena[start[r], start[r+1]) */
    uint32_t slot[TK_SLOTS];            /* rank + 1, 0 = empty */
};

static uint64_t fnv1a(const unsigned char *b, size_t n)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; i++) {
        h = (h ^ b[i]) * 0x100000001b3ull;
    }
    return h;
}

static unsigned tk_find(const lunelette_tokenizer *t, const unsigned char *b, size_t n)
{
    if (n > TK_MAX_TOKEN) {
        return TK_NONE;
    }
    for (uint32_t s = (uint32_t)fnv1a(b, n) & (TK_SLOTS - 1); t->slot[s];
         s = (s + 1) & (TK_SLOTS - 1)) {
        const uint32_t r = t->slot[s] - 1;
        if (t->start[r + 1] - t->start[r] == n && !memcmp(t->arena + t->start[r], b, n)) {
            return r;
        }
    }
    return TK_NONE;
}

static void tk_insert(lunelette_tokenizer *t, uint32_t rank)
{
    const unsigned char *b = t->arena + t->start[rank];
    uint32_t s = (uint32_t)fnv1a(b, t->start[rank + 1] - t->start[rank]) & (TK_SLOTS - 1);
    while (t->slot[s]) {
        s = (s + 1) & (TK_SLOTS - 1);
    }
    t->slot[s] = rank + 1;
}

static int b64_digit(unsigned c)
{
    return c >= 'A' && c <= 'Z' ? (int)(c - 'A') : c >= 'a' && c <= 'z' ? (int)(c - 'a' + 26) :
        c >= '0' && c <= '9' ? (int)(c - '0' + 52) : c == '+' ? 62 : c == '/' ? 63 : -1;
}

/* Canonical padded base64 of 1..1024 bytes: '=' only at the end, unused
 * bits zero. Writes at most 1024 bytes to out (NULL: length only). */
static int b64_decode(const jdoc *d, uint32_t node, unsigned char *out, size_t *length)
{
    if (!node || d->node[node].kind != '"') {
        return 0;
    }
    const unsigned char *s = d->node[node].text;
    const size_t n = d->node[node].length;
    if (!n || n % 4 || n > 4 * ((TK_MAX_TOKEN + 2) / 3)) {
        return 0;
    }
    size_t w = 0;
    for (size_t i = 0; i < n; i += 4) {
        const int last = i + 4 == n;
        const int a = b64_digit(s[i]), b = b64_digit(s[i + 1]);
        const int pad2 = s[i + 2] == '=', pad3 = s[i + 3] == '=';
        const int c = pad2 ? 0 : b64_digit(s[i + 2]), e = pad3 ? 0 : b64_digit(s[i + 3]);
        if (a < 0 || b < 0 || c < 0 || e < 0 || (pad2 && !pad3) || ((pad2 || pad3) && !last) ||
            (pad2 && (b & 15)) || (pad3 && !pad2 && (c & 3))) {
            return 0;
        }
        const unsigned char bytes[3] = {(unsigned char)(a << 2 | b >> 4),
            (unsigned char)((b & 15) << 4 | c >> 2), (unsigned char)((c & 3) << 6 | e)};
        const size_t k = pad2 ? 1 : pad3 ? 2 : 3;
        if (w + k > TK_MAX_TOKEN) {
            return 0;
        }
        if (out) {
            memcpy(out + w, bytes, k);
        }
        w += k;
    }
    *length = w;
    return 1;
}

void lunelette_tokenizer_close(lunelette_tokenizer *t)
{
    if (t) {
        lh_free(t->arena);
        lh_free(t);
    }
}

/* Ordinary ranks: pass 1 checks every entry and records its length by rank,
 * pass 2 decodes into the arena in rank order and fills the table. */
static int load_vocab(const jdoc *d, uint32_t vocab, lunelette_tokenizer *t, char *error,
    size_t size)
{
    uint32_t *node_of = lh_calloc(TK_ORDINARY, sizeof(*node_of));
    uint32_t *length_of = lh_calloc(TK_ORDINARY, sizeof(*length_of));
    int ok = 0;
    if (!node_of || !length_of) {
        fail(error, size, "tokenizer open: out of memory");
        goto done;
    }
    unsigned entries = 0;
    size_t total = 0;
    for (uint32_t e = d->node[vocab].child; e; e = d->node[e].next, entries++) {
        unsigned rank;
        size_t n;
        const uint32_t bytes = j_field(d, e, "token_bytes");
        if (!j_u32(d, j_field(d, e, "rank"), &rank) || rank >= TK_ORDINARY || node_of[rank] ||
            !b64_decode(d, bytes, NULL, &n)) {
            fail(error, size, "tokenizer open: vocabulary entry %u has a bad rank, bad base64 or a repeated rank",
                entries);
            goto done;
        }
        if (total > TK_MAX_VOCAB_BYTES - n) {
            fail(error, size, "tokenizer open: token bytes total more than 16 MiB");
            goto done;
        }
        node_of[rank] = bytes;
        length_of[rank] = (uint32_t)n;
        total += n;
    }
    if (entries != TK_ORDINARY) {
        fail(error, size, "tokenizer open: %u ordinary ranks where the format has 130072", entries);
        goto done;
    }
    t->arena = lh_malloc(total ? total : 1);
    if (!t->arena) {
        fail(error, size, "tokenizer open: out of memory");
        goto done;
    }
    t->start[0] = 0;
    for (uint32_t r = 0; r < TK_ORDINARY; r++) {
        size_t n;
        b64_decode(d, node_of[r], t->arena + t->start[r], &n);
        t->start[r + 1] = t->start[r] + (uint32_t)n;
        if (tk_find(t, t->arena + t->start[r], n) != TK_NONE) {
            fail(error, size, "tokenizer open: rank %u repeats the bytes of a lower rank", r);
            goto done;
        }
        tk_insert(t, r);
    }
    for (unsigned byte = 0; byte < 256; byte++) {
        const unsigned char b = (unsigned char)byte;
        if (tk_find(t, &b, 1) == TK_NONE) {
            fail(error, size, "tokenizer open: no single-byte token for byte %u", byte);
            goto done;
        }
    }
    ok = 1;
done:
    lh_free(node_of);
    lh_free(length_of);
    return ok;
}

/* Specials: 1000 entries, unique ranks and spellings, boolean is_control,
 * and the framing spellings the chat prompt relies on. */
static int check_specials(const jdoc *d, uint32_t specials, char *error, size_t size)
{
    uint32_t spelling[TK_SPECIALS] = {0};
    unsigned entries = 0;
    for (uint32_t e = d->node[specials].child; e; e = d->node[e].next, entries++) {
        unsigned rank;
        const uint32_t text = j_field(d, e, "token_str"), control = j_field(d, e, "is_control");
        if (!j_u32(d, j_field(d, e, "rank"), &rank) || rank >= TK_SPECIALS || spelling[rank] ||
            !text || d->node[text].kind != '"' || !d->node[text].length || !control ||
            (d->node[control].kind != 't' && d->node[control].kind != 'f')) {
            return fail(error, size, "tokenizer open: a special token has a bad or repeated rank or spelling");
        }
        for (unsigned r = 0; r < TK_SPECIALS; r++) {
            const uint32_t other = spelling[r];
            if (other && d->node[other].length == d->node[text].length &&
                !memcmp(d->node[other].text, d->node[text].text, d->node[text].length)) {
                return fail(error, size, "tokenizer open: two special tokens share a spelling");
            }
        }
        spelling[rank] = text;
    }
    static const struct { unsigned rank; const char *text; } framing[] = {
        {LUNELETTE_TOKEN_BOS, "<s>"}, {LUNELETTE_TOKEN_EOS, "</s>"},
        {LUNELETTE_TOKEN_INST, "[INST]"}, {LUNELETTE_TOKEN_END_INST, "[/INST]"},
        {LUNELETTE_TOKEN_SYSTEM, "[SYSTEM_PROMPT]"},
        {LUNELETTE_TOKEN_END_SYSTEM, "[/SYSTEM_PROMPT]"}};
    int framed = entries == TK_SPECIALS;
    for (size_t i = 0; i < sizeof(framing) / sizeof(framing[0]); i++) {
        framed &= j_is_string(d, spelling[framing[i].rank], framing[i].text);
    }
    return framed ? 1 :
        fail(error, size, "tokenizer open: the special tokens are not the 1000 of the format with its framing ids");
}

int lunelette_tokenizer_open(const char *path, lunelette_tokenizer **out, char *error,
    size_t error_size)
{
    if (!out) {
        return fail(error, error_size, "tokenizer open: no place for the handle");
    }
    *out = NULL;
    jdoc d;
    const int read = path ? j_read(path, &d) : 0;
    if (read < 0) {
        return fail(error, error_size, "tokenizer open %s: out of memory", path);
    }
    if (!read) {
        return fail(error, error_size, "tokenizer open %s: unreadable, not JSON, or past the reader's "
            "limits (32 MiB, nesting 32, 1500000 values)", path ? path : "(null)");
    }
    lunelette_tokenizer *t = NULL;
    int ok = 0;
    const uint32_t config = j_field(&d, 1, "config");
    if (!j_is_string(&d, j_field(&d, config, "version"), "v13") ||
        !j_is_string(&d, j_field(&d, config, "pattern"), tk_pattern) ||
        !j_is_u32(&d, config, "num_vocab_tokens", LUNELETTE_TOKENIZER_VOCAB_SIZE) ||
        !j_is_u32(&d, config, "default_vocab_size", LUNELETTE_TOKENIZER_VOCAB_SIZE) ||
        !j_is_u32(&d, config, "default_num_special_tokens", TK_SPECIALS)) {
        fail(error, error_size, "tokenizer open %s: config is not the Tekken v13 one this reader knows "
            "(version, pattern or vocabulary sizes)", path);
        goto done;
    }
    const uint32_t vocab = j_field(&d, 1, "vocab"), specials = j_field(&d, 1, "special_tokens");
    if (!vocab || d.node[vocab].kind != '[') {
        fail(error, error_size, "tokenizer open: the file has no vocab list");
        goto done;
    }
    t = lh_calloc(1, sizeof(*t));
    if (!t) {
        fail(error, error_size, "tokenizer open: out of memory");
        goto done;
    }
    if (!load_vocab(&d, vocab, t, error, error_size)) {
        goto done;
    }
    if (!specials || d.node[specials].kind != '[') {
        fail(error, error_size, "tokenizer open: the file has no special_tokens list");
        goto done;
    }
    ok = check_specials(&d, specials, error, error_size);
done:
    j_free(&d);
    if (!ok) {
        lunelette_tokenizer_close(t);
        return 0;
    }
    *out = t;
    return 1;
}

/* ---- pre-tokenizer ---- */

typedef struct {
    unsigned cp;
    unsigned mask;
    size_t offset;
} tk_char;

static unsigned class_of(unsigned cp)
{
    size_t lo = 0, hi = sizeof(lh_unicode_classes) / sizeof(lh_unicode_classes[0]);
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (cp < lh_unicode_classes[mid].first) {
            hi = mid;
        } else if (cp > lh_unicode_classes[mid].last) {
            lo = mid + 1;
        } else {
            return lh_unicode_classes[mid].mask;
        }
    }
    return 0;
}

static int is_crlf(unsigned cp)
{
    return cp == '\r' || cp == '\n';
}

/* [^\r\n\p{L}\p{N}] */
static int is_lead(const tk_char *c)
{
    return !is_crlf(c->cp) && !(c->mask & (LH_UC_LETTER | LH_UC_NUMBER));
}

static size_t run(const tk_char *c, size_t n, size_t at, unsigned mask)
{
    while (at < n && (c[at].mask & mask)) {
        at++;
    }
    return at;
}

/* UPPER* LOWER+ from p, UPPER* backtracking until a LOWER follows; 0 if none. */
static size_t upper_star_lower_plus(const tk_char *c, size_t n, size_t p)
{
    for (size_t k = run(c, n, p, LH_UC_UPPER);; k--) {
        if (k < n && (c[k].mask & LH_UC_LOWER)) {
            return run(c, n, k, LH_UC_LOWER);
        }
        if (k == p) {
            return 0;
        }
    }
}

/* UPPER+ LOWER* from p; 0 if no UPPER at p. */
static size_t upper_plus_lower_star(const tk_char *c, size_t n, size_t p)
{
    const size_t k = run(c, n, p, LH_UC_UPPER);
    return k > p ? run(c, n, k, LH_UC_LOWER) : 0;
}

/* End of the piece starting at s: the first alternative of the pattern that
 * matches there, with that alternative's own backtracking. */
static size_t piece_end(const tk_char *c, size_t n, size_t s)
{
    /* 1, 2: [lead]? UPPER* LOWER+ | [lead]? UPPER+ LOWER* (lead taken first). */
    for (int alt = 0; alt < 2; alt++) {
        size_t (*word)(const tk_char *, size_t, size_t) =
            alt ? upper_plus_lower_star : upper_star_lower_plus;
        if (is_lead(&c[s]) && s + 1 < n) {
            const size_t e = word(c, n, s + 1);
            if (e) {
                return e;
            }
        }
        const size_t e = word(c, n, s);
        if (e) {
            return e;
        }
    }
    /* 3: \p{N} */
    if (c[s].mask & LH_UC_NUMBER) {
        return s + 1;
    }
    /* 4: ' '? [^\s\p{L}\p{N}]+ [\r\n/]* */
    const unsigned other = LH_UC_SPACE | LH_UC_LETTER | LH_UC_NUMBER;
    for (size_t b = c[s].cp == ' ' ? s + 1 : s;; b = s) {
        size_t e = b;
        while (e < n && !(c[e].mask & other)) {
            e++;
        }
        if (e > b) {
            while (e < n && (is_crlf(c[e].cp) || c[e].cp == '/')) {
                e++;
            }
            return e;
        }
        if (b == s) {
            break;
        }
    }
    /* 5: \s* [\r\n]+ ends after the last CR/LF of the whitespace run. */
    const size_t space_end = run(c, n, s, LH_UC_SPACE);
    size_t after_crlf = s;
    for (size_t i = s; i < space_end; i++) {
        if (is_crlf(c[i].cp)) {
            after_crlf = i + 1;
        }
    }
    if (after_crlf > s) {
        return after_crlf;
    }
    /* 6: \s+(?!\S): the run to the end of text, or all but its last char. */
    if (space_end == n && space_end > s) {
        return space_end;
    }
    if (space_end > s + 1) {
        return space_end - 1;
    }
    /* 7: \s+ */
    return space_end;
}

/* Strict UTF-8 decode into classified characters; chars[n].offset = length. */
static tk_char *decode_text(const unsigned char *text, size_t length, size_t *count,
    size_t *bad_at)
{
    tk_char *chars = lh_malloc((length + 1) * sizeof(*chars));
    if (!chars) {
        *bad_at = (size_t)-1;
        return NULL;
    }
    size_t n = 0;
    for (size_t at = 0; at < length;) {
        unsigned cp;
        const size_t width = utf8_scalar(text + at, length - at, &cp);
        if (!width) {
            lh_free(chars);
            *bad_at = at;
            return NULL;
        }
        chars[n].cp = cp;
        chars[n].mask = class_of(cp);
        chars[n++].offset = at;
        at += width;
    }
    chars[n].offset = length;
    *count = n;
    return chars;
}

long lunelette_tokenizer_split(const unsigned char *text, size_t length, size_t *ends,
    size_t capacity)
{
    if ((!text && length) || !ends || length > LUNELETTE_TOKENIZER_LONG_INPUT) {
        return -1;
    }
    size_t n, bad;
    tk_char *chars = decode_text(text, length, &n, &bad);
    if (!chars) {
        return -1;
    }
    long pieces = 0;
    for (size_t s = 0; s < n;) {
        const size_t e = piece_end(chars, n, s);
        if (e <= s || e > n || (size_t)pieces == capacity) {
            lh_free(chars);
            return -1;
        }
        ends[pieces++] = chars[e].offset;
        s = e;
    }
    lh_free(chars);
    return pieces;
}

/* ---- byte-pair merges ---- */

typedef struct {
    uint32_t rank, left, stamp;
} merge_entry;

static int entry_before(const merge_entry *a, const merge_entry *b)
{
    return a->rank < b->rank || (a->rank == b->rank && a->left < b->left);
}

static void heap_push(merge_entry *h, size_t *n, merge_entry e)
{
    size_t i = (*n)++;
    while (i && entry_before(&e, &h[(i - 1) / 2])) {
        h[i] = h[(i - 1) / 2];
        i = (i - 1) / 2;
    }
    h[i] = e;
}

static merge_entry heap_pop(merge_entry *h, size_t *n)
{
    const merge_entry top = h[0], last = h[--*n];
    size_t i = 0;
    for (;;) {
        size_t child = 2 * i + 1;
        if (child >= *n) {
            break;
        }
        if (child + 1 < *n && entry_before(&h[child + 1], &h[child])) {
            child++;
        }
        if (!entry_before(&h[child], &last)) {
            break;
        }
        h[i] = h[child];
        i = child;
    }
    if (*n) {
        h[i] = last;
    }
    return top;
}

/* Ids of one piece appended at out + *count. Parts are byte ranges
 * [p, end[p]) linked by next/prev; a heap entry (rank, left, stamp) is current
 * while left is alive with that stamp (every merge touching left's pair
 * bumps it). */
static int merge_piece(const lunelette_tokenizer *t, const unsigned char *b, size_t n,
    uint32_t *out, size_t *count)
{
    const unsigned whole = tk_find(t, b, n);
    if (whole != TK_NONE) {
        out[(*count)++] = whole + TK_SPECIALS;
        return 1;
    }
    if (!n) {
        return 1;
    }
    size_t *end = lh_malloc(n * sizeof(*end)), *next = lh_malloc(n * sizeof(*next));
    size_t *prev = lh_malloc(n * sizeof(*prev));
    uint32_t *stamp = lh_calloc(n, sizeof(*stamp));
    merge_entry *heap = lh_malloc(3 * n * sizeof(*heap));
    int ok = end && next && prev && stamp && heap;
    if (ok) {
        size_t queued = 0;
        for (size_t i = 0; i < n; i++) {
            end[i] = i + 1;
            next[i] = i + 1;
            prev[i] = i ? i - 1 : n;
        }
        for (size_t i = 0; i + 1 < n; i++) {
            const unsigned r = tk_find(t, b + i, 2);
            if (r != TK_NONE) {
                heap_push(heap, &queued, (merge_entry){r, (uint32_t)i, 0});
            }
        }
        while (queued) {
            const merge_entry e = heap_pop(heap, &queued);
            const size_t left = e.left;
            if (e.stamp != stamp[left] || next[left] >= n) {
                continue;                      /* stale: the pair has changed */
            }
            const size_t right = next[left];
            end[left] = end[right];
            next[left] = next[right];
            if (next[left] < n) {
                prev[next[left]] = left;
            }
            next[right] = n + 1;                /* right is gone */
            stamp[left]++;
            if (next[left] < n) {
                const unsigned r = tk_find(t, b + left, end[next[left]] - left);
                if (r != TK_NONE) {
                    heap_push(heap, &queued, (merge_entry){r, (uint32_t)left, stamp[left]});
                }
            }
            const size_t before = prev[left];
            if (before < n) {
                stamp[before]++;
                const unsigned r = tk_find(t, b + before, end[left] - before);
                if (r != TK_NONE) {
                    heap_push(heap, &queued, (merge_entry){r, (uint32_t)before, stamp[before]});
                }
            }
        }
        for (size_t i = 0; i < n; i = next[i]) {
            out[(*count)++] = tk_find(t, b + i, end[i] - i) + TK_SPECIALS;
        }
    }
    lh_free(end);
    lh_free(next);
    lh_free(prev);
    lh_free(stamp);
    lh_free(heap);
    return ok;
}

/* ---- encode / decode ---- */

int lunelette_tokenizer_encode(const lunelette_tokenizer *t, const unsigned char *text,
    size_t length, uint32_t **ids, size_t *count, char *error, size_t error_size)
{
    return lunelette_tokenizer_encode_with_limit(t, text, length, LUNELETTE_TOKENIZER_MAX_INPUT,
        ids, count, error, error_size);
}

int lunelette_tokenizer_encode_with_limit(const lunelette_tokenizer *t,
    const unsigned char *text, size_t length, size_t input_limit, uint32_t **ids,
    size_t *count, char *error, size_t error_size)
{
    if (ids) {
        *ids = NULL;
    }
    if (count) {
        *count = 0;
    }
    if (!t || !ids || !count || (!text && length) ||
        (input_limit != LUNELETTE_TOKENIZER_MAX_INPUT &&
         input_limit != LUNELETTE_TOKENIZER_LONG_INPUT) || length > input_limit) {
        return fail(error, error_size, "tokenizer encode: bad arguments, or the text is longer than "
            "%u bytes", input_limit == LUNELETTE_TOKENIZER_LONG_INPUT ?
            LUNELETTE_TOKENIZER_LONG_INPUT : LUNELETTE_TOKENIZER_MAX_INPUT);
    }
    size_t n, bad;
    tk_char *chars = decode_text(text, length, &n, &bad);
    if (!chars) {
        return bad == (size_t)-1 ? fail(error, error_size, "tokenizer encode: out of memory") :
            fail(error, error_size, "tokenizer encode: invalid UTF-8 at byte %zu", bad);
    }
    uint32_t *result = lh_malloc((length ? length : 1) * sizeof(*result));
    size_t produced = 0;
    int ok = result != NULL;
    for (size_t s = 0; ok && s < n;) {
        const size_t e = piece_end(chars, n, s);
        if (e <= s || e > n) {
            ok = 0;
            break;
        }
        ok = merge_piece(t, text + chars[s].offset, chars[e].offset - chars[s].offset, result,
            &produced);
        s = e;
    }
    lh_free(chars);
    if (!ok) {
        lh_free(result);
        return fail(error, error_size, "tokenizer encode: out of memory");
    }
    *ids = result;
    *count = produced;
    return 1;
}

int lunelette_tokenizer_decode(const lunelette_tokenizer *t, const uint32_t *ids, size_t count,
    unsigned char **bytes, size_t *length, char *error, size_t error_size)
{
    if (bytes) {
        *bytes = NULL;
    }
    if (length) {
        *length = 0;
    }
    if (!t || !bytes || !length || (!ids && count) || count > LUNELETTE_TOKENIZER_MAX_INPUT) {
        return fail(error, error_size, "tokenizer decode: bad arguments or more than 4096 ids");
    }
    size_t total = 0;
    for (size_t i = 0; i < count; i++) {
        if (ids[i] < TK_SPECIALS || ids[i] >= LUNELETTE_TOKENIZER_VOCAB_SIZE) {
            return fail(error, error_size, "tokenizer decode: id %u at %zu is a special token or "
                "outside the vocabulary", ids[i], i);
        }
        const uint32_t r = ids[i] - TK_SPECIALS;
        const size_t n = t->start[r + 1] - t->start[r];
        if (n > TK_MAX_DECODE - total) {
            return fail(error, error_size, "tokenizer decode: the text would pass 4 MiB");
        }
        total += n;
    }
    unsigned char *result = lh_malloc(total + 1);
    if (!result) {
        return fail(error, error_size, "tokenizer decode: out of memory");
    }
    size_t at = 0;
    for (size_t i = 0; i < count; i++) {
        const uint32_t r = ids[i] - TK_SPECIALS;
        memcpy(result + at, t->arena + t->start[r], t->start[r + 1] - t->start[r]);
        at += t->start[r + 1] - t->start[r];
    }
    result[total] = 0;
    *bytes = result;
    *length = total;
    return 1;
}
