/* Safetensors container reader and the checkpoint tensor contract.
 *
 * Container (behaviour of src/safetensors.c:9-424): an 8-byte little-endian
 * header length n (2 <= n <= 1 MiB, within the file), an n-byte JSON object
 * starting with '{', then the data section. Accepted grammar, scanned left to
 * right without recursion:
 *   - top level: name -> tensor object, or "__metadata__" -> object of
 *     string -> string (at most once, at most 64 unique keys);
 *   - strings: printable ASCII after decoding; escapes \" \\ \/ and \uXXXX
 *     (which must decode to printable ASCII); names non-empty, < 256 chars,
 *     unique; metadata values < 4096 chars;
 *   - tensor object: exactly the keys dtype (F8_E4M3, BF16, F32, I64), shape
 *     (at most 8 unsigned integers) and data_offsets (two), each once, any
 *     order; integers are plain decimal without leading zeros or overflow;
 *   - whitespace: space, \n, \r, \t between tokens; nothing after the object.
 * Layout: every size is overflow-checked and equals the element count times
 * the element size; the non-empty tensors tile the data section exactly (no
 * gap, overlap or trailing byte); an empty tensor may not start strictly
 * inside another tensor.
 *
 * Contract (behaviour of src/metal_weights.c:9-150): the embedding, the final
 * norm and 9 tensors per layer with the names and shapes of
 * src/model_facts.c; each FP8 matrix has BF16 rank-0 companions
 * <prefix>weight_scale_inv and <prefix>activation_scale, both positive and
 * finite; the first is the per-tensor scale, the second is only validated.
 * Any other language_model.* tensor is rejected; other prefixes (vision
 * tower, projector) are ignored.
 */
#define _POSIX_C_SOURCE 200809L
#include "lh_weights.h"
#include "lunelette_weights.h"

#include <limits.h>
#include <math.h>
#include <stdbool.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- header grammar ---- */

typedef struct {
    const unsigned char *at, *end;
} scan;

static void skip_space(scan *s)
{
    while (s->at < s->end &&
        (*s->at == ' ' || *s->at == '\n' || *s->at == '\r' || *s->at == '\t')) {
        s->at++;
    }
}

/* Consumes ch after optional whitespace. */
static bool take(scan *s, unsigned char ch)
{
    skip_space(s);
    if (s->at < s->end && *s->at == ch) {
        s->at++;
        return true;
    }
    return false;
}

static int hex_digit(unsigned char c)
{
    if (c >= '0' && c <= '9') {
        return c - '0';
    }
    if (c >= 'a' && c <= 'f') {
        return c - 'a' + 10;
    }
    if (c >= 'A' && c <= 'F') {
        return c - 'A' + 10;
    }
    return -1;
}

/* A JSON string of at most cap - 1 printable ASCII characters into out. */
static bool take_string(scan *s, char *out, size_t cap)
{
    if (!take(s, '"')) {
        return false;
    }
    size_t length = 0;
    while (s->at < s->end) {
        unsigned ch = *s->at++;
        if (ch == '"') {
            out[length] = '\0';
            return true;
        }
        if (ch == '\\') {
            if (s->at == s->end) {
                return false;
            }
            ch = *s->at++;
            if (ch == 'u') {
                unsigned code = 0;
                for (int k = 0; k < 4; k++) {
                    const int digit = s->at < s->end ? hex_digit(*s->at++) : -1;
                    if (digit < 0) {
                        return false;
                    }
                    code = code * 16 + (unsigned)digit;
                }
                ch = code;
            } else if (ch != '"' && ch != '\\' && ch != '/') {
                return false;
            }
        }
        if (ch < 32 || ch > 126 || length + 1 >= cap) {
            return false;
        }
        out[length++] = (char)ch;
    }
    return false;
}

static bool take_u64(scan *s, uint64_t *out)
{
    skip_space(s);
    if (s->at == s->end || *s->at < '0' || *s->at > '9') {
        return false;
    }
    const bool leading_zero = *s->at == '0';
    uint64_t value = 0;
    size_t digits = 0;
    while (s->at < s->end && *s->at >= '0' && *s->at <= '9') {
        const unsigned d = *s->at - '0';
        if (value > (UINT64_MAX - d) / 10 || (leading_zero && digits == 1)) {
            return false;
        }
        value = value * 10 + d;
        digits++;
        s->at++;
    }
    *out = value;
    return true;
}

/* [a, b, ...] with at most cap entries. */
static bool take_u64_list(scan *s, uint64_t *out, size_t cap, size_t *count)
{
    *count = 0;
    if (!take(s, '[')) {
        return false;
    }
    if (take(s, ']')) {
        return true;
    }
    for (;;) {
        if (*count == cap || !take_u64(s, &out[*count])) {
            return false;
        }
        (*count)++;
        if (take(s, ']')) {
            return true;
        }
        if (!take(s, ',')) {
            return false;
        }
    }
}

static bool take_dtype(scan *s, lh_st_dtype *out)
{
    static const struct {
        const char *text;
        lh_st_dtype dtype;
    } known[] = {{"F8_E4M3", LH_ST_F8_E4M3}, {"BF16", LH_ST_BF16}, {"F32", LH_ST_F32},
        {"I64", LH_ST_I64}};
    char text[16];
    if (!take_string(s, text, sizeof text)) {
        return false;
    }
    for (size_t i = 0; i < sizeof known / sizeof known[0]; i++) {
        if (!strcmp(text, known[i].text)) {
            *out = known[i].dtype;
            return true;
        }
    }
    return false;
}

static bool take_tensor(scan *s, lh_st_tensor *t)
{
    enum { DTYPE = 1, SHAPE = 2, OFFSETS = 4 };
    unsigned seen = 0;
    if (!take(s, '{')) {
        return false;
    }
    for (;;) {
        char key[LH_ST_MAX_NAME];
        unsigned field;
        if (!take_string(s, key, sizeof key) || !take(s, ':')) {
            return false;
        }
        if (!strcmp(key, "dtype")) {
            field = DTYPE;
            if (!take_dtype(s, &t->dtype)) {
                return false;
            }
        } else if (!strcmp(key, "shape")) {
            size_t rank;
            field = SHAPE;
            if (!take_u64_list(s, t->shape, LH_ST_MAX_DIMS, &rank)) {
                return false;
            }
            t->rank = (uint32_t)rank;
        } else if (!strcmp(key, "data_offsets")) {
            uint64_t range[2];
            size_t n;
            field = OFFSETS;
            if (!take_u64_list(s, range, 2, &n) || n != 2) {
                return false;
            }
            t->begin = range[0];
            t->end = range[1];
        } else {
            return false;
        }
        if (seen & field) {
            return false;
        }
        seen |= field;
        if (take(s, '}')) {
            return seen == (DTYPE | SHAPE | OFFSETS);
        }
        if (!take(s, ',')) {
            return false;
        }
    }
}

static bool take_metadata(scan *s)
{
    char keys[64][LH_ST_MAX_NAME];
    char value[4096];
    size_t n = 0;
    if (!take(s, '{')) {
        return false;
    }
    if (take(s, '}')) {
        return true;
    }
    for (;;) {
        if (n == 64 || !take_string(s, keys[n], sizeof keys[n])) {
            return false;
        }
        for (size_t i = 0; i < n; i++) {
            if (!strcmp(keys[i], keys[n])) {
                return false;
            }
        }
        n++;
        if (!take(s, ':') || !take_string(s, value, sizeof value)) {
            return false;
        }
        if (take(s, '}')) {
            return true;
        }
        if (!take(s, ',')) {
            return false;
        }
    }
}

static int parse_header(lh_st_file *f, const unsigned char *header, size_t length)
{
    scan s = {header, header + length};
    bool metadata = false;
    if (header[0] != '{' || !take(&s, '{')) {
        return -1;
    }
    if (!take(&s, '}')) {
        for (;;) {
            char name[LH_ST_MAX_NAME];
            if (!take_string(&s, name, sizeof name) || !name[0] || !take(&s, ':')) {
                return -1;
            }
            if (!strcmp(name, "__metadata__")) {
                if (metadata || !take_metadata(&s)) {
                    return -1;
                }
                metadata = true;
            } else {
                if (f->count == LH_ST_MAX_TENSORS || lh_st_find(f, name)) {
                    return -1;
                }
                lh_st_tensor *t = &f->tensors[f->count];
                memcpy(t->name, name, strlen(name) + 1);
                if (!take_tensor(&s, t)) {
                    return -1;
                }
                f->count++;
            }
            if (take(&s, '}')) {
                break;
            }
            if (!take(&s, ',')) {
                return -1;
            }
        }
    }
    skip_space(&s);
    return s.at == s.end ? 0 : -1;
}

/* ---- data layout ---- */

/* Byte size of a tensor from its dtype and shape: every dimension at most
 * INT64_MAX, a zero dimension makes it empty, and neither the element count
 * nor the byte count may overflow 64 bits. */
static int tensor_bytes(const lh_st_tensor *t, uint64_t *bytes)
{
    uint64_t elements = 1;
    bool empty = false;
    for (uint32_t k = 0; k < t->rank; k++) {
        if (t->shape[k] > (uint64_t)INT64_MAX) {
            return -1;
        }
        empty = empty || t->shape[k] == 0;
    }
    for (uint32_t k = 0; k < t->rank && !empty; k++) {
        if (elements > UINT64_MAX / t->shape[k]) {
            return -1;
        }
        elements *= t->shape[k];
    }
    if (empty) {
        elements = 0;
    }
    if (elements > UINT64_MAX / (uint64_t)t->dtype) {
        return -1;
    }
    *bytes = elements * (uint64_t)t->dtype;
    return 0;
}

static int by_begin(const void *a, const void *b)
{
    const lh_st_tensor *x = *(const lh_st_tensor *const *)a;
    const lh_st_tensor *y = *(const lh_st_tensor *const *)b;
    return x->begin < y->begin ? -1 : (x->begin > y->begin);
}

/* The data section must be tiled exactly by the non-empty tensors: sorted by
 * offset, the first starts at 0, each starts where the previous ends (so two
 * at one offset fail), and the last ends at the section's end. An empty
 * tensor may sit at any tile boundary but not strictly inside a tile. Every
 * tensor's byte range must match its dtype and shape and lie in the section. */
static int check_layout(const lh_st_file *f, uint64_t data_bytes)
{
    const lh_st_tensor **tiles = malloc((f->count ? f->count : 1) * sizeof *tiles);
    if (!tiles) {
        return -1;
    }
    size_t n = 0;
    int status = -1;
    for (size_t i = 0; i < f->count; i++) {
        const lh_st_tensor *t = &f->tensors[i];
        uint64_t bytes;
        if (tensor_bytes(t, &bytes) || t->end < t->begin || t->end > data_bytes ||
            t->end - t->begin != bytes) {
            goto done;
        }
        if (bytes) {
            tiles[n++] = t;
        }
    }
    qsort(tiles, n, sizeof *tiles, by_begin);
    uint64_t expected = 0;
    for (size_t i = 0; i < n; i++) {
        if (tiles[i]->begin != expected) {
            goto done;
        }
        expected = tiles[i]->end;
    }
    if (expected != data_bytes) {
        goto done;
    }
    for (size_t i = 0; i < f->count; i++) {
        const lh_st_tensor *t = &f->tensors[i];
        if (t->begin != t->end || n == 0) {
            continue;
        }
        /* Last tile starting at or before the empty tensor's offset. */
        size_t lo = 0, hi = n;
        while (hi - lo > 1) {
            const size_t mid = lo + (hi - lo) / 2;
            if (tiles[mid]->begin <= t->begin) {
                lo = mid;
            } else {
                hi = mid;
            }
        }
        if (tiles[lo]->begin < t->begin && t->begin < tiles[lo]->end) {
            goto done;
        }
    }
    status = 0;
done:
    free(tiles);
    return status;
}

/* ---- container API ---- */

void lh_st_close(lh_st_file *f)
{
    if (!f) {
        return;
    }
    if (f->file) {
        fclose(f->file);
    }
    free(f->tensors);
    memset(f, 0, sizeof *f);
}

const lh_st_tensor *lh_st_find(const lh_st_file *f, const char *name)
{
    if (!f || !name) {
        return NULL;
    }
    for (size_t i = 0; i < f->count; i++) {
        if (!strcmp(f->tensors[i].name, name)) {
            return &f->tensors[i];
        }
    }
    return NULL;
}

int lh_st_open(lh_st_file *f, const char *path, char *error, size_t capacity)
{
    const char *why = "invalid arguments";
    unsigned char *header = NULL;
    if (!f) {
        goto report;
    }
    memset(f, 0, sizeof *f);
    if (!path) {
        goto fail;
    }
    why = "cannot open or size the file (a seekable file of at most LONG_MAX bytes)";
    f->file = fopen(path, "rb");
    if (!f->file || fseek(f->file, 0, SEEK_END)) {
        goto fail;
    }
    const long size = ftell(f->file);
    if (size < 8 || fseek(f->file, 0, SEEK_SET)) {
        goto fail;
    }
    why = "header length missing, truncated or above 1 MiB";
    unsigned char prefix[8];
    if (fread(prefix, 1, 8, f->file) != 8) {
        goto fail;
    }
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) {
        n = n << 8 | prefix[i];
    }
    if (n < 2 || n > LH_ST_MAX_HEADER || n > (uint64_t)size - 8) {
        goto fail;
    }
    f->base = 8 + n;
    why = "allocation failure";
    header = malloc((size_t)n);
    f->tensors = calloc(LH_ST_MAX_TENSORS, sizeof *f->tensors);
    if (!header || !f->tensors) {
        goto fail;
    }
    why = "truncated header";
    if (fread(header, 1, (size_t)n, f->file) != n) {
        goto fail;
    }
    why = "invalid header: unique printable-ASCII names, dtypes F8_E4M3/BF16/F32/I64, "
        "rank <= 8, plain JSON";
    if (parse_header(f, header, (size_t)n)) {
        goto fail;
    }
    why = "tensor sizes/offsets do not tile the data section";
    if (check_layout(f, (uint64_t)size - f->base)) {
        goto fail;
    }
    free(header);
    if (error && capacity) {
        error[0] = '\0';
    }
    return 0;
fail:
    free(header);
    lh_st_close(f);
report:
    if (error && capacity) {
        snprintf(error, capacity, "safetensors: %s", why);
    }
    return -1;
}

int lh_st_read(lh_st_file *f, const lh_st_tensor *t, uint64_t offset, void *out, size_t bytes)
{
    if (!f || !f->file || !t || (!out && bytes) || t < f->tensors ||
        t >= f->tensors + f->count) {
        return -1;
    }
    const uint64_t size = t->end - t->begin;
    if (offset > size || bytes > size - offset) {
        return -1;
    }
    const uint64_t position = f->base + t->begin + offset;
    if (position > (uint64_t)LONG_MAX || fseek(f->file, (long)position, SEEK_SET)) {
        return -1;
    }
    return !bytes || fread(out, 1, bytes, f->file) == bytes ? 0 : -1;
}

/* ---- checkpoint contract ---- */

static const struct {
    const char *suffix;
    size_t rows, cols;              /* cols 0: a vector */
} block_tensor[9] = {
    {"input_layernorm.weight", LH_HIDDEN, 0},
    {"self_attn.q_proj.weight", LH_QUERY, LH_HIDDEN},
    {"self_attn.k_proj.weight", LH_KV, LH_HIDDEN},
    {"self_attn.v_proj.weight", LH_KV, LH_HIDDEN},
    {"self_attn.o_proj.weight", LH_HIDDEN, LH_QUERY},
    {"post_attention_layernorm.weight", LH_HIDDEN, 0},
    {"mlp.gate_proj.weight", LH_INNER, LH_HIDDEN},
    {"mlp.up_proj.weight", LH_INNER, LH_HIDDEN},
    {"mlp.down_proj.weight", LH_HIDDEN, LH_INNER},
};

static const char *const companion_suffix[2] = {"weight_scale_inv", "activation_scale"};

/* name ends in "weight"; out = name without it + suffix. */
static void companion_name(const char *name, const char *suffix, char out[LH_ST_MAX_NAME])
{
    snprintf(out, LH_ST_MAX_NAME, "%.*s%s", (int)(strlen(name) - 6), name, suffix);
}

static float bf16_value(const unsigned char bytes[2])
{
    const uint32_t word = ((uint32_t)bytes[1] << 24) | ((uint32_t)bytes[0] << 16);
    float value;
    memcpy(&value, &word, sizeof value);
    return value;
}

static int expect_tensor(lh_weights *w, size_t slot, const char *name, size_t rows, size_t cols,
    char *error, size_t capacity)
{
    const lh_st_tensor *t = lh_st_find(&w->file, name);
    const bool matrix = cols != 0 && slot != 0;
    const lh_st_dtype dtype = matrix ? LH_ST_F8_E4M3 : LH_ST_BF16;
    if (!t || t->dtype != dtype || t->rank != (cols ? 2u : 1u) || t->shape[0] != rows ||
        (cols && t->shape[1] != cols)) {
        if (cols) {
            snprintf(error, capacity, "tensor %s: expected %s [%zu,%zu]", name,
                matrix ? "F8_E4M3" : "BF16", rows, cols);
        } else {
            snprintf(error, capacity, "tensor %s: expected BF16 [%zu]", name, rows);
        }
        return -1;
    }
    if (matrix) {
        for (int k = 0; k < 2; k++) {
            char companion[LH_ST_MAX_NAME];
            companion_name(name, companion_suffix[k], companion);
            const lh_st_tensor *c = lh_st_find(&w->file, companion);
            if (!c || c->dtype != LH_ST_BF16 || c->rank != 0 || c->end - c->begin != 2) {
                snprintf(error, capacity, "scalar %s: expected BF16 rank 0", companion);
                return -1;
            }
        }
    }
    w->slot[slot].tensor = t;
    w->slot[slot].scale = 1.0f;
    return 0;
}

static int check_contract(lh_weights *w, char *error, size_t capacity)
{
    if (expect_tensor(w, 0, "language_model.model.embed_tokens.weight", LH_VOCAB, LH_HIDDEN,
            error, capacity) ||
        expect_tensor(w, 1, "language_model.model.norm.weight", LH_HIDDEN, 0, error, capacity)) {
        return -1;
    }
    for (size_t layer = 0; layer < LH_LAYERS; layer++) {
        for (size_t i = 0; i < 9; i++) {
            char name[LH_ST_MAX_NAME];
            snprintf(name, sizeof name, "language_model.model.layers.%zu.%s", layer,
                block_tensor[i].suffix);
            if (expect_tensor(w, 2 + 9 * layer + i, name, block_tensor[i].rows,
                    block_tensor[i].cols, error, capacity)) {
                return -1;
            }
        }
    }
    for (size_t i = 0; i < w->file.count; i++) {
        const char *name = w->file.tensors[i].name;
        if (strncmp(name, "language_model.", 15) != 0) {
            continue;
        }
        bool known = false;
        for (size_t s = 0; s < LH_WEIGHT_SLOTS && !known; s++) {
            const lh_st_tensor *t = w->slot[s].tensor;
            known = !strcmp(name, t->name);
            for (int k = 0; k < 2 && !known && t->dtype == LH_ST_F8_E4M3; k++) {
                char companion[LH_ST_MAX_NAME];
                companion_name(t->name, companion_suffix[k], companion);
                known = !strcmp(name, companion);
            }
        }
        if (!known) {
            snprintf(error, capacity, "unexpected text tensor: %s", name);
            return -1;
        }
    }
    return 0;
}

static int read_scales(lh_weights *w, char *error, size_t capacity)
{
    for (size_t s = 0; s < LH_WEIGHT_SLOTS; s++) {
        const lh_st_tensor *t = w->slot[s].tensor;
        if (t->dtype != LH_ST_F8_E4M3) {
            continue;
        }
        for (int k = 0; k < 2; k++) {
            char companion[LH_ST_MAX_NAME];
            companion_name(t->name, companion_suffix[k], companion);
            unsigned char bytes[2];
            const lh_st_tensor *c = lh_st_find(&w->file, companion);
            const float value = lh_st_read(&w->file, c, 0, bytes, 2) ? NAN : bf16_value(bytes);
            if (!isfinite(value) || !(value > 0)) {
                snprintf(error, capacity, "scalar %s: expected positive finite BF16", companion);
                return -1;
            }
            if (k == 0) {
                w->slot[s].scale = value;
            }
        }
    }
    return 0;
}

void lh_weights_close(lh_weights *w)
{
    if (w) {
        lh_st_close(&w->file);
        memset(w, 0, sizeof *w);
    }
}

int lh_weights_open(lh_weights *w, const char *path, char *error, size_t capacity)
{
    char fallback[512];
    if (!error || !capacity) {
        error = fallback;
        capacity = sizeof fallback;
    }
    if (!w) {
        snprintf(error, capacity, "weights: missing handle");
        return -1;
    }
    memset(w, 0, sizeof *w);
    if (!path) {
        snprintf(error, capacity, "requires one explicit FP8 safetensors path");
        return -1;
    }
    if (lh_st_open(&w->file, path, error, capacity) || check_contract(w, error, capacity) ||
        read_scales(w, error, capacity)) {
        lh_weights_close(w);
        return -1;
    }
    return 0;
}

/* ---- inspection seams (ABI, include/lunelette_kernels.h) ---- */

static const char *dtype_text(lh_st_dtype dtype)
{
    switch (dtype) {
    case LH_ST_F8_E4M3: return "F8_E4M3";
    case LH_ST_BF16: return "BF16";
    case LH_ST_F32: return "F32";
    default: return "I64";
    }
}

int lh_st_inspect(const char *path, char *listing, size_t listing_capacity, char *error,
    size_t capacity)
{
    lh_st_file f;
    if (lh_st_open(&f, path, error, capacity)) {
        return -1;
    }
    size_t used = 0;
    int rc = 0;
    if (listing && listing_capacity) {
        listing[0] = '\0';
    }
    for (size_t i = 0; i < f.count && listing && listing_capacity; i++) {
        const lh_st_tensor *t = &f.tensors[i];
        char dims[8 * 21 + 1] = "";
        size_t d = 0;
        for (uint32_t k = 0; k < t->rank; k++) {
            d += (size_t)snprintf(dims + d, sizeof dims - d, "%s%llu", k ? "," : "",
                (unsigned long long)t->shape[k]);
        }
        const int n = snprintf(listing + used, listing_capacity - used, "%s|%s|%u|%s|%llu|%llu\n",
            t->name, dtype_text(t->dtype), t->rank, dims, (unsigned long long)t->begin,
            (unsigned long long)t->end);
        if (n < 0 || (size_t)n >= listing_capacity - used) {
            rc = -1;
            if (error && capacity) {
                snprintf(error, capacity, "listing buffer too small");
            }
            break;
        }
        used += (size_t)n;
    }
    lh_st_close(&f);
    return rc;
}

int lh_st_read_tensor(const char *path, const char *name, uint64_t offset, void *out,
    size_t bytes, char *error, size_t capacity)
{
    lh_st_file f;
    if (lh_st_open(&f, path, error, capacity)) {
        return -1;
    }
    const lh_st_tensor *t = lh_st_find(&f, name);
    const int rc = t ? lh_st_read(&f, t, offset, out, bytes) : -1;
    if (rc && error && capacity) {
        snprintf(error, capacity, t ? "read out of bounds or failed" : "no such tensor");
    }
    lh_st_close(&f);
    return rc;
}

int lh_checkpoint_check(const char *path, float *scales, char *error, size_t capacity)
{
    lh_weights *w = malloc(sizeof *w);
    if (!w) {
        if (error && capacity) {
            snprintf(error, capacity, "allocation failure");
        }
        return -1;
    }
    const int rc = lh_weights_open(w, path, error, capacity);
    if (!rc && scales) {
        for (size_t s = 0; s < LH_WEIGHT_SLOTS; s++) {
            scales[s] = w->slot[s].scale;
        }
    }
    lh_weights_close(w);
    free(w);
    return rc;
}

/* include/lunelette_weights.h: the metadata handle of src/metal_weights.h for
 * callers that validate a checkpoint without creating a runtime. */
int lunelette_metal_weights_open(lunelette_metal_weights *weights, const char *path,
    char *error, size_t capacity)
{
    char fallback[512];
    if (!error || !capacity) {
        error = fallback;
        capacity = sizeof fallback;
    }
    if (!weights) {
        snprintf(error, capacity, "checkpoint metadata needs a handle");
        return -1;
    }
    weights->opened = NULL;
    lh_weights *w = malloc(sizeof *w);
    if (!w) {
        snprintf(error, capacity, "checkpoint handle allocation failed");
        return -1;
    }
    if (lh_weights_open(w, path, error, capacity)) {
        free(w);
        return -1;
    }
    weights->opened = w;
    return 0;
}

void lunelette_metal_weights_close(lunelette_metal_weights *weights)
{
    if (weights && weights->opened) {
        lh_weights_close(weights->opened);
        free(weights->opened);
    }
    if (weights) {
        weights->opened = NULL;
    }
}
