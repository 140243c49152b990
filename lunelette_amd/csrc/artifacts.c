/* Native logit-regression artifacts (LUN1/LUN2): writer, reader, strict
 * comparison and the capture/check runs over a runtime context (behaviour of
 * tests/compare_native.c:22-194 and :348-450). Host code only; the files are
 * little-endian and this library only builds for little-endian IEEE hosts,
 * so a vector is read and written as one block of binary32 words. */
#define _POSIX_C_SOURCE 200809L
#include "lunelette_artifacts.h"
#include "lunelette_generation.h"
#include "lh_scan.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define VOCAB LUNELETTE_VOCAB_SIZE
#define STEPS LUNELETTE_NATIVE_STEPS

_Static_assert(sizeof(float) == 4, "binary32 logits");

static int failed(char *error, size_t capacity, const char *format, ...)
{
    if (error && capacity) {
        va_list args;
        va_start(args, format);
        vsnprintf(error, capacity, format, args);
        va_end(args);
    }
    return 1;
}

/* Rank order of the top-64 list: higher value first, equal values by lower
 * index (an empty slot ranks last). The list is filled in index order, so a
 * candidate enters before the first entry it outranks; entries below shift
 * down and the 64th drops out. While every entry is finite the list stays
 * sorted, and a candidate below the last entry cannot enter anywhere. */
void lunelette_logits_top64(const float *values, size_t count, size_t ids[64])
{
    for (int k = 0; k < 64; k++) {
        ids[k] = count;
    }
    int sorted = 1;
    for (size_t i = 0; i < count; i++) {
        const float v = values[i];
        if (sorted && ids[63] != count && isfinite(v) && v < values[ids[63]]) {
            continue;
        }
        for (int k = 0; k < 64; k++) {
            const size_t at = ids[k];
            if (at == count || v > values[at] || (v == values[at] && i < at)) {
                memmove(ids + k + 1, ids + k, (size_t)(63 - k) * sizeof(*ids));
                ids[k] = i;
                sorted &= isfinite(v) != 0;
                break;
            }
        }
    }
}

static size_t shared(const size_t *a, const size_t *b, size_t k)
{
    size_t n = 0;
    for (size_t i = 0; i < k; i++) {
        for (size_t j = 0; j < k; j++) {
            n += a[i] == b[j];
        }
    }
    return n;
}

int lunelette_logits_compare(const float *a, const float *b, size_t count,
    lunelette_logit_metrics *m)
{
    lunelette_logit_metrics local;
    if (!m) {
        m = &local;
    }
    memset(m, 0, sizeof(*m));
    double square = 0.0, aa = 0.0, bb = 0.0, ab = 0.0;
    for (size_t i = 0; i < count; i++) {
        m->finite_a += isfinite(a[i]) != 0;
        m->finite_b += isfinite(b[i]) != 0;
        const double d = (double)a[i] - (double)b[i];
        m->max_abs = fmax(m->max_abs, fabs(d));
        square += d * d;
        aa += (double)a[i] * a[i];
        bb += (double)b[i] * b[i];
        ab += (double)a[i] * b[i];
    }
    size_t top_a[64], top_b[64];
    lunelette_logits_top64(a, count, top_a);
    lunelette_logits_top64(b, count, top_b);
    m->exact = memcmp(a, b, count * sizeof(float)) == 0;
    m->top1_a = top_a[0];
    m->top1_b = top_b[0];
    m->top5 = shared(top_a, top_b, 5);
    m->top20 = shared(top_a, top_b, 20);
    m->top64 = shared(top_a, top_b, 64);
    m->rms = count ? sqrt(square / (double)count) : 0.0;
    m->cosine = aa != 0.0 && bb != 0.0 ? ab / sqrt(aa * bb) : (m->exact ? 1.0 : 0.0);
    const int accepted = m->finite_a == count && m->finite_b == count && m->exact &&
        m->top1_a == m->top1_b && m->top5 == 5 && m->top20 == 20 && m->top64 == 64;
    return !accepted;
}

static void put_u32(unsigned char *at, uint32_t v)
{
    at[0] = (unsigned char)v;
    at[1] = (unsigned char)(v >> 8);
    at[2] = (unsigned char)(v >> 16);
    at[3] = (unsigned char)(v >> 24);
}

static uint32_t get_u32(const unsigned char *at)
{
    return (uint32_t)at[0] | (uint32_t)at[1] << 8 | (uint32_t)at[2] << 16 |
        (uint32_t)at[3] << 24;
}

static int read_words(FILE *f, uint32_t *out, size_t n)
{
    unsigned char bytes[4 * 64];
    while (n) {
        const size_t k = n < 64 ? n : 64;
        if (fread(bytes, 4, k, f) != k) {
            return 1;
        }
        for (size_t i = 0; i < k; i++) {
            *out++ = get_u32(bytes + 4 * i);
        }
        n -= k;
    }
    return 0;
}

/* Header words for a trajectory: magic, [strategy], mode, 256, count, 8,
 * vocabulary, prompt ids, forced ids. */
static size_t encode_header(const lunelette_native_trajectory *t, uint32_t *w)
{
    size_t n = 0;
    w[n++] = t->magic;
    if (t->magic == LUNELETTE_NATIVE_LUN2) {
        w[n++] = (uint32_t)t->strategy;
    }
    w[n++] = t->mode;
    w[n++] = LUNELETTE_NATIVE_CONTEXT;
    w[n++] = (uint32_t)t->count;
    w[n++] = STEPS;
    w[n++] = VOCAB;
    for (size_t i = 0; i < t->count; i++) {
        w[n++] = (uint32_t)t->ids[i];
    }
    for (size_t i = 0; i < STEPS; i++) {
        w[n++] = (uint32_t)t->forced[i];
    }
    return n;
}

static int trajectory_valid(const lunelette_native_trajectory *t)
{
    if (!t || !t->count || t->count > LUNELETTE_NATIVE_MAX_PROMPT || t->mode > 1 ||
        (unsigned)t->strategy > LUNELETTE_METAL_COMPACT_FP8_LOOKUP) {
        return 0;
    }
    for (size_t i = 0; i < t->count; i++) {
        if (t->ids[i] < 0 || t->ids[i] >= VOCAB) {
            return 0;
        }
    }
    for (size_t i = 0; i < STEPS; i++) {
        if (t->forced[i] < 0 || t->forced[i] >= VOCAB) {
            return 0;
        }
    }
    return 1;
}

/* Reads one header and checks it against the trajectory: either format, the
 * strategy word (LUN1: resident) equal to the trajectory's, every fixed field
 * and every id equal. */
static int check_header(FILE *f, const lunelette_native_trajectory *t, char *error,
    size_t capacity)
{
    uint32_t magic;
    if (read_words(f, &magic, 1) ||
        (magic != LUNELETTE_NATIVE_LUN1 && magic != LUNELETTE_NATIVE_LUN2)) {
        return failed(error, capacity, "artifact: unknown format");
    }
    uint32_t strategy = 0;
    if (magic == LUNELETTE_NATIVE_LUN2 && read_words(f, &strategy, 1)) {
        return failed(error, capacity, "artifact: truncated header");
    }
    if (strategy > 2 || strategy != (uint32_t)t->strategy) {
        return failed(error, capacity, "artifact: strategy mismatch or invalid strategy");
    }
    lunelette_native_trajectory expected = *t;
    expected.magic = magic;
    uint32_t want[7 + LUNELETTE_NATIVE_MAX_PROMPT + STEPS];
    uint32_t got[7 + LUNELETTE_NATIVE_MAX_PROMPT + STEPS];
    const size_t n = encode_header(&expected, want);
    const size_t skip = magic == LUNELETTE_NATIVE_LUN2 ? 2 : 1;
    if (read_words(f, got + skip, n - skip)) {
        return failed(error, capacity, "artifact: truncated header");
    }
    for (size_t i = skip; i < n; i++) {
        if (got[i] != want[i]) {
            return failed(error, capacity, "artifact: header word %zu differs", i);
        }
    }
    return 0;
}

/* One vector of binary32 logits; every value must be finite. */
static int read_vector(FILE *f, float *v)
{
    return fread(v, sizeof(float), VOCAB, f) != VOCAB ||
        lh_first_nonfinite(v, VOCAB) < VOCAB;
}

static int write_vector(FILE *f, const float *v)
{
    return lh_first_nonfinite(v, VOCAB) < VOCAB || fwrite(v, sizeof(float), VOCAB, f) != VOCAB;
}

static FILE *create_artifact(const char *path, const lunelette_native_trajectory *t,
    char *error, size_t capacity)
{
    if (!path || !trajectory_valid(t) ||
        (t->magic != LUNELETTE_NATIVE_LUN1 && t->magic != LUNELETTE_NATIVE_LUN2) ||
        (t->magic == LUNELETTE_NATIVE_LUN1 && t->strategy != LUNELETTE_METAL_RESIDENT_FP32)) {
        failed(error, capacity, "artifact: invalid trajectory or format (LUN1 is resident only)");
        return NULL;
    }
    FILE *f = fopen(path, "wbx");
    if (!f) {
        failed(error, capacity, "artifact: cannot create %s (it must not exist)", path);
        return NULL;
    }
    uint32_t words[7 + LUNELETTE_NATIVE_MAX_PROMPT + STEPS];
    unsigned char bytes[4 * (7 + LUNELETTE_NATIVE_MAX_PROMPT + STEPS)];
    const size_t n = encode_header(t, words);
    for (size_t i = 0; i < n; i++) {
        put_u32(bytes + 4 * i, words[i]);
    }
    if (fwrite(bytes, 4, n, f) != n) {
        fclose(f);
        failed(error, capacity, "artifact: header write failed");
        return NULL;
    }
    return f;
}

int lunelette_native_write(const char *path, const lunelette_native_trajectory *t,
    const float *logits, char *error, size_t capacity)
{
    if (!logits) {
        return failed(error, capacity, "artifact: require logits");
    }
    FILE *f = create_artifact(path, t, error, capacity);
    if (!f) {
        return 1;
    }
    int bad = 0;
    for (size_t s = 0; s < STEPS && !bad; s++) {
        bad = write_vector(f, logits + s * VOCAB);
    }
    bad |= fclose(f) != 0;
    return bad ? failed(error, capacity, "artifact: nonfinite logit or write failure") : 0;
}

int lunelette_native_read(const char *path, const lunelette_native_trajectory *t,
    float *logits, char *error, size_t capacity)
{
    if (!path || !trajectory_valid(t)) {
        return failed(error, capacity, "artifact: require a path and a valid trajectory");
    }
    FILE *f = fopen(path, "rb");
    if (!f) {
        return failed(error, capacity, "artifact: cannot open %s", path);
    }
    float *scratch = logits ? NULL : malloc(VOCAB * sizeof(float));
    int status = check_header(f, t, error, capacity);
    for (size_t s = 0; s < STEPS && !status; s++) {
        if (!logits && !scratch) {
            status = failed(error, capacity, "artifact: out of host memory");
        } else if (read_vector(f, logits ? logits + s * VOCAB : scratch)) {
            status = failed(error, capacity, "artifact: step %zu truncated or nonfinite", s);
        }
    }
    if (!status && (fgetc(f) != EOF || ferror(f))) {
        status = failed(error, capacity, "artifact: trailing bytes");
    }
    free(scratch);
    fclose(f);
    return status;
}

int lunelette_native_compare_files(const char *left, const char *right, uint32_t mode,
    size_t count, lunelette_metal_strategy strategy, lunelette_logit_metrics *metrics,
    char *error, size_t capacity)
{
    if (!left || !right || !count || count > LUNELETTE_NATIVE_MAX_PROMPT || mode > 1 ||
        (unsigned)strategy > LUNELETTE_METAL_COMPACT_FP8_LOOKUP) {
        return failed(error, capacity, "artifact: require files, mode 0/1, count 1..248");
    }
    FILE *a = fopen(left, "rb"), *b = fopen(right, "rb");
    float *av = malloc(VOCAB * sizeof(float)), *bv = malloc(VOCAB * sizeof(float));
    int status = 1;
    if (!a || !b || !av || !bv) {
        failed(error, capacity, "artifact: cannot open both files");
        goto done;
    }
    /* The trajectory is the left file's own; both headers must carry it. */
    uint32_t magic, words[LUNELETTE_NATIVE_MAX_PROMPT + STEPS];
    if (read_words(a, &magic, 1) ||
        (magic != LUNELETTE_NATIVE_LUN1 && magic != LUNELETTE_NATIVE_LUN2) ||
        fseek(a, magic == LUNELETTE_NATIVE_LUN2 ? 28 : 24, SEEK_SET) ||
        read_words(a, words, count + STEPS)) {
        failed(error, capacity, "artifact: unreadable left header");
        goto done;
    }
    rewind(a);
    lunelette_native_trajectory t = {.magic = magic, .strategy = strategy, .mode = mode,
        .count = count};
    for (size_t i = 0; i < count + STEPS; i++) {
        const int64_t id = (int64_t)words[i];
        if (i < count) {
            t.ids[i] = id;
        } else {
            t.forced[i - count] = id;
        }
    }
    if (!trajectory_valid(&t)) {
        failed(error, capacity, "artifact: token outside the vocabulary");
        goto done;
    }
    if (check_header(a, &t, error, capacity) || check_header(b, &t, error, capacity)) {
        goto done;
    }
    for (size_t s = 0; s < STEPS; s++) {
        if (read_vector(a, av) || read_vector(b, bv)) {
            failed(error, capacity, "artifact: step %zu truncated or nonfinite", s);
            goto done;
        }
        if (lunelette_logits_compare(av, bv, VOCAB, metrics ? metrics + s : NULL)) {
            failed(error, capacity, "artifact: step %zu differs", s);
            goto done;
        }
    }
    status = fgetc(a) != EOF || fgetc(b) != EOF || ferror(a) || ferror(b);
    if (status) {
        failed(error, capacity, "artifact: trailing bytes");
    }
done:
    if (a) {
        fclose(a);
    }
    if (b) {
        fclose(b);
    }
    free(av);
    free(bv);
    return status;
}

/* One step of the trajectory: the prefill of the prompt (step 0) or the
 * decode of forced[step - 1]. */
static int run_step(lunelette_metal *rt, const lunelette_native_trajectory *t, size_t step,
    const float **logits, char *error, size_t capacity)
{
    if (step == 0) {
        return lunelette_metal_prefill(rt, t->ids, t->count, logits, error, capacity);
    }
    return lunelette_metal_decode(rt, t->forced[step - 1], logits, error, capacity);
}

int lunelette_native_run(lunelette_metal *rt, const char *path,
    const lunelette_native_trajectory *t, int check, lunelette_logit_metrics *metrics,
    char *error, size_t capacity)
{
    lunelette_metal_memory memory;
    lunelette_metal_limits limits;
    if (!rt || !path || !trajectory_valid(t)) {
        return failed(error, capacity, "artifact: require a runtime, a path and a trajectory");
    }
    if (lunelette_metal_get_memory(rt, &memory) || memory.strategy != t->strategy) {
        return failed(error, capacity, "artifact: runtime strategy differs from the request");
    }
    if (lunelette_metal_get_limits(rt, &limits) || limits.block < t->count ||
        limits.context < t->count + STEPS - 1) {
        return failed(error, capacity, "artifact: runtime limits too small for the trajectory");
    }
    if (!check) {
        FILE *f = create_artifact(path, t, error, capacity);
        if (!f) {
            return 1;
        }
        int status = lunelette_metal_reset(rt, error, capacity);
        for (size_t s = 0; s < STEPS && !status; s++) {
            const float *logits = NULL;
            status = run_step(rt, t, s, &logits, error, capacity);
            if (!status && write_vector(f, logits)) {
                status = failed(error, capacity, "artifact: step %zu not written", s);
            }
        }
        if (fclose(f) && !status) {
            status = failed(error, capacity, "artifact: close failed");
        }
        return status;
    }
    /* Validate the whole file before any model work, then two reset cycles. */
    lunelette_native_trajectory any = *t;
    if (lunelette_native_read(path, &any, NULL, error, capacity)) {
        return 1;
    }
    float *expected = malloc(VOCAB * sizeof(float));
    if (!expected) {
        return failed(error, capacity, "artifact: out of host memory");
    }
    int status = 0;
    for (int cycle = 0; cycle < 2 && !status; cycle++) {
        FILE *f = fopen(path, "rb");
        status = !f ? failed(error, capacity, "artifact: cannot reopen %s", path) :
            check_header(f, t, error, capacity);
        if (!status) {
            status = lunelette_metal_reset(rt, error, capacity);
        }
        for (size_t s = 0; s < STEPS && !status; s++) {
            const float *logits = NULL;
            status = run_step(rt, t, s, &logits, error, capacity);
            if (!status && read_vector(f, expected)) {
                status = failed(error, capacity, "artifact: step %zu unreadable", s);
            }
            if (!status && lunelette_logits_compare(logits, expected, VOCAB,
                    metrics ? metrics + cycle * STEPS + s : NULL)) {
                status = failed(error, capacity, "artifact: cycle %d step %zu differs", cycle, s);
            }
        }
        if (f) {
            fclose(f);
        }
    }
    free(expected);
    return status;
}
