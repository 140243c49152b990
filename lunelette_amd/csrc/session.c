/* Native session adapter: the service's model-facing state machine over the
 * runtime C-ABI (behaviour of service/native.c:19-34 state, 65-117
 * lifecycle, 161-327 materialize/save/restore, 336-416 selection and capture,
 * 431-560 admission). Host code only: every device operation goes through
 * lunelette_metal_* and the borrowed host logits it returns.
 *
 * Sequence state. prefix[0..length) is what the runtime holds in its KV
 * cache. After a selection the chosen token is pending: the next materialize
 * must begin with it, and until it is committed no new selection or save is
 * allowed. A materialize request toward a longer target becomes an ingestion
 * of one runtime block per call; the ingestion keeps its target fixed until
 * it completes or fails.
 *
 * Reuse policies (service/native.c:180-200):
 *   legacy: rebuild from an empty sequence unless the request appends exactly
 *           the pending non-EOS token;
 *   on:     extend the committed prefix; restore rewinds to the checkpoint;
 *   off:    rebuild at every generation boundary (begin), and restore drops
 *           the sequence so the next materialize recomputes the saved prefix.
 */
#define _POSIX_C_SOURCE 200809L
#include "lunelette_session.h"
#include "lunelette_generation.h"
#include "lh_scan.h"

#include <fcntl.h>
#include <float.h>
#include <inttypes.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#define SESSION_MAX LUNELETTE_LONG_CONTEXT_LIMIT
#define REPLAY_MAGIC "LNRPLY1"   /* eight bytes with the terminating zero */

struct lunelette_session {
    lunelette_metal *runtime;
    lunelette_metal_checkpoint *checkpoint;
    const float *logits;            /* borrowed from the runtime; NULL when stale */
    unsigned capacity, block, policy;
    unsigned length;                /* committed prefix length */
    int pending;                    /* a selected token awaits materialization */
    unsigned emitted;
    int ingesting, rebuilding, boundary;
    unsigned target, pending_position, recompute_length, recompute_hint;
    unsigned saved_length;
    lunelette_session_work work;
    FILE *replay;
    unsigned replay_index;
    int replay_failed;
    uint32_t *record;               /* staging of one capture record */
    char error[512];
    char info[2048];
    unsigned prefix[SESSION_MAX];
    unsigned saved_prefix[SESSION_MAX];
};

static void fail_text(char *error, size_t capacity, const char *format, ...)
{
    if (error && capacity) {
        va_list args;
        va_start(args, format);
        vsnprintf(error, capacity, format, args);
        va_end(args);
    }
}

static double now_seconds(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + t.tv_nsec * 1e-9;
}

/* The capture format is little-endian IEEE binary32 (service/native.c:419-429
 * refuses other hosts); on such a host a record is the in-memory words. */
static int host_is_le_ieee(void)
{
    const float probe[2] = {1.0f, -2.5f};
    uint32_t bits[2];
    memcpy(bits, probe, sizeof(bits));
    const uint16_t one = 1;
    unsigned char low;
    memcpy(&low, &one, 1);
    return sizeof(float) == 4 && FLT_RADIX == 2 && FLT_MANT_DIG == 24 && FLT_MAX_EXP == 128 &&
        bits[0] == UINT32_C(0x3f800000) && bits[1] == UINT32_C(0xc0200000) && low == 1;
}

static int options_valid(const lunelette_session_options *o)
{
    return o && (o->context == LUNELETTE_CONTEXT_LIMIT ||
                 o->context == LUNELETTE_LONG_CONTEXT_LIMIT) &&
        (o->block == 256 || o->block == 128) &&
        !(o->context == LUNELETTE_CONTEXT_LIMIT && o->block != 256) &&
        (unsigned)o->prefix_reuse <= LUNELETTE_SESSION_REUSE_OFF &&
        (!o->replay_path || o->replay_path[0]);
}

static const char *strategy_name(lunelette_metal_strategy strategy)
{
    return strategy == LUNELETTE_METAL_RESIDENT_FP32 ? "resident-fp32" :
        strategy == LUNELETTE_METAL_COMPACT_FP8_LOOKUP ? "compact-fp8-lookup" :
        "compact-fp8-arithmetic";
}

static void release(lunelette_session *s)
{
    if (!s) {
        return;
    }
    lunelette_metal_checkpoint_destroy(s->checkpoint);
    lunelette_metal_destroy(s->runtime);
    if (s->replay) {
        fclose(s->replay);
    }
    free(s->record);
    free(s);
}

/* Allocates the session and, in replay mode, creates the capture file with
 * its 16-byte header (magic, vocabulary, record limit). */
static lunelette_session *allocate(const lunelette_session_options *o, char *error,
    size_t capacity)
{
    lunelette_session *s = calloc(1, sizeof(*s));
    if (!s) {
        fail_text(error, capacity, "session: out of host memory");
        return NULL;
    }
    s->capacity = (unsigned)o->context;
    s->block = (unsigned)o->block;
    s->policy = (unsigned)o->prefix_reuse;
    if (!o->replay_path) {
        return s;
    }
    const size_t words = 4 + SESSION_MAX + LUNELETTE_VOCAB_SIZE;
    s->record = malloc(words * sizeof(uint32_t));
    int fd = open(o->replay_path, O_WRONLY | O_CREAT | O_EXCL, 0600);
    if (!s->record || fd < 0) {
        fail_text(error, capacity, "session: cannot create replay capture %s", o->replay_path);
        if (fd >= 0) {
            close(fd);
        }
        release(s);
        return NULL;
    }
    s->replay = fdopen(fd, "wb");
    if (!s->replay) {
        close(fd);
        fail_text(error, capacity, "session: cannot open replay capture stream");
        release(s);
        return NULL;
    }
    const uint32_t header[2] = {LUNELETTE_VOCAB_SIZE, LUNELETTE_SESSION_REPLAY_TOKENS};
    if (fwrite(REPLAY_MAGIC, 1, 8, s->replay) != 8 ||
        fwrite(header, sizeof(uint32_t), 2, s->replay) != 2 || fflush(s->replay)) {
        fail_text(error, capacity, "session: cannot write the replay capture header");
        release(s);
        return NULL;
    }
    return s;
}

/* The runtime half of the info object of service/native.c:562-616. */
static int describe(lunelette_session *s, const lunelette_metal_memory *m,
    lunelette_metal_prefill_mode prefill, double load_ms)
{
    const int replay = s->replay != NULL;
    const char *policy = s->policy == LUNELETTE_SESSION_REUSE_ON ? "on" :
        s->policy == LUNELETTE_SESSION_REUSE_OFF ? "off" : "legacy";
    int written = snprintf(s->info, sizeof(s->info),
        "{\"generator\":\"%s\",%s\"model_loaded\":true,\"runtime_ready\":true,"
        "\"model_load_count\":1,\"loading_duration_ms\":%.3f,"
        "\"execution_strategy\":\"%s\",\"prefill\":\"%s\","
        "\"context_capacity\":%u,\"prefill_chunk_size\":%u,"
        "\"checkpoint_payload_bytes_per_handle\":%u,"
        "\"checkpoints\":%s,\"reuse_new_turn\":%s,\"prefix_reuse\":\"%s\","
        "\"named_resident_weight_bytes\":%" PRIu64 ",\"named_conversion_stage_bytes\":%" PRIu64 ","
        "\"named_scratch_bytes\":%" PRIu64 ",\"named_kv_bytes\":%" PRIu64 ","
        "\"named_buffer_total_bytes\":%" PRIu64 ",\"device\":\"gfx950\"}",
        replay ? "native_controlled_replay" : "native_greedy",
        replay ? "\"evaluation_mode\":\"controlled_replay\",\"replay_max_tokens\":16,"
                 "\"replay_capture_limit\":16," : "",
        load_ms, strategy_name(m->strategy),
        prefill == LUNELETTE_METAL_PREFILL_MPS ? "mps" : "custom",
        s->capacity, s->block, (unsigned)(LUNELETTE_VOCAB_SIZE * sizeof(float)),
        s->policy ? "true" : "false", s->policy == LUNELETTE_SESSION_REUSE_ON ? "true" : "false",
        policy, m->weight_bytes, m->conversion_stage_bytes, m->scratch_bytes, m->kv_bytes,
        m->total_bytes);
    return written > 0 && (size_t)written < sizeof(s->info);
}

/* Shared tail of open and adopt: the runtime must report the requested
 * strategy and the session's limits (a valid but different strategy is not
 * a fallback, service/native.c:551-557). */
static lunelette_session *attach(lunelette_session *s, lunelette_metal *runtime,
    lunelette_metal_strategy expected, lunelette_metal_prefill_mode prefill, double load_ms,
    char *error, size_t capacity)
{
    s->runtime = runtime;
    lunelette_metal_memory memory;
    lunelette_metal_limits limits;
    if (lunelette_metal_get_memory(runtime, &memory) || memory.strategy != expected) {
        fail_text(error, capacity, "session: runtime strategy/allocation accounting query "
            "failed or strategy mismatch");
        release(s);
        return NULL;
    }
    if (lunelette_metal_get_limits(runtime, &limits) || limits.context != s->capacity ||
        limits.block != s->block) {
        fail_text(error, capacity, "session: runtime limits differ from the session's");
        release(s);
        return NULL;
    }
    if (!describe(s, &memory, prefill, load_ms)) {
        fail_text(error, capacity, "session: info exceeds its fixed capacity");
        release(s);
        return NULL;
    }
    return s;
}

lunelette_session *lunelette_session_open(const char *model,
    const lunelette_metal_options *runtime, const lunelette_session_options *options,
    char *error, size_t capacity)
{
    if (!model || !runtime || !options_valid(options) ||
        (options->replay_path && !host_is_le_ieee())) {
        fail_text(error, capacity, "session: require model, runtime options, context 256 or "
            "4352, block 256 or 128 (256 at context 256), policy 0..2");
        return NULL;
    }
    lunelette_session *s = allocate(options, error, capacity);
    if (!s) {
        return NULL;
    }
    const lunelette_metal_limits limits = {options->context, options->block};
    const double start = now_seconds();
    lunelette_metal *rt = lunelette_metal_create_configured(model, runtime, &limits, error,
        capacity);
    if (!rt) {
        release(s);
        return NULL;
    }
    return attach(s, rt, runtime->strategy, runtime->prefill, (now_seconds() - start) * 1e3,
        error, capacity);
}

lunelette_session *lunelette_session_adopt(lunelette_metal *runtime,
    const lunelette_metal_options *created, const lunelette_session_options *options,
    char *error, size_t capacity)
{
    if (!runtime || !created || !options_valid(options) ||
        (options->replay_path && !host_is_le_ieee())) {
        fail_text(error, capacity, "session: require a runtime, context 256 or 4352, block "
            "256 or 128 (256 at context 256), policy 0..2");
        lunelette_metal_destroy(runtime);
        return NULL;
    }
    lunelette_session *s = allocate(options, error, capacity);
    if (!s) {
        lunelette_metal_destroy(runtime);
        return NULL;
    }
    return attach(s, runtime, created->strategy, created->prefill, 0.0, error, capacity);
}

void lunelette_session_destroy(lunelette_session *s)
{
    if (s) {
        lunelette_session_invalidate(s);
        release(s);
    }
}

void lunelette_session_invalidate(lunelette_session *s)
{
    lunelette_metal_checkpoint_destroy(s->checkpoint);
    s->checkpoint = NULL;
    s->saved_length = 0;
    s->recompute_hint = 0;
    s->ingesting = 0;
    s->logits = NULL;
    s->pending = 0;
    s->emitted = 0;
}

void lunelette_session_begin(lunelette_session *s)
{
    s->boundary = 1;
}

void lunelette_session_take_work(lunelette_session *s, lunelette_session_work *work)
{
    *work = s->work;
    memset(&s->work, 0, sizeof(s->work));
}

void lunelette_session_reset(lunelette_session *s)
{
    lunelette_session_invalidate(s);
    s->length = 0;
    s->boundary = 0;
    s->error[0] = '\0';
    lunelette_metal_reset(s->runtime, s->error, sizeof(s->error));
}

/* A request may only extend the committed prefix, and while a selected token
 * is pending (outside an ingestion) it must continue with that token. */
static int admissible(const lunelette_session *s, const unsigned *tokens, unsigned length)
{
    if (!tokens || !length || length > s->capacity || length < s->length ||
        memcmp(s->prefix, tokens, s->length * sizeof(*tokens))) {
        return 0;
    }
    return s->ingesting || !s->pending ||
        (length > s->length && tokens[s->length] == s->emitted);
}

/* Opens an ingestion toward length and decides whether it rebuilds from an
 * empty sequence. Returns 0 when the runtime reset fails. */
static int open_ingestion(lunelette_session *s, unsigned length)
{
    const unsigned committed = s->length;
    const int continues_pending = s->pending && length == committed + 1 &&
        s->emitted != LUNELETTE_SESSION_EOS;
    s->rebuilding = !committed ||
        (s->policy == LUNELETTE_SESSION_REUSE_OFF && s->boundary) ||
        (s->policy == LUNELETTE_SESSION_REUSE_LEGACY && !continues_pending);
    s->target = length;
    s->pending_position = committed;
    s->recompute_length = s->rebuilding ? committed : 0;
    if (s->recompute_hint > s->recompute_length) {
        s->recompute_length = s->recompute_hint;
    }
    s->recompute_hint = 0;
    s->boundary = 0;
    s->work.reused = s->rebuilding ? 0 : committed;
    if (s->rebuilding) {
        s->logits = NULL;
        if (lunelette_metal_reset(s->runtime, s->error, sizeof(s->error))) {
            return 0;
        }
        s->length = 0;
    }
    s->ingesting = 1;
    return 1;
}

int lunelette_session_materialize(lunelette_session *s, const unsigned *tokens,
    unsigned length)
{
    memset(&s->work, 0, sizeof(s->work));
    s->error[0] = '\0';
    if (!admissible(s, tokens, length)) {
        return 0;
    }
    if (!s->ingesting && length == s->length &&
        !(s->policy == LUNELETTE_SESSION_REUSE_OFF && s->boundary)) {
        /* Nothing to run: the committed sequence is the request. */
        s->boundary = 0;
        s->work.reused = length;
        return s->logits != NULL;
    }
    if (!s->ingesting) {
        if (!open_ingestion(s, length)) {
            return 0;
        }
    } else if (s->target != length) {
        return 0;
    }
    const unsigned first = s->length;
    const unsigned remaining = length - first;
    const unsigned count = remaining < s->block ? remaining : s->block;
    int64_t ids[256];
    for (unsigned i = 0; i < count; i++) {
        ids[i] = tokens[first + i];
    }
    lunelette_session_work *w = &s->work;
    w->pending_attempted = s->pending && s->pending_position >= first &&
        s->pending_position < first + count;
    int status;
    if (!first) {
        w->full_attempted = count;
        w->prefill_calls = 1;
        status = lunelette_metal_prefill(s->runtime, ids, count, &s->logits, s->error,
            sizeof(s->error));
    } else if (!s->rebuilding && s->pending && remaining == 1) {
        /* Exactly the pending token on the reused prefix: one decode step. */
        w->decode_calls = 1;
        w->decode_attempted = 1;
        status = lunelette_metal_decode(s->runtime, s->emitted, &s->logits, s->error,
            sizeof(s->error));
    } else {
        w->suffix_attempted = count;
        w->append_calls = 1;
        status = lunelette_metal_append(s->runtime, ids, count, &s->logits, s->error,
            sizeof(s->error));
    }
    if (first < s->recompute_length) {
        const unsigned repeated = s->recompute_length - first;
        w->recompute_attempted = repeated < count ? repeated : count;
    }
    if (status) {
        s->ingesting = 0;
        s->logits = NULL;
        return 0;
    }
    w->recompute_committed = w->recompute_attempted;
    w->full_committed = w->full_attempted;
    w->suffix_committed = w->suffix_attempted;
    w->pending_committed = w->pending_attempted;
    w->decode_committed = w->decode_attempted;
    memcpy(s->prefix + first, tokens + first, count * sizeof(*tokens));
    s->length = first + count;
    if (w->pending_committed) {
        s->pending = 0;
    }
    if (s->length != length) {
        return LUNELETTE_SESSION_MORE;
    }
    s->ingesting = 0;
    s->pending = 0;
    return 1;
}

int lunelette_session_materialize_step(lunelette_session *s, const unsigned *tokens,
    unsigned length, unsigned *cursor)
{
    const int result = lunelette_session_materialize(s, tokens, length);
    if (cursor) {
        *cursor = s->length;
    }
    return result;
}

int lunelette_session_save(lunelette_session *s)
{
    if (!s->logits || !s->length || s->pending) {
        return -1;
    }
    lunelette_metal_checkpoint *replacement = NULL;
    if (lunelette_metal_checkpoint_create(s->runtime, &replacement, s->error,
            sizeof(s->error))) {
        /* A nonfinite logit invalidated the runtime: recovery is required.
         * Any other rejection keeps the previous handle and the sequence. */
        return lh_first_nonfinite(s->logits, LUNELETTE_VOCAB_SIZE) < LUNELETTE_VOCAB_SIZE ?
            -1 : 0;
    }
    lunelette_metal_checkpoint_destroy(s->checkpoint);
    s->checkpoint = replacement;
    s->saved_length = s->length;
    memcpy(s->saved_prefix, s->prefix, s->length * sizeof(*s->prefix));
    return 1;
}

int lunelette_session_restore(lunelette_session *s)
{
    memset(&s->work, 0, sizeof(s->work));
    if (!s->saved_length) {
        return 0;
    }
    if (s->policy == LUNELETTE_SESSION_REUSE_OFF) {
        /* Strict recompute: drop the sequence; the next materialize rebuilds
         * the saved prefix from the start and counts it as recomputation. */
        s->logits = NULL;
        s->pending = 0;
        s->emitted = 0;
        s->boundary = 0;
        s->ingesting = 0;
        memset(s->prefix, 0, sizeof(s->prefix));
        s->length = 0;
        s->recompute_hint = s->saved_length;
        return lunelette_metal_reset(s->runtime, s->error, sizeof(s->error)) ? -1 : 1;
    }
    const float *restored = NULL;
    if (lunelette_metal_checkpoint_restore(s->runtime, s->checkpoint, &restored, s->error,
            sizeof(s->error))) {
        return 0;
    }
    s->logits = restored;
    memcpy(s->prefix, s->saved_prefix, s->saved_length * sizeof(*s->prefix));
    s->length = s->saved_length;
    s->pending = 0;
    s->emitted = 0;
    s->boundary = 0;
    s->ingesting = 0;
    s->work.logit_restores = 1;
    return 1;
}

/* One LNRPLY1 record (selection index, prefix length, forced id, greedy id,
 * prefix ids, all logits as binary32), written with one fwrite and flushed.
 * A nonfinite logit or a short write latches the failure; the index only
 * advances on success. */
static int capture(lunelette_session *s, unsigned forced, unsigned greedy)
{
    if (lh_first_nonfinite(s->logits, LUNELETTE_VOCAB_SIZE) < LUNELETTE_VOCAB_SIZE) {
        s->replay_failed = 1;
        return 0;
    }
    uint32_t *r = s->record;
    r[0] = s->replay_index;
    r[1] = s->length;
    r[2] = forced;
    r[3] = greedy;
    memcpy(r + 4, s->prefix, s->length * sizeof(uint32_t));
    memcpy(r + 4 + s->length, s->logits, LUNELETTE_VOCAB_SIZE * sizeof(float));
    const size_t words = 4 + (size_t)s->length + LUNELETTE_VOCAB_SIZE;
    if (fwrite(r, sizeof(uint32_t), words, s->replay) != words || fflush(s->replay)) {
        s->replay_failed = 1;
        return 0;
    }
    s->replay_index++;
    return 1;
}

static int select_token(lunelette_session *s, int replay, unsigned forced)
{
    if (s->pending) {
        return -1;
    }
    if (replay && (!s->replay || s->replay_failed ||
            s->replay_index >= LUNELETTE_SESSION_REPLAY_TOKENS ||
            !(forced == LUNELETTE_SESSION_EOS ||
              (forced >= 1000 && forced < LUNELETTE_VOCAB_SIZE)))) {
        return -1;
    }
    /* A full context has no room for the next token, but its ids are still
     * validated first, as the generation loop does. */
    if ((s->capacity != LUNELETTE_CONTEXT_LIMIT && s->capacity != LUNELETTE_LONG_CONTEXT_LIMIT) ||
        !s->length || s->length > s->capacity) {
        return -1;
    }
    for (unsigned i = 0; i < s->length; i++) {
        if (s->prefix[i] >= LUNELETTE_VOCAB_SIZE) {
            return -1;
        }
    }
    if (s->length == s->capacity) {
        return -1;
    }
    int64_t token;
    if (lunelette_select_greedy(s->logits, &token, s->error, sizeof(s->error))) {
        return -1;
    }
    if (replay && !capture(s, forced, (unsigned)token)) {
        return -1;
    }
    s->emitted = replay ? forced : (unsigned)token;
    s->pending = 1;
    return (int)s->emitted;
}

int lunelette_session_next(lunelette_session *s)
{
    return select_token(s, 0, 0);
}

int lunelette_session_replay_next(lunelette_session *s, unsigned forced)
{
    return select_token(s, 1, forced);
}

unsigned lunelette_session_length(const lunelette_session *s)
{
    return s->length;
}

unsigned lunelette_session_context_capacity(const lunelette_session *s)
{
    return s->capacity;
}

unsigned lunelette_session_block_capacity(const lunelette_session *s)
{
    return s->block;
}

unsigned lunelette_session_prefix_reuse(const lunelette_session *s)
{
    return s->policy;
}

const char *lunelette_session_error(const lunelette_session *s)
{
    return s->error;
}

const float *lunelette_session_logits(const lunelette_session *s)
{
    return s->logits;
}

const char *lunelette_session_info(const lunelette_session *s)
{
    return s->info;
}
