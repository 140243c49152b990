/* CPU stand-in for the runtime C-ABI, linked with the session adapter
 * (lunelette_amd/csrc/session.c) into a test library so the adapter's
 * contract can be checked without a GPU: it records the token sequence the
 * adapter commits, counts the calls, and fails on request. Its behaviour is
 * the one the reference's adapter tests assume of their stub
 * (tests/support/native_runtime.h:19-182): logits are zero except ids 22177
 * and 22178 (a tie the lowest id wins), a checkpoint keeps a copy of the
 * logits and the token prefix, and only the context's active handle
 * restores. A call that breaks a runtime precondition is counted in
 * stub_violations and fails instead of aborting the test process.
 * Test infrastructure only. */
#include "lunelette_runtime.h"
#include "lunelette_generation.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct lunelette_metal {
    int64_t ids[LUNELETTE_LONG_CONTEXT_LIMIT];
    unsigned count, capacity, block;
    lunelette_metal_checkpoint *active;
    lunelette_metal_strategy strategy;
    lunelette_metal_prefill_mode prefill;
};

struct lunelette_metal_checkpoint {
    lunelette_metal *owner;
    unsigned count;
    int64_t ids[LUNELETTE_LONG_CONTEXT_LIMIT];
    float *saved;
};

/* Counters and switches the tests read and set through ctypes. */
unsigned stub_creates, stub_destroys, stub_prefills, stub_decodes, stub_appends, stub_resets;
unsigned stub_snapshots, stub_restores, stub_violations;
int stub_fail, stub_fail_memory, stub_fail_snapshot, stub_wrong_strategy;
int stub_last_prefill = -1;
float stub_logits[LUNELETTE_VOCAB_SIZE];
lunelette_metal *stub_last_runtime;

unsigned stub_count(const lunelette_metal *runtime)
{
    return runtime->count;
}

const int64_t *stub_ids(const lunelette_metal *runtime)
{
    return runtime->ids;
}

static int violation(char *error, size_t capacity, const char *what)
{
    stub_violations++;
    if (error && capacity) {
        snprintf(error, capacity, "stub precondition: %s", what);
    }
    return -1;
}

lunelette_metal *lunelette_metal_create_configured(const char *path,
    const lunelette_metal_options *options, const lunelette_metal_limits *limits,
    char *error, size_t capacity)
{
    (void)path;
    if (!options || !limits ||
        !(limits->context == 256 || limits->context == 4352) ||
        !(limits->block == 256 || (limits->context == 4352 && limits->block == 128))) {
        violation(error, capacity, "create limits");
        return NULL;
    }
    lunelette_metal *runtime = calloc(1, sizeof(*runtime));
    if (!runtime) {
        return NULL;
    }
    stub_creates++;
    runtime->strategy = stub_wrong_strategy ? LUNELETTE_METAL_RESIDENT_FP32 : options->strategy;
    runtime->prefill = options->prefill;
    runtime->capacity = (unsigned)limits->context;
    runtime->block = (unsigned)limits->block;
    stub_last_prefill = (int)options->prefill;
    stub_last_runtime = runtime;
    return runtime;
}

int lunelette_metal_get_limits(const lunelette_metal *runtime, lunelette_metal_limits *limits)
{
    if (!runtime || !limits) {
        return -1;
    }
    limits->context = runtime->capacity;
    limits->block = runtime->block;
    return 0;
}

/* The reference's byte accounting for the two storage families. */
int lunelette_metal_get_memory(const lunelette_metal *runtime, lunelette_metal_memory *memory)
{
    if (!runtime || !memory || stub_fail_memory) {
        return -1;
    }
    const int compact = runtime->strategy != LUNELETTE_METAL_RESIDENT_FP32;
    memory->strategy = runtime->strategy;
    memory->weight_bytes = compact ? 4637454336ULL : 13716025344ULL;
    memory->conversion_stage_bytes = compact ? 113246208ULL : 0;
    memory->scratch_bytes = 87819264ULL;
    memory->kv_bytes = 54525952ULL;
    memory->total_bytes = compact ? 4893045760ULL : 13858370560ULL;
    return 0;
}

void lunelette_metal_destroy(lunelette_metal *runtime)
{
    if (runtime) {
        stub_destroys++;
        if (stub_last_runtime == runtime) {
            stub_last_runtime = NULL;
        }
        free(runtime);
    }
}

int lunelette_metal_reset(lunelette_metal *runtime, char *error, size_t capacity)
{
    (void)error;
    (void)capacity;
    stub_resets++;
    runtime->count = 0;
    runtime->active = NULL;
    return 0;
}

static int result(lunelette_metal *runtime, const float **out, char *error, size_t capacity)
{
    if (stub_fail) {
        *out = NULL;
        runtime->active = NULL;
        if (error && capacity) {
            snprintf(error, capacity, "deliberate test failure");
        }
        return -1;
    }
    memset(stub_logits, 0, sizeof(stub_logits));
    stub_logits[22177] = stub_logits[22178] = 1.0f;
    *out = stub_logits;
    return 0;
}

int lunelette_metal_prefill(lunelette_metal *runtime, const int64_t *ids, size_t count,
    const float **out, char *error, size_t capacity)
{
    if (runtime->count || !count || count > runtime->block) {
        return violation(error, capacity, "prefill on a nonempty sequence or bad count");
    }
    memcpy(runtime->ids, ids, count * sizeof(*ids));
    runtime->count = (unsigned)count;
    stub_prefills++;
    return result(runtime, out, error, capacity);
}

int lunelette_metal_decode(lunelette_metal *runtime, int64_t token, const float **out,
    char *error, size_t capacity)
{
    if (!runtime->count || runtime->count >= runtime->capacity) {
        return violation(error, capacity, "decode on an empty or full sequence");
    }
    runtime->ids[runtime->count++] = token;
    stub_decodes++;
    return result(runtime, out, error, capacity);
}

int lunelette_metal_append(lunelette_metal *runtime, const int64_t *ids, size_t count,
    const float **out, char *error, size_t capacity)
{
    if (!runtime->count || !count || runtime->count + count > runtime->capacity ||
        count > runtime->block) {
        return violation(error, capacity, "append bounds");
    }
    memcpy(runtime->ids + runtime->count, ids, count * sizeof(*ids));
    runtime->count += (unsigned)count;
    stub_appends++;
    return result(runtime, out, error, capacity);
}

int lunelette_metal_checkpoint_create(lunelette_metal *runtime,
    lunelette_metal_checkpoint **out, char *error, size_t capacity)
{
    *out = NULL;
    if (stub_fail_snapshot) {
        if (error && capacity) {
            snprintf(error, capacity, "deliberate snapshot failure");
        }
        return -1;
    }
    if (!runtime->count) {
        return violation(error, capacity, "checkpoint of an empty sequence");
    }
    lunelette_metal_checkpoint *c = calloc(1, sizeof(*c));
    if (!c || !(c->saved = malloc(sizeof(stub_logits)))) {
        free(c);
        return -1;
    }
    memcpy(c->saved, stub_logits, sizeof(stub_logits));
    memcpy(c->ids, runtime->ids, sizeof(c->ids));
    c->owner = runtime;
    c->count = runtime->count;
    runtime->active = c;
    *out = c;
    stub_snapshots++;
    return 0;
}

int lunelette_metal_checkpoint_restore(lunelette_metal *runtime,
    const lunelette_metal_checkpoint *c, const float **out, char *error, size_t capacity)
{
    *out = NULL;
    if (!c || c->owner != runtime || runtime->active != c || runtime->count < c->count ||
        memcmp(runtime->ids, c->ids, c->count * sizeof(*c->ids))) {
        if (error && capacity) {
            snprintf(error, capacity, "inactive or incompatible checkpoint");
        }
        return -1;
    }
    runtime->count = c->count;
    memcpy(stub_logits, c->saved, sizeof(stub_logits));
    *out = stub_logits;
    stub_restores++;
    return 0;
}

void lunelette_metal_checkpoint_destroy(lunelette_metal_checkpoint *c)
{
    if (c) {
        if (c->owner->active == c) {
            c->owner->active = NULL;
        }
        free(c->saved);
        free(c);
    }
}
