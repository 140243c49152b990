/* CPU stand-in for the runtime C-ABI (include/lunelette_runtime.h), linked
 * with the session adapter (lunelette_amd/csrc/session.c) into a test library
 * so the adapter's contract runs without a GPU. Test infrastructure only.
 *
 * It models only what the adapter can observe through the ABI:
 * - the committed id sequence (prefill on an empty sequence, decode of one id,
 *   append of up to one block), bounded by the configured context;
 * - published logits: all zero except ids 22177 and 22178, which tie at 1, so
 *   greedy selection yields 22177 (the fixture the reference's adapter tests
 *   are written against);
 * - one active checkpoint per context, holding its prefix and logits; only
 *   the active handle restores, and only onto a sequence that still begins
 *   with that prefix;
 * - the reference's byte accounting for the compact and resident families.
 * Calls the runtime would reject as misuse fail here too and are counted in
 * stub_violations, so a test sees the misuse instead of a crash. Counters and
 * switches are plain globals the tests read and set through ctypes. */
#include "lunelette_runtime.h"
#include "lunelette_generation.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define STUB_CAPACITY LUNELETTE_LONG_CONTEXT_LIMIT

struct lunelette_metal {
    size_t context, block;
    lunelette_metal_strategy strategy;
    size_t length;
    int64_t sequence[STUB_CAPACITY];
    lunelette_metal_checkpoint *active;
};

struct lunelette_metal_checkpoint {
    lunelette_metal *context;
    size_t length;
    int64_t prefix[STUB_CAPACITY];
    float logits[LUNELETTE_VOCAB_SIZE];
};

/* Call counters. */
unsigned stub_creates, stub_destroys, stub_prefills, stub_decodes, stub_appends, stub_resets;
unsigned stub_snapshots, stub_restores, stub_violations;
/* Switches: fail every execution, the memory query, checkpoint creation; report
 * the resident strategy whatever was asked. */
int stub_fail, stub_fail_memory, stub_fail_snapshot, stub_wrong_strategy;
/* The prefill mode of the last create, and the last context created. */
int stub_last_prefill = -1;
lunelette_metal *stub_last_runtime;
/* The published logits. */
float stub_logits[LUNELETTE_VOCAB_SIZE];

unsigned stub_count(const lunelette_metal *context)
{
    return (unsigned)context->length;
}

const int64_t *stub_ids(const lunelette_metal *context)
{
    return context->sequence;
}

static int note(char *error, size_t capacity, const char *text)
{
    if (error && capacity) {
        snprintf(error, capacity, "%s", text);
    }
    return -1;
}

static int misuse(char *error, size_t capacity, const char *text)
{
    stub_violations++;
    return note(error, capacity, text);
}

lunelette_metal *lunelette_metal_create_configured(const char *path,
    const lunelette_metal_options *options, const lunelette_metal_limits *limits,
    char *error, size_t capacity)
{
    (void)path;
    const int profile = limits && ((limits->context == 256 && limits->block == 256) ||
        (limits->context == 4352 && (limits->block == 256 || limits->block == 128)));
    if (!options || !profile) {
        misuse(error, capacity, "stub: create needs options and a supported profile");
        return NULL;
    }
    lunelette_metal *context = calloc(1, sizeof *context);
    if (!context) {
        note(error, capacity, "stub: out of memory");
        return NULL;
    }
    context->context = limits->context;
    context->block = limits->block;
    context->strategy = stub_wrong_strategy ? LUNELETTE_METAL_RESIDENT_FP32 : options->strategy;
    stub_last_prefill = (int)options->prefill;
    stub_last_runtime = context;
    stub_creates++;
    return context;
}

int lunelette_metal_get_limits(const lunelette_metal *context, lunelette_metal_limits *limits)
{
    if (!context || !limits) {
        return -1;
    }
    limits->context = context->context;
    limits->block = context->block;
    return 0;
}

int lunelette_metal_get_memory(const lunelette_metal *context, lunelette_metal_memory *memory)
{
    if (!context || !memory || stub_fail_memory) {
        return -1;
    }
    /* Compact: FP8 codes plus the conversion stage; resident: FP32 weights. */
    static const lunelette_metal_memory compact = {LUNELETTE_METAL_COMPACT_FP8_ARITHMETIC,
        4637454336ULL, 113246208ULL, 87819264ULL, 54525952ULL, 4893045760ULL};
    static const lunelette_metal_memory resident = {LUNELETTE_METAL_RESIDENT_FP32,
        13716025344ULL, 0, 87819264ULL, 54525952ULL, 13858370560ULL};
    *memory = context->strategy == LUNELETTE_METAL_RESIDENT_FP32 ? resident : compact;
    memory->strategy = context->strategy;
    return 0;
}

void lunelette_metal_destroy(lunelette_metal *context)
{
    if (!context) {
        return;
    }
    if (stub_last_runtime == context) {
        stub_last_runtime = NULL;
    }
    stub_destroys++;
    free(context);
}

int lunelette_metal_reset(lunelette_metal *context, char *error, size_t capacity)
{
    (void)error;
    (void)capacity;
    context->length = 0;
    context->active = NULL;
    stub_resets++;
    return 0;
}

/* Commits ids to the sequence and publishes logits, or fails the execution
 * (which, as in the runtime, withdraws the active checkpoint). */
static int execute(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity)
{
    memcpy(context->sequence + context->length, ids, count * sizeof *ids);
    context->length += count;
    if (stub_fail) {
        *logits = NULL;
        context->active = NULL;
        return note(error, capacity, "stub: execution failed on request");
    }
    memset(stub_logits, 0, sizeof stub_logits);
    stub_logits[22177] = 1.0f;
    stub_logits[22178] = 1.0f;
    *logits = stub_logits;
    return 0;
}

int lunelette_metal_prefill(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity)
{
    if (context->length != 0 || count < 1 || count > context->block) {
        return misuse(error, capacity, "stub: prefill needs an empty sequence and 1..block ids");
    }
    stub_prefills++;
    return execute(context, ids, count, logits, error, capacity);
}

int lunelette_metal_decode(lunelette_metal *context, int64_t token, const float **logits,
    char *error, size_t capacity)
{
    if (context->length == 0 || context->length >= context->context) {
        return misuse(error, capacity, "stub: decode needs a sequence with room for one id");
    }
    stub_decodes++;
    return execute(context, &token, 1, logits, error, capacity);
}

int lunelette_metal_append(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity)
{
    if (context->length == 0 || count < 1 || count > context->block ||
        context->length + count > context->context) {
        return misuse(error, capacity, "stub: append needs a sequence and 1..block ids that fit");
    }
    stub_appends++;
    return execute(context, ids, count, logits, error, capacity);
}

int lunelette_metal_checkpoint_create(lunelette_metal *context,
    lunelette_metal_checkpoint **checkpoint, char *error, size_t capacity)
{
    *checkpoint = NULL;
    if (stub_fail_snapshot) {
        return note(error, capacity, "stub: checkpoint failed on request");
    }
    if (context->length == 0) {
        return misuse(error, capacity, "stub: checkpoint of an empty sequence");
    }
    lunelette_metal_checkpoint *saved = malloc(sizeof *saved);
    if (!saved) {
        return note(error, capacity, "stub: out of memory");
    }
    saved->context = context;
    saved->length = context->length;
    memcpy(saved->prefix, context->sequence, context->length * sizeof *saved->prefix);
    memcpy(saved->logits, stub_logits, sizeof saved->logits);
    context->active = saved;
    *checkpoint = saved;
    stub_snapshots++;
    return 0;
}

int lunelette_metal_checkpoint_restore(lunelette_metal *context,
    const lunelette_metal_checkpoint *checkpoint, const float **logits, char *error,
    size_t capacity)
{
    *logits = NULL;
    const int usable = checkpoint && checkpoint->context == context &&
        context->active == checkpoint && context->length >= checkpoint->length &&
        memcmp(context->sequence, checkpoint->prefix,
            checkpoint->length * sizeof *checkpoint->prefix) == 0;
    if (!usable) {
        return note(error, capacity, "stub: the checkpoint is not this context's active prefix");
    }
    context->length = checkpoint->length;
    memcpy(stub_logits, checkpoint->logits, sizeof stub_logits);
    *logits = stub_logits;
    stub_restores++;
    return 0;
}

void lunelette_metal_checkpoint_destroy(lunelette_metal_checkpoint *checkpoint)
{
    if (!checkpoint) {
        return;
    }
    if (checkpoint->context->active == checkpoint) {
        checkpoint->context->active = NULL;
    }
    free(checkpoint);
}
