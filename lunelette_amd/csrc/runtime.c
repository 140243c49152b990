/* Lunelette runtime on one MI355X: the include/metal.h contract over HIP.
 *
 * Replaces src/metal_runtime.m (lifetime, residency, execute, checkpoints,
 * memory query), src/metal_encode.m (operator sequence, via lh_layer_forward),
 * src/metal_mps.m (prefill GEMM, via the MFMA path) and src/metal_weights.c
 * (FP8 admission and byte accounting). State machine and validation follow
 * src/metal_runtime.m:333-575 exactly: argument errors before any mutation,
 * withdraw-then-publish around execution, host finite scan of the logits,
 * checkpoints holding a logit copy plus length/epoch/identity, no KV copy.
 */
#include "lunelette_runtime.h"
#include "lunelette_kernels.h"
#include "lh_internal.h"
#include "lh_layer.h"
#include "lh_scan.h"
#include "lh_weights.h"

#include <math.h>
#include <stdatomic.h>
#include <stdbool.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifndef LH_HAVE_MFMA
#define LH_HAVE_MFMA 1
#endif

struct lunelette_metal_checkpoint {
    struct lh_runtime *owner; /* borrowed; handles are destroyed before the context */
    uint64_t identity, epoch;
    size_t length;
    float logits[LH_VOCAB];
};

typedef struct lh_runtime {
    lunelette_metal_limits limits;
    lunelette_metal_prefill_mode prefill_mode;
    lunelette_metal_strategy strategy;
    lunelette_metal_memory memory;
    uint32_t layers;
    hipStream_t stream;
    hipEvent_t started, finished;
    float last_ms;
    void *d_weights;          /* FP8 codes (compact) or their exact FP32 decode (resident) */
    uint16_t *d_embedding;    /* BF16 [131072][3072], also the tied head */
    float *d_norms;           /* FP32 [2*layers+1][3072] */
    lh_layer_weights layer[LH_LAYERS];
    float *d_kv;              /* keys [layers][8][C][128] then values */
    float *d_keys, *d_values;
    float *d_x;               /* [B][3072] residual stream */
    float *h_logits;          /* [131072] pinned, coherent; borrowed by callers */
    float *d_logits;          /* the same buffer as the head kernel addresses it */
    volatile uint32_t *h_nonfinite; /* pinned, coherent: set by the head kernel */
    uint32_t *d_nonfinite;
    lh_workspace *ws;
    size_t length;
    bool valid, endpoint_logits_valid;
    uint64_t identity, checkpoint_epoch;
    lunelette_metal_checkpoint *active_checkpoint;
    struct {                  /* host-forced faults (lh_runtime_fault) */
        bool before_device, nonfinite, checkpoint_alloc;
        int handoff;              /* LH_HANDOFF_* wait that gives up; 0 off */
        uint32_t after_layer;     /* fail after layer after_layer - 1; 0 off */
    } fault;
} lh_runtime;

struct lunelette_metal {
    lh_runtime *rt;
};

static _Atomic uint64_t last_identity;

static void report(char *error, size_t capacity, const char *format, const char *detail)
{
    if (error && capacity) {
        snprintf(error, capacity, format, detail ? detail : "");
    }
}

/* Profiles of src/metal_plan.h:37-41 plus the additive long profile. */
static int profile_supported(lunelette_metal_limits limits)
{
    return (limits.context == 256 && limits.block == 256) ||
        (limits.context == 4352 && (limits.block == 256 || limits.block == 128)) ||
        (limits.context == 17920 && (limits.block == 256 || limits.block == 128));
}

/* src/metal_options.h:9-30. */
static int resolve_options(const lunelette_metal_options *options, lunelette_metal_options *out,
    char *error, size_t capacity)
{
    lunelette_metal_options selected = LUNELETTE_METAL_OPTIONS_DEFAULT;
    if (options) {
        selected = *options;
    }
    if (selected.prefill != LUNELETTE_METAL_PREFILL_MPS &&
        selected.prefill != LUNELETTE_METAL_PREFILL_CUSTOM) {
        report(error, capacity, "%sinvalid prefill option; select MPS or CUSTOM", NULL);
        return -1;
    }
    if (selected.strategy != LUNELETTE_METAL_RESIDENT_FP32 &&
        selected.strategy != LUNELETTE_METAL_COMPACT_FP8_ARITHMETIC &&
        selected.strategy != LUNELETTE_METAL_COMPACT_FP8_LOOKUP) {
        report(error, capacity, "%sinvalid strategy; select resident-fp32, "
            "compact-fp8-arithmetic or compact-fp8-lookup", NULL);
        return -1;
    }
    *out = selected;
    return 0;
}

static uint64_t layer_fp8_bytes(void)
{
    return (uint64_t)LH_QKV_ROWS * LH_HIDDEN + (uint64_t)LH_HIDDEN * LH_QUERY +
        2ull * LH_INNER * LH_HIDDEN + (uint64_t)LH_HIDDEN * LH_INNER;
}

static void destroy_runtime(lh_runtime *rt)
{
    if (!rt) {
        return;
    }
    if (rt->stream) {
        (void)hipStreamSynchronize(rt->stream);
    }
    void *device[] = {rt->d_weights, rt->d_embedding, rt->d_norms, rt->d_kv, rt->d_x};
    for (size_t i = 0; i < sizeof device / sizeof device[0]; i++) {
        lh_dev_free(device[i]);
    }
    lh_host_free(rt->h_logits);
    lh_host_free((void *)rt->h_nonfinite);
    lh_workspace_destroy(rt->ws);
    if (rt->started) {
        (void)hipEventDestroy(rt->started);
    }
    if (rt->finished) {
        (void)hipEventDestroy(rt->finished);
    }
    if (rt->stream) {
        (void)hipStreamDestroy(rt->stream);
    }
    free(rt);
}

static int hip_ok(hipError_t status, const char *what, char *error, size_t capacity)
{
    if (status != hipSuccess) {
        if (error && capacity) {
            snprintf(error, capacity, "HIP %s failed: %s", what, hipGetErrorString(status));
        }
        return -1;
    }
    return 0;
}

/* FP8 admission, per strategy. Compact (src/metal_weights.c:174-231): the
 * scale must be positive, FP32-normal and BF16-exact; every code finite; every
 * nonzero reconstructed product normal. Resident (st_load_fp8,
 * src/safetensors.c:521-548): the scale positive and finite; every product
 * fl(dec * scale) finite, so NaN codes and overflow are refused while
 * subnormal scales and products are accepted. Builds the 256-entry allowed
 * table; -1 when the scale itself is refused. */
static int fp8_admission_table(float scale, bool resident, unsigned char allowed[256])
{
    uint32_t bits;
    memcpy(&bits, &scale, sizeof bits);
    if (resident ? !(scale > 0) || !isfinite(scale) :
            !(scale > 0) || !isnormal(scale) || (bits & 0xffffu)) {
        return -1;
    }
    for (unsigned code = 0; code < 256; code++) {
        unsigned e = (code >> 3) & 15u, f = code & 7u;
        if (e == 15 && f == 7) {
            allowed[code] = 0;
            continue;
        }
        float magnitude = e == 0 ? ldexpf((float)f, -9) : ldexpf((float)(8 + f), (int)e - 10);
        float product = magnitude * scale;
        allowed[code] = isfinite(product) && (resident || magnitude == 0 || isnormal(product));
    }
    return 0;
}

int lh_fp8_admit(const uint8_t *codes, size_t n, float scale, int strategy, char *error,
    size_t capacity)
{
    if (!codes || (strategy != LUNELETTE_METAL_RESIDENT_FP32 &&
            strategy != LUNELETTE_METAL_COMPACT_FP8_ARITHMETIC &&
            strategy != LUNELETTE_METAL_COMPACT_FP8_LOOKUP)) {
        report(error, capacity, "%sadmission needs codes and a strategy", NULL);
        return -1;
    }
    const bool resident = strategy == LUNELETTE_METAL_RESIDENT_FP32;
    unsigned char allowed[256];
    if (fp8_admission_table(scale, resident, allowed)) {
        report(error, capacity, resident ? "%sscale must be positive and finite" :
            "%sscale must be positive FP32-normal widened BF16", NULL);
        return -1;
    }
    for (size_t i = 0; i < n; i++) {
        if (!allowed[codes[i]]) {
            if (error && capacity) {
                snprintf(error, capacity, "byte %zu code 0x%02x: %s", i, codes[i], resident ?
                    "NaN or overflowing reconstructed product" :
                    "NaN or non-normal/overflow reconstructed product");
            }
            return -1;
        }
    }
    return 0;
}

static float fp8_value(unsigned char code)
{
    unsigned e = (code >> 3) & 15u, f = code & 7u;
    float magnitude = e == 0 ? ldexpf((float)f, -9) : ldexpf((float)(8 + f), (int)e - 10);
    return (code & 128u) ? -magnitude : magnitude;
}

#define STAGE_BYTES ((size_t)64 << 20)

typedef struct {
    hipStream_t stream;
    void *stage[2];
    hipEvent_t done[2];
    int next;
} uploader;

static void *stage_slot(uploader *up)
{
    int k = up->next;
    (void)hipEventSynchronize(up->done[k]);
    return up->stage[k];
}

static int stage_push(uploader *up, void *dst, size_t bytes, char *error, size_t capacity)
{
    int k = up->next;
    if (hip_ok(hipMemcpyAsync(dst, up->stage[k], bytes, hipMemcpyHostToDevice, up->stream),
            "weight upload", error, capacity) ||
        hip_ok(hipEventRecord(up->done[k], up->stream), "upload event", error, capacity)) {
        return -1;
    }
    up->next ^= 1;
    return 0;
}

/* Where the tensor bytes come from: the seeded synthetic generator or a
 * checkpoint file. read() copies elements [offset, offset + count) of a slot
 * (FP8 codes, 1 byte each; BF16 bits, 2 bytes each, little-endian). */
typedef struct weight_source {
    int (*read)(struct weight_source *src, uint32_t slot, uint64_t offset, void *dst,
        size_t count);
    float (*scale)(struct weight_source *src, uint32_t slot);
    uint64_t seed;
    lh_weights *file;
} weight_source;

static bool norm_slot(uint32_t slot)
{
    return slot == 1 || (slot >= 2 && ((slot - 2) % 9 == 0 || (slot - 2) % 9 == 5));
}

static int synthetic_read(weight_source *src, uint32_t slot, uint64_t offset, void *dst,
    size_t count)
{
    if (slot == 0) {
        lh_synth_normal_bf16(src->seed, 0, offset, 0.0f, 0.02f, dst, count);
    } else if (norm_slot(slot)) {
        lh_synth_normal_bf16(src->seed, slot, offset, 1.0f, 0.02f, dst, count);
    } else {
        lh_synth_fp8(src->seed, slot, offset, dst, count);
    }
    return 0;
}

static float synthetic_scale(weight_source *src, uint32_t slot)
{
    return lh_synth_scale(src->seed, slot);
}

static int file_read(weight_source *src, uint32_t slot, uint64_t offset, void *dst, size_t count)
{
    const lh_st_tensor *t = src->file->slot[slot].tensor;
    const size_t esize = t->dtype == LH_ST_F8_E4M3 ? 1 : 2;
    return lh_st_read(&src->file->file, t, offset * esize, dst, count * esize);
}

static float file_scale(weight_source *src, uint32_t slot)
{
    return src->file->slot[slot].scale;
}

static int source_read(weight_source *src, uint32_t slot, uint64_t offset, void *dst, size_t count,
    char *error, size_t capacity)
{
    if (src->read(src, slot, offset, dst, count)) {
        if (error && capacity) {
            snprintf(error, capacity, "checkpoint read failed: %s",
                src->file ? src->file->slot[slot].tensor->name : "synthetic");
        }
        return -1;
    }
    return 0;
}

/* FP8 tensor `tensor` of n codes: admit, then store the codes (compact) or
 * their exact FP32 decode (resident); both strategies multiply the row total
 * by the per-tensor scale, so on what both admit their results are bitwise
 * identical. */
static int upload_fp8(uploader *up, weight_source *src, uint32_t tensor, float scale, size_t n,
    bool resident, void *dst, char *error, size_t capacity)
{
    unsigned char allowed[256];
    if (fp8_admission_table(scale, resident, allowed)) {
        if (error && capacity) {
            snprintf(error, capacity, resident ?
                "resident tensor %u: scale must be positive and finite" :
                "compact tensor %u: scale must be positive FP32-normal widened BF16", tensor);
        }
        return -1;
    }
    float table[256];
    for (int b = 0; b < 256; b++) {
        table[b] = fp8_value((unsigned char)b);
    }
    const size_t chunk = resident ? STAGE_BYTES / 4 / 2 : STAGE_BYTES / 2;
    uint8_t *codes = malloc(chunk);
    if (!codes) {
        report(error, capacity, "%shost staging allocation failed", NULL);
        return -1;
    }
    for (size_t offset = 0; offset < n; offset += chunk) {
        size_t m = n - offset < chunk ? n - offset : chunk;
        void *slot = stage_slot(up);
        uint8_t *dst_codes = resident ? codes : (uint8_t *)slot;
        if (source_read(src, tensor, offset, dst_codes, m, error, capacity)) {
            free(codes);
            return -1;
        }
        for (size_t i = 0; i < m; i++) {
            if (!allowed[dst_codes[i]]) {
                if (error && capacity) {
                    snprintf(error, capacity, resident ?
                        "resident tensor %u byte %zu code 0x%02x: NaN or overflowing "
                        "reconstructed product" :
                        "compact tensor %u byte %zu code 0x%02x: NaN or non-normal/overflow "
                        "reconstructed product", tensor, offset + i, dst_codes[i]);
                }
                free(codes);
                return -1;
            }
        }
        if (resident) {
            float *out = slot;
            for (size_t i = 0; i < m; i++) {
                out[i] = table[codes[i]];
            }
            if (stage_push(up, (float *)dst + offset, m * sizeof(float), error, capacity)) {
                free(codes);
                return -1;
            }
        } else if (stage_push(up, (uint8_t *)dst + offset, m, error, capacity)) {
            free(codes);
            return -1;
        }
    }
    free(codes);
    return 0;
}

static int upload_bf16(uploader *up, weight_source *src, uint32_t tensor, size_t n, uint16_t *dst,
    char *error, size_t capacity)
{
    const size_t chunk = STAGE_BYTES / 2;
    for (size_t offset = 0; offset < n; offset += chunk) {
        size_t m = n - offset < chunk ? n - offset : chunk;
        uint16_t *slot = stage_slot(up);
        if (source_read(src, tensor, offset, slot, m, error, capacity) ||
            stage_push(up, dst + offset, m * sizeof(uint16_t), error, capacity)) {
            return -1;
        }
    }
    return 0;
}

/* Norm vectors are BF16 in the checkpoint and widened to FP32 (exact). */
static int upload_norm(uploader *up, weight_source *src, uint32_t tensor, float *dst, char *error,
    size_t capacity)
{
    uint16_t bits[LH_HIDDEN];
    if (source_read(src, tensor, 0, bits, LH_HIDDEN, error, capacity)) {
        return -1;
    }
    float *slot = stage_slot(up);
    for (size_t i = 0; i < LH_HIDDEN; i++) {
        uint32_t word = (uint32_t)bits[i] << 16;
        memcpy(&slot[i], &word, sizeof(float));
    }
    return stage_push(up, dst, LH_HIDDEN * sizeof(float), error, capacity);
}

/* Device residency for `layers` layers from src, after the profile and the
 * options have been resolved. */
static lunelette_metal *build_runtime(weight_source *src, uint32_t layers,
    lunelette_metal_limits resolved, lunelette_metal_options selected, char *error,
    size_t capacity)
{
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1) {
        snprintf(error, capacity, "no HIP device: the gfx950 runtime needs an MI355X");
        return NULL;
    }
    lh_runtime *rt = calloc(1, sizeof *rt);
    if (!rt) {
        snprintf(error, capacity, "runtime allocation failed");
        return NULL;
    }
    rt->limits = resolved;
    rt->prefill_mode = selected.prefill;
    rt->strategy = selected.strategy;
    rt->layers = layers;
    const bool resident = selected.strategy == LUNELETTE_METAL_RESIDENT_FP32;
    const size_t C = resolved.context, B = resolved.block;
    const uint64_t fp8_bytes = layer_fp8_bytes() * rt->layers;
    const uint64_t weight_bytes = (resident ? 4 : 1) * fp8_bytes;
    const uint64_t embedding_bytes = (uint64_t)LH_VOCAB * LH_HIDDEN * sizeof(uint16_t);
    const uint64_t norm_bytes = (2ull * rt->layers + 1) * LH_HIDDEN * sizeof(float);
    const uint64_t kv_bytes = 2ull * rt->layers * LH_KV_HEADS * C * LH_HEAD_DIM * sizeof(float);
    uploader up = {0};
    if (hip_ok(hipStreamCreate(&rt->stream), "stream creation", error, capacity) ||
        hip_ok(hipEventCreate(&rt->started), "event creation", error, capacity) ||
        hip_ok(hipEventCreate(&rt->finished), "event creation", error, capacity)) {
        goto failure;
    }
    size_t free_bytes = 0, total_bytes = 0;
    if (hip_ok(hipMemGetInfo(&free_bytes, &total_bytes), "memory query", error, capacity)) {
        goto failure;
    }
    if (weight_bytes + embedding_bytes + kv_bytes + ((uint64_t)1 << 30) > free_bytes) {
        snprintf(error, capacity, "weights and KV exceed free device memory");
        goto failure;
    }
    rt->ws = lh_workspace_create(C, B);
    if (!rt->ws || lh_mfma_prepare(rt->ws) || lh_workspace_prepare_decode(rt->ws)) {
        snprintf(error, capacity, "workspace: %s", lh_last_error());
        goto failure;
    }
    if (hip_ok(lh_dev_malloc(&rt->d_weights, weight_bytes), "weight allocation", error,
            capacity) ||
        hip_ok(lh_dev_malloc((void **)&rt->d_embedding, embedding_bytes), "embedding allocation",
            error, capacity) ||
        hip_ok(lh_dev_malloc((void **)&rt->d_norms, norm_bytes), "norm allocation", error,
            capacity) ||
        hip_ok(lh_dev_malloc((void **)&rt->d_kv, kv_bytes), "KV allocation", error, capacity) ||
        hip_ok(lh_dev_malloc((void **)&rt->d_x, B * LH_HIDDEN * sizeof(float)),
            "scratch allocation", error, capacity) ||
        /* The head kernel writes the logits straight into coherent pinned
         * memory: no device-to-host copy after the step. */
        hip_ok(lh_host_malloc((void **)&rt->h_logits, LH_VOCAB * sizeof(float),
            hipHostMallocMapped | hipHostMallocCoherent), "pinned logits", error, capacity) ||
        hip_ok(hipHostGetDevicePointer((void **)&rt->d_logits, rt->h_logits, 0),
            "mapped logits", error, capacity) ||
        hip_ok(lh_host_malloc((void **)&rt->h_nonfinite, 64,
            hipHostMallocMapped | hipHostMallocCoherent), "pinned flag", error, capacity) ||
        hip_ok(hipHostGetDevicePointer((void **)&rt->d_nonfinite, (void *)rt->h_nonfinite, 0),
            "mapped flag", error, capacity)) {
        goto failure;
    }
    rt->d_keys = rt->d_kv;
    rt->d_values = rt->d_kv + kv_bytes / sizeof(float) / 2;
    if (hip_ok(hipMemsetAsync(rt->d_kv, 0, kv_bytes, rt->stream), "KV clear", error, capacity)) {
        goto failure;
    }
    /* Upload: tensor ids follow the reference slot order (metal_weights.h):
     * 0 embedding, 1 final norm, then 2 + 9*layer + {in_norm, q, k, v, o,
     * post_norm, gate, up, down}. */
    up.stream = rt->stream;
    for (int k = 0; k < 2; k++) {
        if (hip_ok(lh_host_malloc(&up.stage[k], STAGE_BYTES, hipHostMallocDefault),
                "pinned staging", error, capacity) ||
            hip_ok(hipEventCreate(&up.done[k]), "staging event", error, capacity)) {
            goto failure;
        }
    }
    if (upload_bf16(&up, src, 0, (size_t)LH_VOCAB * LH_HIDDEN, rt->d_embedding, error,
            capacity) ||
        upload_norm(&up, src, 1, rt->d_norms + 2ull * rt->layers * LH_HIDDEN, error, capacity)) {
        goto failure;
    }
    static const size_t rows[7] = {LH_QUERY, LH_KV, LH_KV, LH_HIDDEN, LH_INNER, LH_INNER, LH_HIDDEN};
    static const size_t cols[7] = {LH_HIDDEN, LH_HIDDEN, LH_HIDDEN, LH_QUERY, LH_HIDDEN, LH_HIDDEN,
        LH_INNER};
    static const uint32_t slot[7] = {1, 2, 3, 4, 6, 7, 8};
    const size_t esize = resident ? 4 : 1;
    for (uint32_t l = 0; l < rt->layers; l++) {
        lh_layer_weights *w = &rt->layer[l];
        char *base = (char *)rt->d_weights + layer_fp8_bytes() * l * esize;
        size_t offset = 0;
        void *ptr[7];
        for (int i = 0; i < 7; i++) {
            const uint32_t tensor = 2 + 9 * l + slot[i];
            ptr[i] = base + offset;
            w->scale[i] = src->scale(src, tensor);
            if (upload_fp8(&up, src, tensor, w->scale[i], rows[i] * cols[i], resident, ptr[i],
                    error, capacity)) {
                goto failure;
            }
            offset += rows[i] * cols[i] * esize;
        }
        if (resident) {
            w->f32_qkv = ptr[0];
            w->f32_o = ptr[3];
            w->f32_gate = ptr[4];
            w->f32_up = ptr[5];
            w->f32_down = ptr[6];
        } else {
            w->qkv = ptr[0];
            w->o = ptr[3];
            w->gate = ptr[4];
            w->up = ptr[5];
            w->down = ptr[6];
        }
        float *in_norm = rt->d_norms + 2ull * l * LH_HIDDEN;
        float *post_norm = in_norm + LH_HIDDEN;
        if (upload_norm(&up, src, 2 + 9 * l + 0, in_norm, error, capacity) ||
            upload_norm(&up, src, 2 + 9 * l + 5, post_norm, error, capacity)) {
            goto failure;
        }
        w->input_norm = in_norm;
        w->post_norm = post_norm;
    }
    if (hip_ok(hipStreamSynchronize(rt->stream), "upload completion", error, capacity)) {
        goto failure;
    }
    for (int k = 0; k < 2; k++) {
        lh_host_free(up.stage[k]);
        (void)hipEventDestroy(up.done[k]);
        up.stage[k] = NULL;
        up.done[k] = NULL;
    }
    rt->memory.strategy = rt->strategy;
    rt->memory.weight_bytes = weight_bytes + embedding_bytes + norm_bytes;
    rt->memory.conversion_stage_bytes = 0;
    rt->memory.scratch_bytes = rt->ws->bytes + B * LH_HIDDEN * sizeof(float);
    rt->memory.kv_bytes = kv_bytes;
    rt->memory.total_bytes = rt->memory.weight_bytes + rt->memory.scratch_bytes + kv_bytes;
    uint64_t previous = atomic_load(&last_identity);
    do {
        if (previous == UINT64_MAX) {
            snprintf(error, capacity, "context identities exhausted");
            goto failure;
        }
    } while (!atomic_compare_exchange_weak(&last_identity, &previous, previous + 1));
    rt->identity = previous + 1;
    rt->valid = true;
    lunelette_metal *context = calloc(1, sizeof *context);
    if (!context) {
        snprintf(error, capacity, "context allocation failed");
        goto failure;
    }
    context->rt = rt;
    return context;
failure:
    for (int k = 0; k < 2; k++) {
        if (up.done[k]) {
            (void)hipEventSynchronize(up.done[k]);
            (void)hipEventDestroy(up.done[k]);
        }
        lh_host_free(up.stage[k]);
    }
    destroy_runtime(rt);
    return NULL;
}

lunelette_metal *lunelette_metal_create_synthetic(const lunelette_synthetic_config *config,
    const lunelette_metal_options *options, const lunelette_metal_limits *limits,
    char *error, size_t capacity)
{
    char fallback[512];
    if (!error || !capacity) {
        error = fallback;
        capacity = sizeof fallback;
    }
    lunelette_metal_limits resolved = limits ? *limits : (lunelette_metal_limits){256, 256};
    if (!profile_supported(resolved)) {
        snprintf(error, capacity, "unsupported context/block profile");
        return NULL;
    }
    lunelette_metal_options selected;
    if (resolve_options(options, &selected, error, capacity)) {
        return NULL;
    }
    if (!config || config->layers < 1 || config->layers > LH_LAYERS) {
        snprintf(error, capacity, "synthetic model needs 1..26 layers");
        return NULL;
    }
    weight_source src = {synthetic_read, synthetic_scale, config->seed, NULL};
    return build_runtime(&src, config->layers, resolved, selected, error, capacity);
}

/* src/metal_runtime.m:199-330: profile, options, then the checkpoint
 * (container, tensor contract, scales) before any device allocation; FP8
 * codes are admitted tensor by tensor during the upload. */
lunelette_metal *lunelette_metal_create_configured(const char *path,
    const lunelette_metal_options *options, const lunelette_metal_limits *limits,
    char *error, size_t capacity)
{
    char fallback[512];
    if (!error || !capacity) {
        error = fallback;
        capacity = sizeof fallback;
    }
    lunelette_metal_limits resolved = limits ? *limits : (lunelette_metal_limits){256, 256};
    if (!profile_supported(resolved)) {
        snprintf(error, capacity, "unsupported context/block profile");
        return NULL;
    }
    lunelette_metal_options selected;
    if (resolve_options(options, &selected, error, capacity)) {
        return NULL;
    }
    lh_weights *checkpoint = malloc(sizeof *checkpoint);
    if (!checkpoint) {
        snprintf(error, capacity, "checkpoint handle allocation failed");
        return NULL;
    }
    if (lh_weights_open(checkpoint, path, error, capacity)) {
        free(checkpoint);
        return NULL;
    }
    weight_source src = {file_read, file_scale, 0, checkpoint};
    lunelette_metal *context = build_runtime(&src, LH_LAYERS, resolved, selected, error,
        capacity);
    lh_weights_close(checkpoint);
    free(checkpoint);
    return context;
}

lunelette_metal *lunelette_metal_create_with_options(const char *path,
    const lunelette_metal_options *options, char *error, size_t capacity)
{
    return lunelette_metal_create_configured(path, options, NULL, error, capacity);
}

lunelette_metal *lunelette_metal_create(const char *path, char *error, size_t capacity)
{
    return lunelette_metal_create_with_options(path, NULL, error, capacity);
}

void lunelette_metal_destroy(lunelette_metal *context)
{
    if (context) {
        destroy_runtime(context->rt);
        free(context);
    }
}

int lunelette_metal_get_limits(const lunelette_metal *context, lunelette_metal_limits *limits)
{
    if (!context || !context->rt || !limits) {
        return -1;
    }
    *limits = context->rt->limits;
    return 0;
}

int lunelette_metal_get_memory(const lunelette_metal *context, lunelette_metal_memory *memory)
{
    if (!context || !context->rt || !memory) {
        return -1;
    }
    *memory = context->rt->memory;
    return 0;
}

int lunelette_metal_reset(lunelette_metal *context, char *error, size_t capacity)
{
    lh_runtime *rt = context ? context->rt : NULL;
    if (!rt) {
        report(error, capacity, "%sreset requires a context", NULL);
        return -1;
    }
    rt->active_checkpoint = NULL;
    rt->endpoint_logits_valid = false;
    rt->length = 0;
    rt->valid = true;
    return 0;
}

static int select_path(const lh_runtime *rt, size_t count)
{
    if (count > 1 && rt->prefill_mode == LUNELETTE_METAL_PREFILL_MPS && LH_HAVE_MFMA &&
        rt->strategy != LUNELETTE_METAL_RESIDENT_FP32) {
        return LH_PATH_MFMA;
    }
    switch (rt->strategy) {
    case LUNELETTE_METAL_RESIDENT_FP32:
        return LH_PATH_RESIDENT;
    case LUNELETTE_METAL_COMPACT_FP8_LOOKUP:
        return LH_PATH_LOOKUP;
    default:
        return LH_PATH_FUSED;
    }
}

/* src/metal_runtime.m:349-432. */
/* Device work of one step: embedding gather, every layer, final norm + head. */
/* embed: gather the step's embedding rows first (a device-side decode step
 * has already written its row together with the step record). */
static int launch_step(lh_runtime *rt, size_t count, int path, int embed, hipStream_t s)
{
    const size_t per_layer = (size_t)LH_KV_HEADS * rt->limits.context * LH_HEAD_DIM;
    if (embed && lh_embed_forward(rt->d_embedding, rt->d_x, rt->ws, s)) {
        return -1;
    }
    for (uint32_t l = 0; l < rt->layers; l++) {
        float *keys = rt->d_keys + l * per_layer, *values = rt->d_values + l * per_layer;
        int rc;
        if (path == LH_PATH_MFMA) {
            /* Each layer's last kernel also splits the next layer's input. */
            const float *next = l + 1 < rt->layers ? rt->layer[l + 1].input_norm : NULL;
            rc = lh_layer_forward_mfma(&rt->layer[l], rt->d_x, keys, values, rt->ws, l > 0, next,
                s);
        } else {
            rc = lh_layer_forward(&rt->layer[l], rt->d_x, keys, values, rt->ws, path, s);
        }
        if (rc) {
            return -1;
        }
        if (rt->fault.after_layer == l + 1) {
            rt->fault.after_layer = 0;
            lh_set_error("injected launch failure after layer %u", l);
            return -1;
        }
    }
    return lh_head_forward_checked(rt->d_embedding, rt->d_norms + 2ull * rt->layers * LH_HIDDEN,
        rt->d_x + (count - 1) * LH_HIDDEN, rt->d_logits, rt->d_nonfinite, s);
}

static int execute(lunelette_metal *context, const int64_t *ids, size_t count, bool prefill,
    const float **logits, char *error, size_t capacity)
{
    char fallback[512];
    if (!error || !capacity) {
        error = fallback;
        capacity = sizeof fallback;
    }
    if (logits) {
        *logits = NULL;
    }
    lh_runtime *rt = context ? context->rt : NULL;
    if (!rt || !logits || !ids || !count || count > rt->limits.block ||
        count > rt->limits.context || !rt->valid || rt->length > rt->limits.context - count ||
        (prefill ? rt->length != 0 : rt->length == 0)) {
        snprintf(error, capacity, "sequence rejected: require reset/valid IDs and configured "
            "block/context capacity");
        return -1;
    }
    for (size_t i = 0; i < count; i++) {
        if (ids[i] < 0 || ids[i] >= LH_VOCAB) {
            snprintf(error, capacity, "invalid token ID at position %zu", i);
            return -1;
        }
    }
    /* Withdraw before any device work; a successful call republishes the
     * checkpoint, a failed one leaves it invalid. */
    lunelette_metal_checkpoint *checkpoint = rt->active_checkpoint;
    rt->active_checkpoint = NULL;
    rt->endpoint_logits_valid = false;
    rt->valid = false;
    if (rt->fault.before_device) {
        rt->fault.before_device = false;
        snprintf(error, capacity, "execution failed; reset required: injected launch failure");
        return -1;
    }
    hipStream_t s = rt->stream;
    /* A decode step writes its record on the device (no host upload). */
    const int device_record = count == 1;
    if (!device_record && lh_workspace_set_tokens(rt->ws, ids, rt->length, count, s)) {
        snprintf(error, capacity, "step parameters failed; reset required: %s", lh_last_error());
        return -1;
    }
    const int path = select_path(rt, count);
    /* The head kernel sets the flag on an Inf/NaN logit; the host then scans
     * only to name the first one. */
    *rt->h_nonfinite = 0;
    rt->ws->handoff_fault = rt->fault.handoff;
    rt->fault.handoff = 0;
    int failed = hipEventRecord(rt->started, s) != hipSuccess ||
        (device_record &&
            lh_workspace_set_decode(rt->ws, rt->d_embedding, ids[0], rt->length, rt->d_x, s)) ||
        launch_step(rt, count, path, !device_record, s) ||
        hipEventRecord(rt->finished, s) != hipSuccess;
    hipError_t status = hipStreamSynchronize(s);
    rt->ws->handoff_fault = 0;
    if (failed || status != hipSuccess) {
        snprintf(error, capacity, "execution failed; reset required: %s",
            failed ? lh_last_error() : hipGetErrorString(status));
        lh_workspace_clear_arrivals(rt->ws);
        return -1;
    }
    if (hipEventElapsedTime(&rt->last_ms, rt->started, rt->finished) != hipSuccess) {
        rt->last_ms = -1.0f;
    }
    if (rt->fault.nonfinite) {
        rt->fault.nonfinite = false;
        rt->h_logits[LH_VOCAB - 1] = INFINITY;
        *rt->h_nonfinite = 1;
    }
    const size_t bad = *rt->h_nonfinite ? lh_first_nonfinite(rt->h_logits, LH_VOCAB) : LH_VOCAB;
    if (bad < LH_VOCAB) {
        snprintf(error, capacity, "nonfinite logit %zu; reset required", bad);
        lh_workspace_clear_arrivals(rt->ws);
        return -1;
    }
    rt->length += count;
    rt->valid = true;
    rt->endpoint_logits_valid = true;
    rt->active_checkpoint = checkpoint;
    *logits = rt->h_logits;
    return 0;
}

int lunelette_metal_prefill(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity)
{
    return execute(context, ids, count, true, logits, error, capacity);
}

int lunelette_metal_decode(lunelette_metal *context, int64_t token, const float **logits,
    char *error, size_t capacity)
{
    return execute(context, &token, 1, false, logits, error, capacity);
}

int lunelette_metal_append(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity)
{
    return execute(context, ids, count, false, logits, error, capacity);
}

/* src/metal_runtime.m:494-538. */
int lunelette_metal_checkpoint_create(lunelette_metal *context,
    lunelette_metal_checkpoint **checkpoint, char *error, size_t capacity)
{
    if (checkpoint) {
        *checkpoint = NULL;
    }
    lh_runtime *rt = context ? context->rt : NULL;
    if (!rt || !checkpoint || !rt->identity || !rt->valid || !rt->endpoint_logits_valid ||
        !rt->length || rt->length > rt->limits.context || rt->checkpoint_epoch == UINT64_MAX) {
        report(error, capacity, "%scheckpoint requires valid endpoint/available epoch", NULL);
        return -1;
    }
    const size_t bad = lh_first_nonfinite(rt->h_logits, LH_VOCAB);
    if (bad < LH_VOCAB) {
        if (error && capacity) {
            snprintf(error, capacity, "checkpoint nonfinite logit %zu", bad);
        }
        rt->valid = false;
        rt->endpoint_logits_valid = false;
        rt->active_checkpoint = NULL;
        return -1;
    }
    lunelette_metal_checkpoint *saved = NULL;
    if (rt->fault.checkpoint_alloc) {
        rt->fault.checkpoint_alloc = false;
    } else {
        saved = malloc(sizeof *saved);
    }
    if (!saved) {
        report(error, capacity, "%scheckpoint allocation failed", NULL);
        return -1;
    }
    saved->owner = rt;
    saved->identity = rt->identity;
    saved->epoch = rt->checkpoint_epoch + 1;
    saved->length = rt->length;
    memcpy(saved->logits, rt->h_logits, sizeof saved->logits);
    rt->checkpoint_epoch = saved->epoch;
    rt->active_checkpoint = saved;
    *checkpoint = saved;
    return 0;
}

/* src/metal_runtime.m:540-564. */
int lunelette_metal_checkpoint_restore(lunelette_metal *context,
    const lunelette_metal_checkpoint *checkpoint, const float **logits, char *error,
    size_t capacity)
{
    if (logits) {
        *logits = NULL;
    }
    lh_runtime *rt = context ? context->rt : NULL;
    if (!rt || !logits || !checkpoint || rt->active_checkpoint != checkpoint ||
        checkpoint->identity != rt->identity || checkpoint->epoch != rt->checkpoint_epoch ||
        !rt->valid || rt->length > rt->limits.context || !checkpoint->length ||
        checkpoint->length > rt->limits.context || checkpoint->length > rt->length) {
        report(error, capacity, "%scheckpoint stale, invalid or wrong context", NULL);
        return -1;
    }
    memcpy(rt->h_logits, checkpoint->logits, sizeof checkpoint->logits);
    rt->length = checkpoint->length;
    rt->endpoint_logits_valid = true;
    *logits = rt->h_logits;
    return 0;
}

void lunelette_metal_checkpoint_destroy(lunelette_metal_checkpoint *checkpoint)
{
    if (checkpoint) {
        lh_runtime *rt = checkpoint->owner;
        if (rt && rt->active_checkpoint == checkpoint) {
            rt->active_checkpoint = NULL;
        }
        free(checkpoint);
    }
}

int lunelette_metal_last_device_ms(const lunelette_metal *context, float *milliseconds)
{
    if (!context || !context->rt || !milliseconds) {
        return -1;
    }
    *milliseconds = context->rt->last_ms;
    return 0;
}

int lunelette_metal_read_kv(const lunelette_metal *context, size_t layer, int kind,
    size_t position, size_t count, float *out)
{
    const lh_runtime *rt = context ? context->rt : NULL;
    if (!rt || !out || layer >= rt->layers || (kind != 0 && kind != 1) ||
        position > rt->limits.context || count > rt->limits.context - position) {
        return -1;
    }
    const size_t C = rt->limits.context;
    const float *base = (kind ? rt->d_values : rt->d_keys) + (size_t)layer * LH_KV_HEADS * C *
        LH_HEAD_DIM;
    if (kind) {
        /* V rows are contiguous per kv head: one strided copy per head into
         * the position-major output. */
        if (!count) {
            return 0;
        }
        for (size_t h = 0; h < LH_KV_HEADS; h++) {
            const float *src = base + lh_kv_index(C, 0, (uint32_t)h, position);
            if (hipMemcpy2D(out + h * LH_HEAD_DIM, LH_KV * sizeof(float), src,
                    LH_HEAD_DIM * sizeof(float), LH_HEAD_DIM * sizeof(float), count,
                    hipMemcpyDeviceToHost) != hipSuccess) {
                return -1;
            }
        }
        return 0;
    }
    /* K: copy each 64-position tile the range touches, then gather its rows
     * out of the tile's word order. */
    float tile[LH_ATTN_BLOCK * LH_HEAD_DIM];
    for (size_t h = 0; h < LH_KV_HEADS; h++) {
        for (size_t t0 = position & ~(size_t)63; t0 < position + count; t0 += LH_ATTN_BLOCK) {
            if (hipMemcpy(tile, base + lh_kv_index(C, 0, (uint32_t)h, t0), sizeof tile,
                    hipMemcpyDeviceToHost) != hipSuccess) {
                return -1;
            }
            for (size_t p = t0 < position ? position : t0;
                 p < t0 + LH_ATTN_BLOCK && p < position + count; p++) {
                for (uint32_t d = 0; d < LH_HEAD_DIM; d++) {
                    out[(p - position) * LH_KV + h * LH_HEAD_DIM + d] =
                        tile[lh_ktile_word((uint32_t)(p - t0), d >> 5, (d >> 2) & 7) * 4 + (d & 3)];
                }
            }
        }
    }
    return 0;
}

/* Host-forced faults (lh_internal.h). Only the test-seam library calls these;
 * the shipped library exports neither. */
int lh_runtime_fault(lunelette_metal *context, int kind, uint64_t arg)
{
    lh_runtime *rt = context ? context->rt : NULL;
    if (!rt) {
        return -1;
    }
    switch (kind) {
    case LH_FAULT_BEFORE_DEVICE:
        rt->fault.before_device = true;
        return 0;
    case LH_FAULT_NONFINITE:
        rt->fault.nonfinite = true;
        return 0;
    case LH_FAULT_CHECKPOINT_ALLOC:
        rt->fault.checkpoint_alloc = true;
        return 0;
    case LH_FAULT_AFTER_LAYER:
        if (arg >= rt->layers) {
            return -1;
        }
        rt->fault.after_layer = (uint32_t)arg + 1;
        return 0;
    case LH_FAULT_EPOCH:
        rt->checkpoint_epoch = arg;
        return 0;
    case LH_FAULT_HANDOFF:
        rt->fault.handoff = LH_HANDOFF_BLOCKS;
        return 0;
    case LH_FAULT_COMBINERS:
        rt->fault.handoff = LH_HANDOFF_COMBINERS;
        return 0;
    default:
        return -1;
    }
}

int lh_runtime_set_logit(lunelette_metal *context, size_t index, float value)
{
    if (!context || !context->rt || index >= LH_VOCAB) {
        return -1;
    }
    context->rt->h_logits[index] = value;
    return 0;
}
