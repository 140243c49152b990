/* Lunelette runtime C-ABI on one MI355X (gfx950, HIP).
 *
 * Drop-in for the reference runtime contract include/metal.h:11-120: the same
 * opaque types, enums, structs, macros and functions, with the same argument
 * meaning, ownership and error behaviour, so src/main.c, service/native.c and
 * the comparators link against this library unchanged.
 * No HIP, torch or C++ types cross this API.
 *
 * Single caller per context: no concurrent calls on one context, including
 * destroy/reset (include/metal.h:8-9). One context owns its weights, scratch,
 * KV cache and borrowed logits.
 */
#ifndef LUNELETTE_RUNTIME_H
#define LUNELETTE_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lunelette_metal lunelette_metal;
typedef struct lunelette_metal_checkpoint lunelette_metal_checkpoint;

/* include/metal.h:17-18. Opens one official mixed FP8/BF16 model.safetensors.
 * NULL on failure with a diagnostic when error/capacity permit. */
lunelette_metal *lunelette_metal_create(const char *path, char *error, size_t capacity);

/* include/metal.h:19-22. MPS selects the MFMA block GEMM for multi-token calls;
 * CUSTOM selects the precise FP32 path (decode-schedule row dots). */
typedef enum {
    LUNELETTE_METAL_PREFILL_MPS = 0,
    LUNELETTE_METAL_PREFILL_CUSTOM = 1
} lunelette_metal_prefill_mode;

/* include/metal.h:24-28. RESIDENT_FP32 stores the exact FP32 decode of every
 * code in HBM; COMPACT_FP8_ARITHMETIC keeps FP8 codes and decodes in
 * registers; COMPACT_FP8_LOOKUP decodes through an unscaled 256-entry table.
 * All three multiply each row total by the per-tensor scale, so on weights
 * every strategy admits they give bitwise identical results. Admission
 * follows the reference per strategy: compact needs a positive, normal,
 * BF16-exact scale, finite codes and normal nonzero products
 * (src/metal_weights.c:174-231); resident needs a positive finite scale and
 * finite products (st_load_fp8, src/safetensors.c:521-548), so subnormal
 * scales and products load resident but not compact. */
typedef enum {
    LUNELETTE_METAL_RESIDENT_FP32 = 0,
    LUNELETTE_METAL_COMPACT_FP8_ARITHMETIC = 1,
    LUNELETTE_METAL_COMPACT_FP8_LOOKUP = 2
} lunelette_metal_strategy;

/* include/metal.h:30-36. */
typedef struct {
    lunelette_metal_prefill_mode prefill;
    lunelette_metal_strategy strategy;
} lunelette_metal_options;

#define LUNELETTE_METAL_OPTIONS_DEFAULT \
    { LUNELETTE_METAL_PREFILL_MPS, LUNELETTE_METAL_COMPACT_FP8_ARITHMETIC }

/* include/metal.h:55-56. NULL options selects the default macro; invalid enum
 * values fail before any file or device work. */
lunelette_metal *lunelette_metal_create_with_options(const char *path,
    const lunelette_metal_options *options, char *error, size_t capacity);

/* include/metal.h:60-65. NULL limits selects C256/B256. Supported pairs:
 * 256/256, 4352/256, 4352/128 (reference) plus the additive long profiles
 * 17920/256 and 17920/128. */
typedef struct {
    size_t context, block;
} lunelette_metal_limits;
lunelette_metal *lunelette_metal_create_configured(const char *path,
    const lunelette_metal_options *options, const lunelette_metal_limits *limits,
    char *error, size_t capacity);

/* include/metal.h:67. Nonmutating; NULL arguments fail. */
int lunelette_metal_get_limits(const lunelette_metal *context, lunelette_metal_limits *limits);

/* include/metal.h:71-75. Named owned device allocations only. */
typedef struct {
    lunelette_metal_strategy strategy;
    uint64_t weight_bytes, conversion_stage_bytes, scratch_bytes, kv_bytes, total_bytes;
} lunelette_metal_memory;
int lunelette_metal_get_memory(const lunelette_metal *context, lunelette_metal_memory *memory);

/* include/metal.h:76. destroy(NULL) is allowed. */
void lunelette_metal_destroy(lunelette_metal *context);

/* include/metal.h:78-79. Makes old cache tails inaccessible; no device work. */
int lunelette_metal_reset(lunelette_metal *context, char *error, size_t capacity);

/* include/metal.h:81-93. Prefill: empty valid sequence, 1..B ids, length<=C.
 * Decode: one token on a nonempty sequence of length < C. On success *logits
 * borrows 131072 FP32 host values until the next mutating call; on failure it
 * is NULL. Argument errors leave the context untouched; execution, allocation
 * or nonfinite failures invalidate the sequence until reset. */
int lunelette_metal_prefill(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity);
int lunelette_metal_decode(lunelette_metal *context, int64_t token,
    const float **logits, char *error, size_t capacity);

/* include/metal.h:95-100. One block per call, count<=B, length+count<=C. */
int lunelette_metal_append(lunelette_metal *context, const int64_t *ids, size_t count,
    const float **logits, char *error, size_t capacity);

/* include/metal.h:102-120. One active handle per context; handles own a
 * finite logit copy (not KV), are caller-owned and destroyed before the
 * context. Restore rewinds length and copies the saved logits with no device
 * work. */
int lunelette_metal_checkpoint_create(lunelette_metal *context,
    lunelette_metal_checkpoint **checkpoint, char *error, size_t capacity);
int lunelette_metal_checkpoint_restore(lunelette_metal *context,
    const lunelette_metal_checkpoint *checkpoint, const float **logits,
    char *error, size_t capacity);
void lunelette_metal_checkpoint_destroy(lunelette_metal_checkpoint *checkpoint);

/* ---- Additive (no counterpart in include/metal.h) ---- */

/* Seeded random-init model of the same architecture: FP8 codes drawn
 * uniformly from the 254 finite E4M3FN codes, per-tensor BF16-exact scales in
 * [0.01, 0.02], BF16 norms 1+N(0,0.02), BF16 embedding N(0,0.02). layers in
 * 1..26 (26 is the model; fewer only for quick tests). Bytes are generated by
 * lh_synth_* (include/lunelette_kernels.h), so a host copy is reproducible. */
typedef struct {
    uint64_t seed;
    uint32_t layers;
} lunelette_synthetic_config;
lunelette_metal *lunelette_metal_create_synthetic(const lunelette_synthetic_config *config,
    const lunelette_metal_options *options, const lunelette_metal_limits *limits,
    char *error, size_t capacity);

/* Device milliseconds of the last successful prefill/decode/append (stream
 * events around the model work, excluding the logits copy). */
int lunelette_metal_last_device_ms(const lunelette_metal *context, float *milliseconds);

/* Copies KV rows [position, position+count) of one layer and kind (0 K, 1 V)
 * to host, [count][1024] in the reference's position-major layout. */
int lunelette_metal_read_kv(const lunelette_metal *context, size_t layer, int kind,
    size_t position, size_t count, float *out);

#ifdef __cplusplus
}
#endif

#endif
