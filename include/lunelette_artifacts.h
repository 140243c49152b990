/* Native logit-regression artifacts (LUN1/LUN2) over the runtime C-ABI.
 *
 * Replaces the reference's native regression runner and its offline reader,
 * tests/compare_native.c (format and metrics :22-150, offline file check
 * :154-194, capture/check over a runtime :348-450; strategy identity
 * tests/comparator_strategy.h:8-64), for the same files:
 *   uint32 LE magic 0x324e554c ("LUN2") or 0x314e554c ("LUN1", no strategy
 *   word, resident only), [LUN2: strategy 0..2], mode (0 MPS, 1 custom),
 *   context 256, prompt count, steps 8, vocabulary 131072, the prompt ids,
 *   the 8 forced ids, then 8 vectors of 131072 IEEE binary32 logits: step 0
 *   after the prefill of the prompt, step k after the decode of forced[k-1].
 * Acceptance is strict: finite vectors on both sides, bitwise equal, the same
 * top-1 id and the same top-5/20/64 sets (ties ranked by lower id).
 */
#ifndef LUNELETTE_ARTIFACTS_H
#define LUNELETTE_ARTIFACTS_H

#include <stddef.h>
#include <stdint.h>

#include "lunelette_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LUNELETTE_NATIVE_STEPS 8
#define LUNELETTE_NATIVE_CONTEXT 256
#define LUNELETTE_NATIVE_MAX_PROMPT 248
#define LUNELETTE_NATIVE_LUN1 0x314e554cu
#define LUNELETTE_NATIVE_LUN2 0x324e554cu

/* tests/compare_native.c:69-96: per-vector comparison figures; intersections
 * count shared ids among the two top-k lists. */
typedef struct {
    size_t finite_a, finite_b;
    int exact;
    size_t top1_a, top1_b;
    size_t top5, top20, top64;
    double max_abs, rms, cosine;
} lunelette_logit_metrics;

/* One artifact's identity: format (LUNELETTE_NATIVE_LUN1 or _LUN2), strategy,
 * prefill mode (0 MPS, 1 custom) and the teacher-forced trajectory. */
typedef struct {
    uint32_t magic;
    lunelette_metal_strategy strategy;
    uint32_t mode;
    size_t count;
    int64_t ids[LUNELETTE_NATIVE_MAX_PROMPT];
    int64_t forced[LUNELETTE_NATIVE_STEPS];
} lunelette_native_trajectory;

/* tests/compare_native.c:41-56: the 64 highest values in rank order, ties by
 * lower index (count >= 64). */
void lunelette_logits_top64(const float *values, size_t count, size_t ids[64]);

/* tests/compare_native.c:69-96: fills *metrics; 0 when accepted under the
 * strict rule above, 1 otherwise. */
int lunelette_logits_compare(const float *a, const float *b, size_t count,
    lunelette_logit_metrics *metrics);

/* Creates path exclusively (an existing file fails) and writes the header and
 * the 8 vectors logits[8][131072]; a nonfinite logit or a LUN1 file of a
 * compact strategy fails. 0 on success. */
int lunelette_native_write(const char *path, const lunelette_native_trajectory *trajectory,
    const float *logits, char *error, size_t capacity);

/* Reads a whole artifact: its header must match trajectory (format, strategy,
 * mode, ids), every vector must be finite and no byte may follow. logits may
 * be NULL (validation only). 0 on success. */
int lunelette_native_read(const char *path, const lunelette_native_trajectory *trajectory,
    float *logits, char *error, size_t capacity);

/* tests/compare_native.c:154-194 (--files): takes the trajectory from the
 * left file, validates both headers against it for the requested mode,
 * prompt count (1..248) and strategy (a LUN1 file counts as resident),
 * compares the 8 steps in order (metrics[0..7], filled up to the first
 * failing step) and requires both files to end there. 0 when accepted. */
int lunelette_native_compare_files(const char *left, const char *right, uint32_t mode,
    size_t count, lunelette_metal_strategy strategy, lunelette_logit_metrics *metrics,
    char *error, size_t capacity);

/* tests/compare_native.c:348-450 for one artifact: the runtime must report
 * trajectory->strategy. Capture (check = 0) resets, prefills the prompt and
 * decodes forced[0..6], and writes the 8 vectors to a new file. Check
 * (check = 1) validates the file first, then runs the trajectory twice from
 * a reset and requires every vector to equal the file's (metrics[0..15]).
 * The runtime's context must hold count + 7 tokens. 0 on success. */
int lunelette_native_run(lunelette_metal *runtime, const char *path,
    const lunelette_native_trajectory *trajectory, int check, lunelette_logit_metrics *metrics,
    char *error, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif
