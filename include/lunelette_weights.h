/* Checkpoint metadata without a runtime: the caller-facing part of the
 * reference's src/metal_weights.h:10-20 and :39, which src/main.c:186-193
 * uses to validate a checkpoint for requests that need no logits step.
 *
 * open runs the safetensors container rules (src/safetensors.c) and the
 * model's tensor contract with its scale companions (src/metal_weights.c:
 * 51-158), the same checks lunelette_metal_create* run before any device
 * allocation; 0 on success, -1 with a diagnostic (NULL/0 error allowed).
 * The handle is caller-allocated and its contents private; open always
 * initializes it, so close is safe after a failed open and on a zeroed
 * handle. */
#ifndef LUNELETTE_WEIGHTS_H
#define LUNELETTE_WEIGHTS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    void *opened;
} lunelette_metal_weights;

int lunelette_metal_weights_open(lunelette_metal_weights *weights, const char *path,
    char *error, size_t capacity);
void lunelette_metal_weights_close(lunelette_metal_weights *weights);

#ifdef __cplusplus
}
#endif

#endif
