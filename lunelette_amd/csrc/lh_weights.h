/* Safetensors container reader and the checkpoint tensor contract of the
 * Ministral-3B-shaped FP8 text model (replaces src/safetensors.c and the
 * validation half of src/metal_weights.c). Host C only. */
#ifndef LH_WEIGHTS_H
#define LH_WEIGHTS_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "lh_schedule.h"

#define LH_ST_MAX_DIMS 8
#define LH_ST_MAX_NAME 256          /* names hold at most 255 characters */
#define LH_ST_MAX_TENSORS 4096
#define LH_ST_MAX_HEADER (1u << 20)

/* Element types; the value is the element size in bytes. */
typedef enum {
    LH_ST_F8_E4M3 = 1,
    LH_ST_BF16 = 2,
    LH_ST_F32 = 4,
    LH_ST_I64 = 8
} lh_st_dtype;

typedef struct {
    char name[LH_ST_MAX_NAME];
    lh_st_dtype dtype;
    uint32_t rank;
    uint64_t shape[LH_ST_MAX_DIMS];
    uint64_t begin, end;            /* byte range inside the data section */
} lh_st_tensor;

typedef struct {
    FILE *file;
    uint64_t base;                  /* file offset of the data section */
    size_t count;
    lh_st_tensor *tensors;          /* header order */
} lh_st_file;

/* Opens and fully validates the container (header grammar, unique names,
 * dtypes, shapes, sizes, and a data section tiled exactly by the non-empty
 * tensors). 0, or -1 with a diagnostic and *f cleared. */
int lh_st_open(lh_st_file *f, const char *path, char *error, size_t capacity);
void lh_st_close(lh_st_file *f);
const lh_st_tensor *lh_st_find(const lh_st_file *f, const char *name);
/* Bounded read of bytes [offset, offset + bytes) of a tensor of f. */
int lh_st_read(lh_st_file *f, const lh_st_tensor *t, uint64_t offset, void *out, size_t bytes);

/* Checkpoint slots in the reference order (src/metal_weights.h): 0 embedding,
 * 1 final norm, then 2 + 9*layer + {input norm, q, k, v, o, post norm, gate,
 * up, down}. */
#define LH_WEIGHT_SLOTS (2 + LH_LAYERS * 9)

typedef struct {
    lh_st_file file;
    struct {
        const lh_st_tensor *tensor;
        float scale;                /* weight_scale_inv for FP8 slots, 1 otherwise */
    } slot[LH_WEIGHT_SLOTS];
} lh_weights;

/* Opens path, checks every expected tensor (dtype, rank, shape, the two BF16
 * scalar companions of each FP8 matrix), rejects unknown language_model.*
 * tensors and reads the scales (positive finite). */
int lh_weights_open(lh_weights *w, const char *path, char *error, size_t capacity);
void lh_weights_close(lh_weights *w);

#endif
