/* Workspace layout shared by layer.c, the MFMA path and the runtime. */
#ifndef LH_LAYER_H
#define LH_LAYER_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "lunelette_kernels.h"
#include "lh_schedule.h"

struct lh_workspace {
    size_t capacity, block;
    size_t length, count;          /* set by lh_workspace_set_tokens */
    uint64_t bytes;                /* device bytes owned */
    lh_step_params *h_params;      /* pinned */
    lh_step_params *d_params;
    float *d_q, *d_attn;           /* [B][4096] */
    float *d_gated, *d_up;         /* [B][9216] */
    float *d_xn;                   /* [B][3072] */
    float *d_qraw, *d_kraw, *d_vraw;
    float *d_PM, *d_PT;            /* [B][32][C/64] block maxima and sums */
    float *d_PA;                   /* [B][32][C/64][128] block P.V partials */
    unsigned long long *d_arrive;  /* one-launch attention: B * 8 arrival words 256 B apart,
                                      then 512 producer flags (ARRIVE_WORDS) */
    unsigned long long *d_bflags;  /* [8][C/64] block flags of one-launch long attention */
    unsigned long long epoch;      /* last epoch stored in the producer and block flags */
    int handoff_fault;             /* test build: LH_HANDOFF_* wait of the next launches gives up */
    float *d_yarn;                 /* [C][128]: cos[64], sin[64] per position (decode) */
    float *h_yarn;                 /* host copy of the same rows, filled on first use */
    uint8_t *h_yarn_ready;         /* [C]: row p of h_yarn holds lh_yarn(p) */
    /* MFMA path: BF16 hi/mid/lo splits of the GEMM inputs, [3][B][K]. */
    uint16_t *d_split;
    float *d_gemm;                 /* [B][18432] GEMM outputs */
};

#ifdef __cplusplus
extern "C" {
#endif
/* Multi-token layer with MFMA GEMM projections (mfma.hip). input_split: the
 * workspace split already holds input_norm(x) (written by the previous layer
 * called with next_norm = this layer's input norm); next_norm: also leave the
 * split of next_norm(x) for the following layer (NULL for the last layer). */
int lh_layer_forward_mfma(const lh_layer_weights *w, float *d_x, float *d_keys,
    float *d_values, lh_workspace *ws, int input_split, const float *next_norm, hipStream_t s);
/* Allocates the MFMA path's extra workspace buffers (idempotent). */
int lh_mfma_prepare(lh_workspace *ws);
/* Returns the one-launch attention's arrival words to zero (after a failed
 * step, whose launches may have left them mid-count). Synchronous. */
int lh_workspace_clear_arrivals(lh_workspace *ws);
/* Builds the device YaRN table of every position below the capacity from the
 * host YaRN (idempotent), for lh_workspace_set_decode. */
int lh_workspace_prepare_decode(lh_workspace *ws);
/* A single-token step without a host upload: one kernel writes the step
 * record (position length, the table's cos/sin, the query factor) and the
 * embedding row of id into d_x, on stream. */
int lh_workspace_set_decode(lh_workspace *ws, const uint16_t *d_embedding, int64_t id,
    size_t length, float *d_x, hipStream_t s);
#ifdef __cplusplus
}
#endif

#endif
