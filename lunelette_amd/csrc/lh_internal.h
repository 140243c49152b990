/* Internal launchers between the C runtime and the gfx950 kernels. Device
 * pointers only; every launcher returns 0 or -1 (launch error). */
#ifndef LH_INTERNAL_H
#define LH_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "lh_schedule.h"

#ifdef __cplusplus
extern "C" {
#endif

/* kind: 0 FP8 codes (scaled), 1 BF16, 2 FP32. residual may be NULL. */
int lh_launch_matvec(int kind, int lookup, const void *W, float scale, const float *x, float *y,
    const float *residual, uint32_t rows, uint32_t cols, uint32_t tokens, hipStream_t s);
int lh_launch_qkv_rope(int lookup, const uint8_t *Wqkv, float sq, float sk, float sv,
    const float *gamma, const float *x, const lh_step_params *params, uint32_t count,
    float *q, float *kcache_layer, float *vcache_layer, uint32_t capacity, hipStream_t s);
int lh_launch_gateup_silu(int lookup, const uint8_t *Wgate, const uint8_t *Wup, float sg,
    float su, const float *gamma, const float *x, uint32_t count, float *gated, hipStream_t s);
/* nonfinite (may be NULL) is set to 1 when any written logit is Inf or NaN. */
int lh_launch_head(const uint16_t *E, const float *gamma, const float *xrow, float *logits,
    uint32_t *nonfinite, hipStream_t s);
int lh_launch_rmsnorm(const float *gamma, const float *x, float *out, uint32_t width,
    uint32_t tokens, hipStream_t s);
/* Query token t attends positions [0, params->length + t]; length (equal to
 * params->length) sizes the block grid only. */
int lh_launch_attention(const float *q, const float *kcache_layer, const float *vcache_layer,
    const lh_step_params *params, uint32_t length, uint32_t count, uint32_t capacity, float *PM,
    float *PT, float *PA, unsigned long long *arrive, unsigned long long *bflags,
    unsigned long long epoch, int fault, float *out, hipStream_t s);
/* Whether a decode token at this length runs q|k|v and its attention blocks
 * in one launch on the current device (its dispatch probed). */
int lh_attention_chained(uint32_t length);
/* One decode token: RMSNorm -> q|k|v -> RoPE -> KV append, the attention
 * blocks and their combine in one launch; arrive: the blocks' arrival words
 * (zeroed, left zeroed); flags: 512 producer flags; bflags: 8 * capacity/64
 * block flags; epoch nonzero and new for every launch on them. Needs
 * lh_attention_chained(length). */
int lh_launch_qkv_attention(int lookup, const uint8_t *Wqkv, float sq, float sk, float sv,
    const float *gamma, const float *x, const lh_step_params *params, uint32_t length, float *q,
    float *kcache_layer, float *vcache_layer, uint32_t capacity, float *PM, float *PT, float *PA,
    unsigned long long *arrive, unsigned long long *flags, unsigned long long *bflags,
    unsigned long long epoch, int fault, float *out, hipStream_t s);
/* Records once per device whether a launch's workgroups whose ids agree mod 8
 * run on one XCD (five probe launches into d_words, at least 2048 words, left
 * zeroed); *ok receives the verdict. A fused attention launch needs it. */
int lh_attention_xcd_probe(uint32_t *d_words, size_t words, int *ok, hipStream_t s);
/* Matrix-core attention for multi-token steps (tolerance path). With xs set
 * the output goes to the two scaled FP16 planes of xs (token stride
 * xs_tokens, the o projection's input) instead of FP32 rows of out, with
 * xs_scale[t][kv head] = 2^-e for the planes of token t's 512 columns of that
 * kv head's query heads. */
int lh_launch_attention_mfma(const float *q, const float *kcache_layer, const float *vcache_layer,
    const lh_step_params *params, uint32_t length, uint32_t count, uint32_t capacity, float *PM,
    float *PT, float *PA, float *out, uint16_t *xs, uint32_t xs_tokens, float *xs_scale,
    hipStream_t s);
/* Block-grid width of the attention kernel. */
uint32_t lh_attention_blocks(uint32_t length, uint32_t count);
int lh_launch_embed(const uint16_t *E, const lh_step_params *params, uint32_t count, float *x,
    hipStream_t s);
/* One decode token: writes params (length, count 1, id, qfactor, cos/sin of
 * position length from yarn [C][128]) and the widened embedding row of id. */
int lh_launch_step_embed(const uint16_t *E, const float *yarn, int32_t id, uint32_t length,
    float qfactor, lh_step_params *params, float *x, hipStream_t s);
int lh_launch_element(int mode, const float *a, const float *b, float *out, size_t n,
    hipStream_t s);
int lh_launch_silu_mul(const float *gate, const float *up, float *out, size_t n, hipStream_t s);
int lh_launch_rope(const float *x, const float *cosine, const float *sine, const float *qfactor,
    float *out, uint32_t width, uint32_t tokens, hipStream_t s);
/* q [count][4096], k/v [count][1024] raw projections. */
int lh_launch_rope_append(const float *q_raw, const float *k_raw, const float *v_raw,
    const lh_step_params *params, uint32_t count, float *q, float *kcache_layer,
    float *vcache_layer, uint32_t capacity, hipStream_t s);
int lh_launch_fp8_decode(const uint8_t *codes, float *out, size_t n, hipStream_t s);
/* Streaming read of bytes (a multiple of grid*4*64*16*unroll; unroll 1, 2, 4, 8). */
int lh_launch_read_floor(const void *src, size_t bytes, uint32_t grid, uint32_t unroll,
    uint32_t *sink, hipStream_t s);
int lh_launch_expf(const float *x, float *out, size_t n, hipStream_t s);

/* Thread-local diagnostic shared by the C ABI layers. */
void lh_set_error(const char *format, ...);

/* Every device and pinned-host allocation of the library goes through these
 * (api.c). They count allocations and frees (relaxed atomics: contexts may be
 * created and destroyed on different threads), and fail the nth allocation
 * after the counter was armed: the host-forced allocation failure of the
 * reference's tests (tests/test_metal.m:888-954). Only the test-seam library
 * (test_seams.c, not part of the shipped library) arms it. */
hipError_t lh_dev_malloc(void **ptr, size_t bytes);
hipError_t lh_host_malloc(void **ptr, size_t bytes, unsigned flags);
void lh_dev_free(void *ptr);
void lh_host_free(void *ptr);
/* Arms the counter: the nth allocation from now fails (1-based; 0 never). */
void lh_allocations_arm(unsigned nth);
/* Allocations since the counter was armed, and allocations not yet freed. */
unsigned lh_allocations_count(void);
long lh_allocations_live(void);

/* Host-forced execution faults of one runtime context (runtime.c), set only
 * by the test-seam library: the analogue of the reference's mocked command
 * failures (tests/test_metal.m:629-860). */
enum {
    LH_FAULT_BEFORE_DEVICE = 1,    /* next execution fails before any device work */
    LH_FAULT_NONFINITE = 2,        /* next execution publishes an Inf logit */
    LH_FAULT_CHECKPOINT_ALLOC = 3, /* next checkpoint allocation fails */
    LH_FAULT_AFTER_LAYER = 4,      /* next execution fails after layer arg's kernels ran */
    LH_FAULT_EPOCH = 5,            /* checkpoint epoch counter set to arg */
    LH_FAULT_HANDOFF = 6,          /* next execution's one-launch attention blocks give up */
    LH_FAULT_COMBINERS = 7         /* next execution's attention flag combiners give up */
};
/* The workspace's handoff_fault (test build): which bounded wait of the next
 * execution's attention launches waits for an epoch nobody stores, and so
 * gives up after LH_GIVE_UP_POLLS polls and writes NaN. */
enum { LH_HANDOFF_BLOCKS = 1, LH_HANDOFF_COMBINERS = 2 };
#define LH_GIVE_UP_POLLS 64
struct lunelette_metal;
int lh_runtime_fault(struct lunelette_metal *context, int kind, uint64_t arg);
int lh_runtime_set_logit(struct lunelette_metal *context, size_t index, float value);

#ifdef __cplusplus
}
#endif

#endif
