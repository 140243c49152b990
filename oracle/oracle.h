/* CPU oracle for the Lunelette forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (lunelette_amd/, include/)
 * links, loads or calls this code. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, to check results against.
 *
 * Two schedules are restated for every reduction:
 *   - ORC_REF    ("ref-literal"): the reference's own arithmetic order where the
 *     reference fixes it. Per-lane Kahan over columns c == lane (mod 32) with
 *     products fl(fl(dec*s)*x), then a 32-lane pairwise tree standing in for
 *     Apple's simd_sum (src/metal_kernels.metal:153-177, :7-27); RMSNorm with
 *     per-lane squares (:29-44); two-pass softmax and sequential P.V
 *     (:80-132); SiLU v/(1+exp(-v)) (:46-57), libm exp.
 *   - ORC_MIRROR: the exact order of the gfx950 kernels (per-lane FMA chains over
 *     the lane's 16-column slice of every 1024-column chunk, one 64-lane
 *     pairwise tree, the per-tensor scale applied to the row total; Cody-Waite
 *     exp; split-KV attention combined in a fixed order). GPU results are
 *     compared to it bit for bit.
 *
 * Parity pins (each function header names its own):
 *   fp8 decode   -- tests/fp8_golden.h (all 256 codes) + oracle/_ref build
 *   yarn         -- tests/rope_golden.h + oracle/_ref build (bitwise)
 *   greedy       -- tests/test_generation.c cases + oracle/_ref build
 *   matvec/norm/attention/rope/silu -- double-precision brute force and the
 *     reference's closed forms (all-ones dot == K, long causal sentinel).
 *   layer/model composition -- an independent float64 restatement of
 *     src/metal_encode.m:124-210 (tests/test_oracle_composition.py), with
 *     planted composition mistakes (orc_model.c, ORC_PLANT) that must fail it.
 *   Apple simd_sum order, Metal precise exp/rsqrt/log: parity unpinned (no
 *   runnable Metal implementation exists; the ref-literal tree is our choice).
 */
#ifndef LUNELETTE_ORACLE_H
#define LUNELETTE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORC_HIDDEN 3072
#define ORC_QUERY 4096
#define ORC_KV 1024
#define ORC_INNER 9216
#define ORC_LAYERS 26
#define ORC_VOCAB 131072
#define ORC_HEADS 32
#define ORC_KV_HEADS 8
#define ORC_HEAD_DIM 128

enum { ORC_REF = 0, ORC_MIRROR = 1 };
/* Weight element kinds for matvec. */
enum { ORC_W_FP8 = 0, ORC_W_BF16 = 1, ORC_W_F32 = 2 };

/* ---- scalar pieces ---- */
float orc_fp8_decode(uint8_t code);
float orc_bf16_widen(uint16_t bits);
uint16_t orc_bf16_round(float value);
int orc_yarn(uint32_t position, float cosine[128], float sine[128]);
float orc_query_factor(uint32_t position);
int orc_select_greedy(const float *logits, size_t count, int64_t *token);
float orc_expf(float x);
float orc_silu_ref(float v);
float orc_silu_mirror(float v);

/* ---- kernels ----
 * matvec: y[t*rows + r] = scale * sum_c w(r,c) * x[t*cols + c] with w the
 * decoded FP8 code, widened BF16, or stored FP32. REF applies an FP8 scale per
 * element (fl(dec*scale)) as the reference does; MIRROR scales the row total. */
void orc_matvec(int schedule, int kind, const void *weights, float scale,
    const float *x, float *y, size_t rows, size_t cols, size_t tokens);
void orc_rmsnorm(int schedule, const float *gamma, const float *x, float *out,
    size_t width, size_t tokens);
/* Split-half rotation over heads of 128; qfactor[t] multiplies when non-NULL. */
void orc_rope(const float *x, const float *cosine, const float *sine,
    const float *qfactor, float *out, size_t width, size_t tokens);
void orc_silu_mul(int schedule, const float *gate, const float *up, float *out, size_t n);
/* Causal GQA attention. Query token t attends positions [0, prefix + t].
 * K/V element (p, kv_head, d) lives at base[kv_head*head_stride + p*pos_stride + d].
 * q: [count][4096]; out: [count][4096]. */
void orc_attention(int schedule, const float *q, const float *keys, const float *values,
    size_t head_stride, size_t pos_stride, size_t prefix, size_t count, float *out);

/* ---- model ---- */
typedef struct {
    const uint16_t *input_norm;  /* bf16 [3072] */
    const uint16_t *post_norm;   /* bf16 [3072] */
    const uint8_t *q, *k, *v, *o, *gate, *up, *down; /* FP8 codes, row-major */
    float scale[7];              /* q,k,v,o,gate,up,down */
} orc_layer;

typedef struct {
    const uint16_t *embedding;   /* bf16 [131072][3072] */
    const uint16_t *final_norm;  /* bf16 [3072] */
    orc_layer layers[ORC_LAYERS];
    size_t layer_count;          /* <= 26; fewer layers for quick tests */
    size_t capacity;             /* KV positions */
    float *keys, *values;        /* [layer][8][capacity][128], owned by caller */
} orc_model;

/* One decoder layer over `count` rows of x (in/out, [count][3072]) at positions
 * [length, length+count). KV for `layer` is appended at `length`. */
void orc_layer_forward(int schedule, orc_model *model, size_t layer, float *x,
    size_t length, size_t count);
/* Embedding + all layers + final norm + tied head on the last row.
 * logits: [131072]. Returns 0, or -1 on invalid ids/capacity. */
int orc_model_forward(int schedule, orc_model *model, const int64_t *ids,
    size_t length, size_t count, float *logits);

/* Threads used by OpenMP regions (0 = library default). */
void orc_set_threads(int threads);
int orc_get_threads(void);

#endif
