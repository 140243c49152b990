/* Kernel-level C-ABI of the gfx950 forward path, below the runtime.
 *
 * This is the analogue of the reference's private projection/operator seam
 * (src/metal_internal.h:57-74: lunelette_metal_project and
 * lunelette_metal_encode_operator), exported so tests and benchmarks can drive
 * single kernels and single decoder layers on device buffers. All pointers
 * named d_* are device pointers; `stream` is a hipStream_t passed as void*
 * (NULL = the null stream). Functions return 0 on success and -1 on invalid
 * arguments or a launch failure (lh_last_error() describes it).
 */
#ifndef LUNELETTE_KERNELS_H
#define LUNELETTE_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- device plumbing (no torch needed by callers) ---- */
const char *lh_last_error(void);
int lh_device_count(void);
void *lh_device_alloc(size_t bytes);
void lh_device_free(void *d_ptr);
void *lh_host_alloc_pinned(size_t bytes);
void lh_host_free_pinned(void *ptr);
int lh_memcpy_htod(void *d_dst, const void *src, size_t bytes);
int lh_memcpy_dtoh(void *dst, const void *d_src, size_t bytes);
int lh_memcpy_dtod(void *d_dst, const void *d_src, size_t bytes);
int lh_memset_device(void *d_dst, int value, size_t bytes);
int lh_device_synchronize(void);
void *lh_stream_create(void);
int lh_stream_synchronize(void *stream);
void lh_stream_destroy(void *stream);
void *lh_event_create(void);
int lh_event_record(void *event, void *stream);
int lh_event_elapsed_ms(void *start, void *stop, float *milliseconds);
void lh_event_destroy(void *event);

/* ---- single kernels ---- */

/* FP8 E4M3FN projection y[t][r] = sum_c fl(dec(W[r][c])*scale) * x[t][c]
 * (src/metal_kernels.metal:136-177 project_fp8, :179-272 project_fp8_lookup
 * when lookup != 0; dispatch at src/metal_encode.m:72-92). W row-major
 * [rows][cols] codes; x [tokens][cols]; y [tokens][rows]. */
int lh_fp8_matvec(const uint8_t *d_w, float scale, const float *d_x, float *d_y,
    size_t rows, size_t cols, size_t tokens, int lookup, void *stream);
/* FP32 projection (src/metal_kernels.metal:7-27 project). */
int lh_f32_matvec(const float *d_w, const float *d_x, float *d_y, size_t rows, size_t cols,
    size_t tokens, void *stream);
/* BF16-weight projection, weights widened exactly (tied head). */
int lh_bf16_matvec(const uint16_t *d_w, const float *d_x, float *d_y, size_t rows,
    size_t cols, size_t tokens, void *stream);
/* RMSNorm out = gamma*(x*rsqrt(mean(x^2)+1e-5)) (src/metal_kernels.metal:29-44),
 * width <= 16384. */
int lh_rmsnorm(const float *d_gamma, const float *d_x, float *d_out, size_t width,
    size_t tokens, void *stream);
/* element modes (src/metal_kernels.metal:46-57): 0 add, 1 SiLU, 2 multiply. */
int lh_element(int mode, const float *d_first, const float *d_second, float *d_out, size_t n,
    void *stream);
/* Split-half RoPE over 128-wide heads with per-token cos/sin [tokens][128];
 * d_qfactor [tokens] or NULL (src/metal_kernels.metal:59-78). */
int lh_rope(const float *d_x, const float *d_cos, const float *d_sin, const float *d_qfactor,
    float *d_out, size_t width, size_t tokens, void *stream);
/* E4M3FN decode of n codes (hardware conversion used by the kernels). */
int lh_fp8_decode(const uint8_t *d_codes, float *d_out, size_t n, void *stream);
/* Streaming-read measurement (no counterpart in the reference): reads `bytes`
 * from d_src with 16-byte non-temporal loads in `grid` workgroups of four
 * waves, `unroll` loads (1, 2, 4 or 8) in flight per lane, folded so that no
 * load is dead; d_sink (grid*4 words) is written only for an improbable fold
 * value. bytes must be a multiple of grid*4*64*16*unroll. bench.py times it
 * over the decode weight shapes as each kernel's pure-read floor. */
int lh_read_floor(const void *d_src, size_t bytes, unsigned grid, unsigned unroll,
    unsigned *d_sink, void *stream);
/* Device exp and SiLU used by the kernels (bitwise checks against the oracle). */
int lh_expf(const float *d_x, float *d_out, size_t n, void *stream);

/* ---- decoder layer ---- */

/* Workspace for one capacity/block profile: step parameters (positions,
 * host YaRN cos/sin, query factors, ids) and scratch. */
typedef struct lh_workspace lh_workspace;
lh_workspace *lh_workspace_create(size_t capacity, size_t block);
void lh_workspace_destroy(lh_workspace *ws);
/* Host-computes YaRN (src/metal_yarn.c) and query factors for positions
 * [length, length+count) and uploads them with the ids on `stream`. */
int lh_workspace_set_tokens(lh_workspace *ws, const int64_t *ids, size_t length, size_t count,
    void *stream);

/* One layer's device weights: FP8 q|k|v fused row-major [6144][3072], o
 * [3072][4096], gate/up [9216][3072], down [3072][9216]; per-tensor scales
 * q,k,v,o,gate,up,down; FP32 norms [3072]. For the resident strategy the
 * f32_* pointers hold fl(dec*scale) with the same shapes. */
typedef struct {
    const uint8_t *qkv, *o, *gate, *up, *down;
    const float *f32_qkv, *f32_o, *f32_gate, *f32_up, *f32_down;
    float scale[7];
    const float *input_norm, *post_norm;
} lh_layer_weights;

enum {
    LH_PATH_FUSED = 0,    /* compact FP8, fused decode-schedule kernels */
    LH_PATH_LOOKUP = 1,   /* same, table decode */
    LH_PATH_UNFUSED = 2,  /* compact FP8, one operator per kernel */
    LH_PATH_RESIDENT = 3, /* FP32 weights, one operator per kernel */
    LH_PATH_MFMA = 4      /* multi-token: MFMA GEMM projections */
};

/* KV cache of one layer (capacity a multiple of 64): d_values is
 * [8][capacity][128] FP32 rows; d_keys holds the same [8][capacity][128]
 * values with each 64-position tile's 16-byte words permuted: dims
 * 32q + 4i .. 32q + 4i + 3 of the tile's position p (0..63) sit at word
 * ((p / 16) * 8 + i) * 64 + (p % 16) * 4 + q of the tile. */

/* One decoder layer (src/metal_encode.m:124-187) over d_x [count][3072] in
 * place, at positions [length, length+count) set by lh_workspace_set_tokens;
 * K/V rows are appended into d_keys/d_values (layout above). */
int lh_layer_forward(const lh_layer_weights *w, float *d_x, float *d_keys, float *d_values,
    lh_workspace *ws, int path, void *stream);
/* One operator of the decode-schedule layer (the analogue of
 * lunelette_metal_encode_operator, src/metal_encode.m:5-50), for timing and
 * tests. Same arguments as lh_layer_forward; compact FP8 weights. */
enum {
    LH_OP_QKV_ROPE = 0,      /* norm + q|k|v + RoPE + KV append */
    LH_OP_ATTENTION = 1,     /* scores, softmax, P.V, combine */
    LH_OP_O_RESIDUAL = 2,    /* o projection + residual add */
    LH_OP_GATEUP_SILU = 3,   /* norm + gate/up + SiLU(gate)*up */
    LH_OP_DOWN_RESIDUAL = 4  /* down projection + residual add */
};
int lh_layer_operator(int op, const lh_layer_weights *w, float *d_x, float *d_keys,
    float *d_values, lh_workspace *ws, void *stream);
/* Causal GQA attention (src/metal_kernels.metal:80-132 scores + attend) of
 * the workspace's count query rows d_q [count][4096] over positions
 * [0, length+t] of d_keys/d_values (layout above) into d_out. */
int lh_attention(const float *d_q, const float *d_keys, const float *d_values, lh_workspace *ws,
    float *d_out, void *stream);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): lh_attention without a workspace. Query rows d_q
 * [count][4096] attend positions [0, length + t] of d_keys/d_values
 * (layout above); bitwise the result of lh_attention for the same
 * length and count. The split-KV partials and the step header live in one
 * static device array per GPU, held until the process ends: count * capacity
 * must not exceed 65536 (17.0 MB of scratch), larger calls are refused. Calls that
 * overlap on one GPU race on that array; callers serialize them. */
int lh_attention_noalloc(const float *d_q, const float *d_keys, const float *d_values,
    size_t length, size_t count, size_t capacity, float *d_out, void *stream);
/* The same attention on the matrix cores (the PREFILL_MPS path's operator;
 * replaces the scores + attend dispatches of src/metal_encode.m:154-159 when
 * prefill runs on MPS): FP32 MFMA with an online softmax, tolerance-equal to
 * lh_attention. */
int lh_attention_mfma(const float *d_q, const float *d_keys, const float *d_values,
    lh_workspace *ws, float *d_out, void *stream);
/* MFMA block projection (PREFILL_MPS; replaces convert_fp8 + MPS GEMM,
 * src/metal_encode.m:94-110): y[t][r] = scale * sum_c dec(W[r][c]) x[t][c],
 * FP8 decoded exactly to BF16 tiles, x split exactly into three BF16 parts,
 * FP32 accumulation. rows % 512 == 0 (<= 3072), cols % 256 == 0 (<= 9216),
 * tokens <= the workspace block. Uses the workspace's scratch. */
int lh_fp8_gemm(lh_workspace *ws, const uint8_t *d_w, float scale, const float *d_x, float *d_y,
    size_t rows, size_t cols, size_t tokens, void *stream);
/* Final RMSNorm + tied BF16 head on one row (src/metal_encode.m:204-210). */
int lh_head_forward(const uint16_t *d_embedding, const float *d_gamma, const float *d_xrow,
    float *d_logits, void *stream);
/* Additive: the runtime's head step. The same logits, and *d_nonfinite = 1
 * when any of them is Inf or NaN (the caller clears it first), which stands in
 * for the host finite scan of src/metal_runtime.m:418-424 on finite steps. */
int lh_head_forward_checked(const uint16_t *d_embedding, const float *d_gamma,
    const float *d_xrow, float *d_logits, uint32_t *d_nonfinite, void *stream);
/* Embedding gather of the workspace's ids into d_x [count][3072]. */
int lh_embed_forward(const uint16_t *d_embedding, float *d_x, lh_workspace *ws, void *stream);

/* ---- host helpers ---- */

/* Host YaRN cos/sin (src/metal_yarn.c:8-33); -1 for position >= 262144. */
int lh_yarn(uint32_t position, float cosine[128], float sine[128]);
/* 1 + 0.1*ln(1 + floor(position/16384)) (src/metal_kernels.metal:72-76). */
float lh_query_factor(uint32_t position);

/* Seeded synthetic tensors: element i of tensor `tensor` depends only on
 * (seed, tensor, offset+i), so any slice is reproducible. */
void lh_synth_fp8(uint64_t seed, uint32_t tensor, uint64_t offset, uint8_t *out, size_t n);
void lh_synth_normal_f32(uint64_t seed, uint32_t tensor, uint64_t offset, float mean, float std,
    float *out, size_t n);
void lh_synth_normal_bf16(uint64_t seed, uint32_t tensor, uint64_t offset, float mean, float std,
    uint16_t *out, size_t n);
/* BF16-exact scale in [0.01, 0.02]. */
float lh_synth_scale(uint64_t seed, uint32_t tensor);
/* Uniform token ids in [0, 131072). */
void lh_synth_tokens(uint64_t seed, uint32_t stream_id, int64_t *out, size_t n);

/* ---- checkpoint files (safetensors) ----
 * The container reader replaces st_open/st_find/st_read
 * (include/safetensors.h:47-53, src/safetensors.c:352-424); the tensor
 * contract replaces lunelette_metal_weights_open (src/metal_weights.c:40-150).
 * lunelette_metal_create*(path) loads through them. */
/* Opens and validates path; on success writes one line per tensor in header
 * order, "name|dtype|rank|d0,d1,..|begin|end\n", into listing. */
int lh_st_inspect(const char *path, char *listing, size_t listing_capacity, char *error,
    size_t capacity);
/* Bytes [offset, offset + bytes) of tensor `name`, bounds-checked. */
int lh_st_read_tensor(const char *path, const char *name, uint64_t offset, void *out,
    size_t bytes, char *error, size_t capacity);
/* FP8 admission of n codes under a per-tensor scale for a strategy
 * (lunelette_metal_strategy), the check the runtime's upload applies to every
 * FP8 tensor: the compact strategies follow lunelette_metal_weights_load_raw
 * (src/metal_weights.c:174-231: positive, normal, BF16-exact scale; finite
 * codes; normal nonzero products), RESIDENT_FP32 follows st_load_fp8
 * (src/safetensors.c:521-548: positive finite scale; finite products).
 * 0 admitted; -1 refused, with the first refused byte in the diagnostic. */
int lh_fp8_admit(const uint8_t *codes, size_t n, float scale, int strategy, char *error,
    size_t capacity);
/* Container + tensor contract + scales of a model checkpoint; scales
 * [2 + 26*9] (slot order of src/metal_weights.h, 1 for non-FP8 slots) or NULL. */
int lh_checkpoint_check(const char *path, float *scales, char *error, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif
