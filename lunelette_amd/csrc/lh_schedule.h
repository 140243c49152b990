/* Shapes, device layouts and the canonical reduction schedule shared by the
 * host runtime (C) and the gfx950 kernels (HIP).
 *
 * Canonical schedule (the CPU oracle's ORC_MIRROR restates it):
 *   row dot  : columns in chunks of 1024; lane l of a 64-lane wave owns columns
 *              [16l, 16l+16) of every chunk and runs acc = fma(w, x, acc) from
 *              0 over all of them (chunk by chunk, column order); the 64 lane
 *              values reduce by the pairwise halving tree (32,16,8,4,2,1);
 *              the row total is multiplied by the per-tensor scale once. w is
 *              the exact unscaled E4M3FN decode (FP8), the exact BF16 widening
 *              (head) or the stored FP32 decode (resident strategy).
 *   RMSNorm  : ss by the row-dot schedule with w = x; r = 1/sqrt(ss/n + 1e-5);
 *              out = gamma * (x * r).
 *   attention: per (token, head) c_i = chain over d in [32i, 32i+32) of
 *              fma(q_d, k_pd); s_p = fl(((c_0 + c_1) + (c_2 + c_3)) * 2^-3.5);
 *              per 64-position block b: m_b = max s_p, e_p = expf_cw(s_p - m_b),
 *              T_b = 64-lane tree of e, A_b[d] chains fma(e_p, v_pd) over the
 *              block's valid positions; M = max m_b, f_b = expf_cw(m_b - M);
 *              groups of 8 blocks chain fma(f_b, A_b[d]) and fma(f_b, T_b)
 *              from 0; group results add left to right; out = A / T.
 */
#ifndef LH_SCHEDULE_H
#define LH_SCHEDULE_H

#include <stdint.h>

#define LH_HIDDEN 3072
#define LH_QUERY 4096
#define LH_KV 1024
#define LH_INNER 9216
#define LH_LAYERS 26
#define LH_VOCAB 131072
#define LH_HEADS 32
#define LH_KV_HEADS 8
#define LH_HEAD_DIM 128
#define LH_QKV_ROWS (LH_QUERY + 2 * LH_KV) /* fused q|k|v rows: 6144 */

#define LH_CHUNK 1024      /* columns per canonical chunk */
#define LH_LANE_COLS 16    /* columns per lane per chunk */
#define LH_ATTN_BLOCK 64   /* positions per attention block */
#define LH_ARRIVE_STRIDE 32 /* 64-bit words between one-launch attention's arrival words */
#define LH_MAX_BLOCK 256   /* largest executed block (B) */

#define LH_SCORE_SCALE 0.08838834764831845f

/* Per-token step record; the host fills count of them after the header. */
typedef struct {
    int32_t id;
    float qfactor;
    uint32_t position;
    uint32_t pad;
    float cosine[128];
    float sine[128];
} lh_token_params;

typedef struct {
    uint32_t length; /* committed prefix before this call */
    uint32_t count;  /* tokens in this call */
    uint32_t pad[2];
    lh_token_params tokens[LH_MAX_BLOCK];
} lh_step_params;

/* Device KV layout: [layer][kv_head][capacity][128] FP32, K rotated (permuted
 * within 64-position tiles, below), V raw. */
#ifdef __HIPCC__
#define LH_HOST_DEVICE __host__ __device__
#else
#define LH_HOST_DEVICE
#endif
static inline LH_HOST_DEVICE uint64_t lh_kv_index(uint64_t capacity, uint32_t layer, uint32_t kv_head,
    uint64_t position)
{
    return (((uint64_t)layer * LH_KV_HEADS + kv_head) * capacity + position) * LH_HEAD_DIM;
}

/* K is stored in 64-position tiles (the attention block) at the same place
 * as that layout, permuted inside each tile: the 16-byte word holding dims
 * 32q + 4i .. 32q + 4i + 3 of the tile's position p is word
 * ((p / 16) * 8 + i) * 64 + (p % 16) * 4 + q. A wave whose lane 4(p % 16) + q
 * owns position 16w + p % 16, quarter q then reads its eight words as eight
 * contiguous 1 KiB loads. V keeps the row layout. */
static inline LH_HOST_DEVICE uint32_t lh_ktile_word(uint32_t p, uint32_t q, uint32_t i)
{
    return ((p >> 4) * 8 + i) * 64 + (p & 15) * 4 + q;
}

/* Float index of K's dim d at a position. */
static inline LH_HOST_DEVICE uint64_t lh_k_index(uint64_t capacity, uint32_t layer, uint32_t kv_head,
    uint64_t position, uint32_t d)
{
    const uint64_t tile = lh_kv_index(capacity, layer, kv_head, position & ~(uint64_t)63);
    return tile + (uint64_t)lh_ktile_word((uint32_t)(position & 63), d >> 5, (d >> 2) & 7) * 4 +
        (d & 3);
}

#endif
