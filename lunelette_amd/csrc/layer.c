/* One decoder layer on device buffers, shared by the runtime and the
 * kernel-level ABI (operator order of src/metal_encode.m:124-187), plus the
 * per-call step parameters (positions, host YaRN, query factors, ids). */
#include "lunelette_kernels.h"
#include "lh_internal.h"
#include "lh_layer.h"

#include <stdlib.h>
#include <string.h>

static int check(hipError_t status, const char *what)
{
    if (status != hipSuccess) {
        lh_set_error("%s: %s", what, hipGetErrorString(status));
        return -1;
    }
    return 0;
}

/* 64-bit words of one-launch attention: an arrival word per (token, kv
 * head), each on a 256-byte line of its own, then the 8 x 64 flags of a
 * chained decode launch's q|k|v workgroups; at least the XCD dispatch
 * probe's 2048 32-bit words. */
#define FLAGS_WORD(B) ((B) * LH_KV_HEADS * LH_ARRIVE_STRIDE)
#define ARRIVE_WORDS(B) (FLAGS_WORD(B) + LH_KV_HEADS * 64 > 1024 ? \
    FLAGS_WORD(B) + LH_KV_HEADS * 64 : 1024)

static int alloc_device(void **out, size_t bytes, uint64_t *total)
{
    *out = NULL;
    if (check(lh_dev_malloc(out, bytes), "workspace allocation")) {
        return -1;
    }
    *total += bytes;
    return 0;
}

lh_workspace *lh_workspace_create(size_t capacity, size_t block)
{
    if (!capacity || !block || block > LH_MAX_BLOCK || capacity % LH_ATTN_BLOCK ||
        capacity > 262144 || block > capacity) {
        lh_set_error("workspace: capacity must be a multiple of 64 up to 262144 and block 1..256");
        return NULL;
    }
    lh_workspace *ws = calloc(1, sizeof *ws);
    if (!ws) {
        lh_set_error("workspace: host allocation failed");
        return NULL;
    }
    ws->capacity = capacity;
    ws->block = block;
    const size_t nbc = capacity / LH_ATTN_BLOCK;
    const size_t B = block;
    if (check(lh_host_malloc((void **)&ws->h_params, sizeof(lh_step_params), hipHostMallocDefault),
            "workspace pinned parameters") ||
        alloc_device((void **)&ws->d_params, sizeof(lh_step_params), &ws->bytes) ||
        alloc_device((void **)&ws->d_q, B * LH_QUERY * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_attn, B * LH_QUERY * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_gated, B * LH_INNER * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_up, B * LH_INNER * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_xn, B * LH_HIDDEN * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_qraw, B * LH_QUERY * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_kraw, B * LH_KV * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_vraw, B * LH_KV * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_PM, B * LH_HEADS * nbc * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_PT, B * LH_HEADS * nbc * sizeof(float), &ws->bytes) ||
        alloc_device((void **)&ws->d_PA, B * LH_HEADS * nbc * LH_HEAD_DIM * sizeof(float),
            &ws->bytes) ||
        alloc_device((void **)&ws->d_arrive, ARRIVE_WORDS(B) * 8, &ws->bytes) ||
        check(hipMemset(ws->d_arrive, 0, ARRIVE_WORDS(B) * 8), "workspace clear") ||
        alloc_device((void **)&ws->d_bflags, LH_KV_HEADS * nbc * 8, &ws->bytes) ||
        check(hipMemset(ws->d_bflags, 0, LH_KV_HEADS * nbc * 8), "workspace clear")) {
        lh_workspace_destroy(ws);
        return NULL;
    }
    int fused = 0;
    if (lh_attention_xcd_probe((uint32_t *)ws->d_arrive, 2 * ARRIVE_WORDS(B), &fused, NULL)) {
        lh_set_error("workspace: XCD dispatch probe failed: %s", hipGetErrorString(hipGetLastError()));
        lh_workspace_destroy(ws);
        return NULL;
    }
    memset(ws->h_params, 0, sizeof(lh_step_params));
    return ws;
}

int lh_workspace_clear_arrivals(lh_workspace *ws)
{
    if (!ws || !ws->d_arrive || !ws->d_bflags) {
        return -1;
    }
    ws->epoch = 0;
    return check(hipMemset(ws->d_arrive, 0, ARRIVE_WORDS(ws->block) * 8), "arrival words clear") ||
        check(hipMemset(ws->d_bflags, 0, LH_KV_HEADS * (ws->capacity / LH_ATTN_BLOCK) * 8),
            "block flags clear");
}

void lh_workspace_destroy(lh_workspace *ws)
{
    if (!ws) {
        return;
    }
    void *device[] = {ws->d_params, ws->d_q, ws->d_attn, ws->d_gated, ws->d_up, ws->d_xn,
        ws->d_qraw, ws->d_kraw, ws->d_vraw, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_arrive,
        ws->d_bflags,
        ws->d_split, ws->d_gemm, ws->d_yarn};
    for (size_t i = 0; i < sizeof device / sizeof device[0]; i++) {
        lh_dev_free(device[i]);
    }
    lh_host_free(ws->h_params);
    free(ws->h_yarn);
    free(ws->h_yarn_ready);
    free(ws);
}

/* Row p of the workspace's host YaRN table (cos[64], sin[64]), computed by
 * lh_yarn on first use: a 256-token chunk otherwise spends about 0.35 ms of
 * host time in powf/sinf/cosf before its first launch. NULL when the table
 * cannot be allocated. */
static const float *yarn_row(lh_workspace *ws, size_t p)
{
    if (!ws->h_yarn) {
        ws->h_yarn = malloc(ws->capacity * 128 * sizeof(float));
        ws->h_yarn_ready = calloc(ws->capacity, 1);
        if (!ws->h_yarn || !ws->h_yarn_ready) {
            free(ws->h_yarn);
            free(ws->h_yarn_ready);
            ws->h_yarn = NULL;
            ws->h_yarn_ready = NULL;
            lh_set_error("workspace: host allocation failed");
            return NULL;
        }
    }
    float *row = ws->h_yarn + p * 128;
    if (!ws->h_yarn_ready[p]) {
        float cosine[128], sine[128];
        lh_yarn((uint32_t)p, cosine, sine);
        memcpy(row, cosine, 64 * sizeof(float));
        memcpy(row + 64, sine, 64 * sizeof(float));
        ws->h_yarn_ready[p] = 1;
    }
    return row;
}

int lh_workspace_set_tokens(lh_workspace *ws, const int64_t *ids, size_t length, size_t count,
    void *stream)
{
    if (!ws || !ids || !count || count > ws->block || length > ws->capacity ||
        count > ws->capacity - length) {
        lh_set_error("set_tokens: require 1..block ids within capacity");
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    /* The pinned record may still feed the previous upload. */
    if (check(hipStreamSynchronize(s), "set_tokens synchronize")) {
        return -1;
    }
    lh_step_params *p = ws->h_params;
    p->length = (uint32_t)length;
    p->count = (uint32_t)count;
    for (size_t t = 0; t < count; t++) {
        if (ids[t] < 0 || ids[t] >= LH_VOCAB) {
            lh_set_error("set_tokens: invalid token id at %zu", t);
            return -1;
        }
        const uint32_t position = (uint32_t)(length + t);
        lh_token_params *tp = &p->tokens[t];
        tp->id = (int32_t)ids[t];
        tp->position = position;
        tp->qfactor = lh_query_factor(position);
        /* lh_yarn's rows repeat their 64 values in both halves. */
        const float *row = yarn_row(ws, position);
        if (!row) {
            return -1;
        }
        memcpy(tp->cosine, row, 64 * sizeof(float));
        memcpy(tp->cosine + 64, row, 64 * sizeof(float));
        memcpy(tp->sine, row + 64, 64 * sizeof(float));
        memcpy(tp->sine + 64, row + 64, 64 * sizeof(float));
    }
    const size_t bytes = offsetof(lh_step_params, tokens) + count * sizeof(lh_token_params);
    if (check(hipMemcpyAsync(ws->d_params, p, bytes, hipMemcpyHostToDevice, s),
            "set_tokens upload")) {
        return -1;
    }
    ws->length = length;
    ws->count = count;
    return 0;
}

int lh_workspace_prepare_decode(lh_workspace *ws)
{
    if (!ws) {
        lh_set_error("prepare_decode: require a workspace");
        return -1;
    }
    if (ws->d_yarn) {
        return 0;
    }
    for (size_t p = 0; p < ws->capacity; p++) {
        if (!yarn_row(ws, p)) {
            return -1;
        }
    }
    const size_t bytes = ws->capacity * 128 * sizeof(float);
    return alloc_device((void **)&ws->d_yarn, bytes, &ws->bytes) ||
        check(hipMemcpy(ws->d_yarn, ws->h_yarn, bytes, hipMemcpyHostToDevice),
            "prepare_decode upload") ? -1 : 0;
}

int lh_workspace_set_decode(lh_workspace *ws, const uint16_t *d_embedding, int64_t id,
    size_t length, float *d_x, hipStream_t s)
{
    if (!ws || !ws->d_yarn || !d_embedding || !d_x || id < 0 || id >= LH_VOCAB ||
        length >= ws->capacity) {
        lh_set_error("set_decode: require a prepared workspace, a valid id and length < capacity");
        return -1;
    }
    ws->length = length;
    ws->count = 1;
    if (lh_launch_step_embed(d_embedding, ws->d_yarn, (int32_t)id, (uint32_t)length,
            lh_query_factor((uint32_t)length), ws->d_params, d_x, s)) {
        lh_set_error("step embed launch failed: %s", hipGetErrorString(hipGetLastError()));
        return -1;
    }
    return 0;
}

static int launched(int status, const char *what)
{
    if (status) {
        hipError_t e = hipGetLastError();
        lh_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

/* Separate-operator path (also the resident FP32 strategy): every operator is
 * its own kernel, every row dot follows the same canonical schedule as the
 * fused kernels, so results are bitwise identical. */
static int layer_unfused(const lh_layer_weights *w, float *x, float *keys, float *values,
    lh_workspace *ws, int resident, hipStream_t s)
{
    const uint32_t n = (uint32_t)ws->count, C = (uint32_t)ws->capacity;
    const int kind = resident ? 2 : 0;
    const void *wq = resident ? (const void *)w->f32_qkv : (const void *)w->qkv;
    const size_t esize = resident ? 4 : 1;
    const char *base = (const char *)wq;
    const void *wk = base + (size_t)LH_QUERY * LH_HIDDEN * esize;
    const void *wv = base + (size_t)(LH_QUERY + LH_KV) * LH_HIDDEN * esize;
    const void *wo = resident ? (const void *)w->f32_o : (const void *)w->o;
    const void *wg = resident ? (const void *)w->f32_gate : (const void *)w->gate;
    const void *wu = resident ? (const void *)w->f32_up : (const void *)w->up;
    const void *wd = resident ? (const void *)w->f32_down : (const void *)w->down;
    const lh_step_params *params = ws->d_params;
    if (launched(lh_launch_rmsnorm(w->input_norm, x, ws->d_xn, LH_HIDDEN, n, s), "input norm") ||
        launched(lh_launch_matvec(kind, 0, wq, w->scale[0], ws->d_xn, ws->d_qraw, NULL,
            LH_QUERY, LH_HIDDEN, n, s), "q") ||
        launched(lh_launch_matvec(kind, 0, wk, w->scale[1], ws->d_xn, ws->d_kraw, NULL,
            LH_KV, LH_HIDDEN, n, s), "k") ||
        launched(lh_launch_matvec(kind, 0, wv, w->scale[2], ws->d_xn, ws->d_vraw, NULL,
            LH_KV, LH_HIDDEN, n, s), "v") ||
        launched(lh_launch_rope_append(ws->d_qraw, ws->d_kraw, ws->d_vraw, params, n, ws->d_q,
            keys, values, C, s), "rope/append") ||
        launched(lh_launch_attention(ws->d_q, keys, values, ws->d_params, (uint32_t)ws->length, n,
            C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_arrive, ws->d_bflags, ++ws->epoch,
            ws->handoff_fault, ws->d_attn, s), "attention") ||
        launched(lh_launch_matvec(kind, 0, wo, w->scale[3], ws->d_attn, x, x, LH_HIDDEN,
            LH_QUERY, n, s), "o") ||
        launched(lh_launch_rmsnorm(w->post_norm, x, ws->d_xn, LH_HIDDEN, n, s), "post norm") ||
        launched(lh_launch_matvec(kind, 0, wg, w->scale[4], ws->d_xn, ws->d_gated, NULL,
            LH_INNER, LH_HIDDEN, n, s), "gate") ||
        launched(lh_launch_matvec(kind, 0, wu, w->scale[5], ws->d_xn, ws->d_up, NULL,
            LH_INNER, LH_HIDDEN, n, s), "up") ||
        launched(lh_launch_silu_mul(ws->d_gated, ws->d_up, ws->d_gated, (size_t)n * LH_INNER, s),
            "silu") ||
        launched(lh_launch_matvec(kind, 0, wd, w->scale[6], ws->d_gated, x, x, LH_HIDDEN,
            LH_INNER, n, s), "down")) {
        return -1;
    }
    return 0;
}

static int layer_fused(const lh_layer_weights *w, float *x, float *keys, float *values,
    lh_workspace *ws, int lookup, hipStream_t s)
{
    const uint32_t n = (uint32_t)ws->count, C = (uint32_t)ws->capacity;
    const lh_step_params *params = ws->d_params;
    /* One decode token: q|k|v and the attention blocks share a launch. */
    const int chained = n == 1 && lh_attention_chained((uint32_t)ws->length);
    if ((chained ?
            launched(lh_launch_qkv_attention(lookup, w->qkv, w->scale[0], w->scale[1],
                w->scale[2], w->input_norm, x, params, (uint32_t)ws->length, ws->d_q, keys,
                values, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_arrive,
                ws->d_arrive + FLAGS_WORD(ws->block), ws->d_bflags, ++ws->epoch,
                ws->handoff_fault, ws->d_attn, s),
                "qkv/attention") :
            launched(lh_launch_qkv_rope(lookup, w->qkv, w->scale[0], w->scale[1], w->scale[2],
                w->input_norm, x, params, n, ws->d_q, keys, values, C, s), "qkv") ||
            launched(lh_launch_attention(ws->d_q, keys, values, ws->d_params,
                (uint32_t)ws->length, n, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_arrive,
                ws->d_bflags, ++ws->epoch, ws->handoff_fault, ws->d_attn, s), "attention")) ||
        launched(lh_launch_matvec(0, lookup, w->o, w->scale[3], ws->d_attn, x, x, LH_HIDDEN,
            LH_QUERY, n, s), "o") ||
        launched(lh_launch_gateup_silu(lookup, w->gate, w->up, w->scale[4], w->scale[5],
            w->post_norm, x, n, ws->d_gated, s), "gate/up") ||
        launched(lh_launch_matvec(0, lookup, w->down, w->scale[6], ws->d_gated, x, x, LH_HIDDEN,
            LH_INNER, n, s), "down")) {
        return -1;
    }
    return 0;
}

int lh_layer_operator(int op, const lh_layer_weights *w, float *d_x, float *d_keys,
    float *d_values, lh_workspace *ws, void *stream)
{
    if (!w || !d_x || !d_keys || !d_values || !ws || !ws->count) {
        lh_set_error("layer_operator: missing argument or tokens not set");
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    const uint32_t n = (uint32_t)ws->count, C = (uint32_t)ws->capacity;
    switch (op) {
    case LH_OP_QKV_ROPE:
        return launched(lh_launch_qkv_rope(0, w->qkv, w->scale[0], w->scale[1], w->scale[2],
            w->input_norm, d_x, ws->d_params, n, ws->d_q, d_keys, d_values, C, s), "qkv");
    case LH_OP_ATTENTION:
        return launched(lh_launch_attention(ws->d_q, d_keys, d_values, ws->d_params,
            (uint32_t)ws->length, n, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_arrive, ws->d_bflags,
            ++ws->epoch, ws->handoff_fault, ws->d_attn, s), "attention");
    case LH_OP_O_RESIDUAL:
        return launched(lh_launch_matvec(0, 0, w->o, w->scale[3], ws->d_attn, d_x, d_x, LH_HIDDEN,
            LH_QUERY, n, s), "o");
    case LH_OP_GATEUP_SILU:
        return launched(lh_launch_gateup_silu(0, w->gate, w->up, w->scale[4], w->scale[5],
            w->post_norm, d_x, n, ws->d_gated, s), "gate/up");
    case LH_OP_DOWN_RESIDUAL:
        return launched(lh_launch_matvec(0, 0, w->down, w->scale[6], ws->d_gated, d_x, d_x,
            LH_HIDDEN, LH_INNER, n, s), "down");
    default:
        lh_set_error("layer_operator: unknown operator %d", op);
        return -1;
    }
}

int lh_layer_forward(const lh_layer_weights *w, float *d_x, float *d_keys, float *d_values,
    lh_workspace *ws, int path, void *stream)
{
    if (!w || !d_x || !d_keys || !d_values || !ws || !ws->count) {
        lh_set_error("layer_forward: missing argument or tokens not set");
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    switch (path) {
    case LH_PATH_FUSED:
        return layer_fused(w, d_x, d_keys, d_values, ws, 0, s);
    case LH_PATH_LOOKUP:
        return layer_fused(w, d_x, d_keys, d_values, ws, 1, s);
    case LH_PATH_UNFUSED:
        return layer_unfused(w, d_x, d_keys, d_values, ws, 0, s);
    case LH_PATH_RESIDENT:
        if (!w->f32_qkv || !w->f32_o || !w->f32_gate || !w->f32_up || !w->f32_down) {
            lh_set_error("layer_forward: resident path needs FP32 weights");
            return -1;
        }
        return layer_unfused(w, d_x, d_keys, d_values, ws, 1, s);
    case LH_PATH_MFMA:
        return lh_layer_forward_mfma(w, d_x, d_keys, d_values, ws, 0, NULL, s);
    default:
        lh_set_error("layer_forward: unknown path %d", path);
        return -1;
    }
}

int lh_attention(const float *d_q, const float *d_keys, const float *d_values, lh_workspace *ws,
    float *d_out, void *stream)
{
    if (!d_q || !d_keys || !d_values || !ws || !ws->count || !d_out) {
        lh_set_error("attention: missing argument or tokens not set");
        return -1;
    }
    return launched(lh_launch_attention(d_q, d_keys, d_values, ws->d_params,
        (uint32_t)ws->length, (uint32_t)ws->count, (uint32_t)ws->capacity, ws->d_PM, ws->d_PT,
        ws->d_PA, ws->d_arrive, ws->d_bflags, ++ws->epoch, ws->handoff_fault, d_out,
        (hipStream_t)stream), "attention");
}

int lh_attention_mfma(const float *d_q, const float *d_keys, const float *d_values,
    lh_workspace *ws, float *d_out, void *stream)
{
    if (!d_q || !d_keys || !d_values || !ws || !ws->count || !d_out) {
        lh_set_error("attention_mfma: missing argument or tokens not set");
        return -1;
    }
    return launched(lh_launch_attention_mfma(d_q, d_keys, d_values, ws->d_params,
        (uint32_t)ws->length, (uint32_t)ws->count, (uint32_t)ws->capacity, ws->d_PM, ws->d_PT,
        ws->d_PA, d_out, NULL, 0, NULL, (hipStream_t)stream), "attention");
}

int lh_head_forward(const uint16_t *d_embedding, const float *d_gamma, const float *d_xrow,
    float *d_logits, void *stream)
{
    if (!d_embedding || !d_gamma || !d_xrow || !d_logits) {
        lh_set_error("head_forward: missing argument");
        return -1;
    }
    return launched(lh_launch_head(d_embedding, d_gamma, d_xrow, d_logits, NULL,
        (hipStream_t)stream), "head");
}

int lh_head_forward_checked(const uint16_t *d_embedding, const float *d_gamma,
    const float *d_xrow, float *d_logits, uint32_t *d_nonfinite, void *stream)
{
    if (!d_embedding || !d_gamma || !d_xrow || !d_logits || !d_nonfinite) {
        lh_set_error("head_forward_checked: missing argument");
        return -1;
    }
    return launched(lh_launch_head(d_embedding, d_gamma, d_xrow, d_logits, d_nonfinite,
        (hipStream_t)stream), "head");
}

int lh_embed_forward(const uint16_t *d_embedding, float *d_x, lh_workspace *ws, void *stream)
{
    if (!d_embedding || !d_x || !ws || !ws->count) {
        lh_set_error("embed_forward: missing argument or tokens not set");
        return -1;
    }
    return launched(lh_launch_embed(d_embedding, ws->d_params, (uint32_t)ws->count, d_x,
        (hipStream_t)stream), "embed");
}
