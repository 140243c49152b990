/* Oracle decoder layer and full-model forward, following the operator order of
 * src/metal_encode.m:124-215 (norm, q/k/v, RoPE with the query factor on Q only,
 * K rotated before caching and V raw, scores/attend, o, residual, norm,
 * gate/up, SiLU*up, down, residual; final norm and tied head on the last row).
 * TEST INFRASTRUCTURE ONLY (see oracle.h). */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>

/* Planted composition mistakes for the tests that show the independent float64
 * restatement of the layer catches them (tests/test_oracle_composition.py
 * builds this file with -DORC_PLANT=n; the shipped oracle has ORC_PLANT 0):
 * 1 attention residual skipped, 2 post-norm fed x instead of x+o,
 * 3 query factor on K instead of Q, 4 V rotated before caching,
 * 5 head on row 0 instead of the last row, 6 K cached unrotated,
 * 7 MLP residual added to the layer input instead of x+o,
 * 8 query factor dropped (neither Q nor K scaled). */
#ifndef ORC_PLANT
#define ORC_PLANT 0
#endif

static void widen(const uint16_t *src, float *dst, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        dst[i] = orc_bf16_widen(src[i]);
    }
}

void orc_layer_forward(int schedule, orc_model *model, size_t layer, float *x,
    size_t length, size_t count)
{
    const orc_layer *w = &model->layers[layer];
    const size_t H = ORC_HIDDEN, Q = ORC_QUERY, KV = ORC_KV, I = ORC_INNER;
    float gamma_in[ORC_HIDDEN], gamma_post[ORC_HIDDEN];
    widen(w->input_norm, gamma_in, H);
    widen(w->post_norm, gamma_post, H);
    float *xn = malloc(count * H * sizeof(float));
    float *q = malloc(count * Q * sizeof(float));
    float *k = malloc(count * KV * sizeof(float));
    float *v = malloc(count * KV * sizeof(float));
    float *rq = malloc(count * Q * sizeof(float));
    float *rk = malloc(count * KV * sizeof(float));
    float *attn = malloc(count * Q * sizeof(float));
    float *o = malloc(count * H * sizeof(float));
    float *gate = malloc(count * I * sizeof(float));
    float *up = malloc(count * I * sizeof(float));
    float *cosine = malloc(count * 128 * sizeof(float));
    float *sine = malloc(count * 128 * sizeof(float));
    float *factor = malloc(count * sizeof(float));
    for (size_t t = 0; t < count; t++) {
        uint32_t position = (uint32_t)(length + t);
        orc_yarn(position, cosine + t * 128, sine + t * 128);
        factor[t] = orc_query_factor(position);
    }
    orc_rmsnorm(schedule, gamma_in, x, xn, H, count);
    orc_matvec(schedule, ORC_W_FP8, w->q, w->scale[0], xn, q, Q, H, count);
    orc_matvec(schedule, ORC_W_FP8, w->k, w->scale[1], xn, k, KV, H, count);
    orc_matvec(schedule, ORC_W_FP8, w->v, w->scale[2], xn, v, KV, H, count);
    orc_rope(q, cosine, sine, ORC_PLANT == 3 || ORC_PLANT == 8 ? NULL : factor, rq, Q, count);
    orc_rope(k, cosine, sine, ORC_PLANT == 3 ? factor : NULL, rk, KV, count);
    if (ORC_PLANT == 4) {
        memcpy(attn, v, count * KV * sizeof(float));
        orc_rope(attn, cosine, sine, NULL, v, KV, count);
    }
    if (ORC_PLANT == 6) {
        memcpy(rk, k, count * KV * sizeof(float));
    }
    size_t cap = model->capacity;
    float *keys = model->keys + layer * ORC_KV_HEADS * cap * 128;
    float *values = model->values + layer * ORC_KV_HEADS * cap * 128;
    for (size_t t = 0; t < count; t++) {
        for (size_t h = 0; h < ORC_KV_HEADS; h++) {
            memcpy(keys + h * cap * 128 + (length + t) * 128, rk + t * KV + h * 128,
                128 * sizeof(float));
            memcpy(values + h * cap * 128 + (length + t) * 128, v + t * KV + h * 128,
                128 * sizeof(float));
        }
    }
    orc_attention(schedule, rq, keys, values, cap * 128, 128, length, count, attn);
    orc_matvec(schedule, ORC_W_FP8, w->o, w->scale[3], attn, o, H, Q, count);
    float *before = ORC_PLANT == 2 || ORC_PLANT == 7 ? malloc(count * H * sizeof(float)) : NULL;
    if (before) {
        memcpy(before, x, count * H * sizeof(float));
    }
    for (size_t i = 0; i < count * H; i++) {
        x[i] = ORC_PLANT == 1 ? x[i] : x[i] + o[i];
    }
    orc_rmsnorm(schedule, gamma_post, ORC_PLANT == 2 ? before : x, xn, H, count);
    orc_matvec(schedule, ORC_W_FP8, w->gate, w->scale[4], xn, gate, I, H, count);
    orc_matvec(schedule, ORC_W_FP8, w->up, w->scale[5], xn, up, I, H, count);
    orc_silu_mul(schedule, gate, up, gate, count * I);
    orc_matvec(schedule, ORC_W_FP8, w->down, w->scale[6], gate, o, H, I, count);
    for (size_t i = 0; i < count * H; i++) {
        x[i] = (ORC_PLANT == 7 ? before[i] : x[i]) + o[i];
    }
    free(before);
    free(xn); free(q); free(k); free(v); free(rq); free(rk); free(attn); free(o);
    free(gate); free(up); free(cosine); free(sine); free(factor);
}

int orc_model_forward(int schedule, orc_model *model, const int64_t *ids,
    size_t length, size_t count, float *logits)
{
    if (!model || !ids || !logits || !count || length + count > model->capacity ||
        model->layer_count > ORC_LAYERS) {
        return -1;
    }
    for (size_t t = 0; t < count; t++) {
        if (ids[t] < 0 || ids[t] >= ORC_VOCAB) {
            return -1;
        }
    }
    float *x = malloc(count * ORC_HIDDEN * sizeof(float));
    if (!x) {
        return -1;
    }
    for (size_t t = 0; t < count; t++) {
        widen(model->embedding + (size_t)ids[t] * ORC_HIDDEN, x + t * ORC_HIDDEN, ORC_HIDDEN);
    }
    for (size_t layer = 0; layer < model->layer_count; layer++) {
        orc_layer_forward(schedule, model, layer, x, length, count);
    }
    float gamma[ORC_HIDDEN], final[ORC_HIDDEN];
    widen(model->final_norm, gamma, ORC_HIDDEN);
    size_t last = ORC_PLANT == 5 ? 0 : count - 1;
    orc_rmsnorm(schedule, gamma, x + last * ORC_HIDDEN, final, ORC_HIDDEN, 1);
    orc_matvec(schedule, ORC_W_BF16, model->embedding, 1.0f, final, logits,
        ORC_VOCAB, ORC_HIDDEN, 1);
    free(x);
    return 0;
}
