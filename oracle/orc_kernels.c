/* Oracle kernels: matvec, RMSNorm, RoPE, SiLU*up, causal GQA attention, in the
 * reference-literal (ORC_REF) and device-mirror (ORC_MIRROR) schedules.
 * TEST INFRASTRUCTURE ONLY (see oracle.h). */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int orc_threads;

void orc_set_threads(int threads)
{
    orc_threads = threads > 0 ? threads : 0;
#ifdef _OPENMP
    if (threads > 0) {
        omp_set_num_threads(threads);
    }
#endif
}

int orc_get_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Pairwise halving trees. tree32 stands in for Apple simd_sum (whose order is
 * unpinned); tree64 is the device wave reduction (shuffle-down by 32,16,..,1). */
static float tree32(float v[32])
{
    for (int s = 16; s >= 1; s >>= 1) {
        for (int i = 0; i < s; i++) {
            v[i] = v[i] + v[i + s];
        }
    }
    return v[0];
}

static float tree64(float v[64])
{
    for (int s = 32; s >= 1; s >>= 1) {
        for (int i = 0; i < s; i++) {
            v[i] = v[i] + v[i + s];
        }
    }
    return v[0];
}

static void weight_row(int kind, const void *weights, const float lut[256], size_t row,
    size_t cols, float *out)
{
    if (kind == ORC_W_FP8) {
        const uint8_t *w = (const uint8_t *)weights + row * cols;
        for (size_t c = 0; c < cols; c++) {
            out[c] = lut[w[c]];
        }
    } else if (kind == ORC_W_BF16) {
        const uint16_t *w = (const uint16_t *)weights + row * cols;
        for (size_t c = 0; c < cols; c++) {
            out[c] = orc_bf16_widen(w[c]);
        }
    } else {
        memcpy(out, (const float *)weights + row * cols, cols * sizeof(float));
    }
}

/* Reference-literal row dot, src/metal_kernels.metal:7-27 and :153-177:
 * lane l Kahan-sums fl(w*x) over c == l (mod 32) in increasing c, then the
 * 32-lane tree. w is already fl(dec*s) for FP8 (weight(), :136-144). */
static float dot_ref(const float *w, const float *x, size_t cols)
{
    float sum[32] = {0}, correction[32] = {0};
    size_t full = cols / 32 * 32;
    for (size_t base = 0; base < full; base += 32) {
        for (int l = 0; l < 32; l++) {
            float product = w[base + l] * x[base + l];
            float value = product - correction[l];
            float next = sum[l] + value;
            correction[l] = (next - sum[l]) - value;
            sum[l] = next;
        }
    }
    for (size_t c = full; c < cols; c++) {
        int l = (int)(c - full);
        float product = w[c] * x[c];
        float value = product - correction[l];
        float next = sum[l] + value;
        correction[l] = (next - sum[l]) - value;
        sum[l] = next;
    }
    return tree32(sum);
}

/* Device-mirror row dot: columns in chunks of 1024; lane l owns columns
 * [16l, 16l+16) of every chunk and runs acc = fma(w, x, acc) from 0 over all
 * of them (chunk by chunk, column order); the 64 lane sums reduce by tree64. */
static float dot_mirror(const float *w, const float *x, size_t cols)
{
    float acc[64] = {0};
    for (size_t base = 0; base < cols; base += 1024) {
        if (base + 1024 <= cols) {
            /* 64 independent chains interleaved; each lane's order is kept. */
            for (int j = 0; j < 16; j++) {
                for (int l = 0; l < 64; l++) {
                    acc[l] = fmaf(w[base + 16 * l + j], x[base + 16 * l + j], acc[l]);
                }
            }
        } else {
            for (int l = 0; l < 64; l++) {
                size_t first = base + 16 * (size_t)l;
                for (size_t c = first; c < first + 16 && c < cols; c++) {
                    acc[l] = fmaf(w[c], x[c], acc[l]);
                }
            }
        }
    }
    return tree64(acc);
}

/* Permuted copy for dot_mirror_perm: in every full 1024-column chunk, element
 * 16l + j moves to j*64 + l, so lane l's sixteen columns sit at stride 64 and
 * the 64 lane chains of one j advance as contiguous vectors. A partial last
 * chunk is copied unchanged. */
static void permute_chunks(const float *src, float *dst, size_t cols)
{
    size_t full = cols / 1024 * 1024;
    for (size_t base = 0; base < full; base += 1024) {
        for (int l = 0; l < 64; l++) {
            for (int j = 0; j < 16; j++) {
                dst[base + (size_t)j * 64 + l] = src[base + 16 * (size_t)l + j];
            }
        }
    }
    memcpy(dst + full, src + full, (cols - full) * sizeof(float));
}

/* dot_mirror over permuted operands: the same chains in the same order (lane l
 * takes its columns chunk by chunk, j = 0..15), evaluated 64 lanes at a time. */
static float dot_mirror_perm(const float *wp, const float *xp, size_t cols)
{
    float acc[64] = {0};
    size_t full = cols / 1024 * 1024;
    for (size_t base = 0; base < full; base += 1024) {
        for (int j = 0; j < 16; j++) {
            const float *wj = wp + base + (size_t)j * 64, *xj = xp + base + (size_t)j * 64;
            for (int l = 0; l < 64; l++) {
                acc[l] = fmaf(wj[l], xj[l], acc[l]);
            }
        }
    }
    for (int l = 0; l < 64; l++) {
        size_t first = full + 16 * (size_t)l;
        for (size_t c = first; c < first + 16 && c < cols; c++) {
            acc[l] = fmaf(wp[c], xp[c], acc[l]);
        }
    }
    return tree64(acc);
}

/* REF: per-element w = fl(dec*scale) (weight(), src/metal_kernels.metal:136-144)
 * then the Kahan lane dot. MIRROR: unscaled exact decode in the dot, the row
 * total times scale once. BF16 and FP32 weights use scale as given (1 for the
 * tied head and plain FP32 projections). Rows are taken in tiles of ORC_TILE so
 * a tile of weights stays in cache across the tokens. */
#define ORC_TILE 8
void orc_matvec(int schedule, int kind, const void *weights, float scale,
    const float *x, float *y, size_t rows, size_t cols, size_t tokens)
{
    float lut[256];
    for (int b = 0; b < 256; b++) {
        lut[b] = schedule == ORC_REF ? orc_fp8_decode((uint8_t)b) * scale :
            orc_fp8_decode((uint8_t)b);
    }
    const float *xs = x;
    float *xperm = NULL;
    if (schedule != ORC_REF) {
        xperm = malloc(tokens * cols * sizeof(float));
        #pragma omp parallel for schedule(static)
        for (size_t t = 0; t < tokens; t++) {
            permute_chunks(x + t * cols, xperm + t * cols, cols);
        }
        xs = xperm;
    }
    #pragma omp parallel
    {
        float *w = malloc(ORC_TILE * cols * sizeof(float));
        float *row = malloc(cols * sizeof(float));
        #pragma omp for schedule(static)
        for (size_t r0 = 0; r0 < rows; r0 += ORC_TILE) {
            size_t n = rows - r0 < ORC_TILE ? rows - r0 : ORC_TILE;
            for (size_t i = 0; i < n; i++) {
                if (schedule == ORC_REF) {
                    weight_row(kind, weights, lut, r0 + i, cols, w + i * cols);
                } else {
                    weight_row(kind, weights, lut, r0 + i, cols, row);
                    permute_chunks(row, w + i * cols, cols);
                }
            }
            for (size_t t = 0; t < tokens; t++) {
                for (size_t i = 0; i < n; i++) {
                    float *out = y + t * rows + r0 + i;
                    if (schedule == ORC_REF) {
                        float dot = dot_ref(w + i * cols, xs + t * cols, cols);
                        *out = kind == ORC_W_FP8 ? dot : dot * scale;
                    } else {
                        *out = dot_mirror_perm(w + i * cols, xs + t * cols, cols) * scale;
                    }
                }
            }
        }
        free(w);
        free(row);
    }
    free(xperm);
}

/* RMSNorm, src/metal_kernels.metal:29-44: out = gamma*(x*r),
 * r = 1/sqrt(ss/width + 1e-5). REF: per-lane v*v sums over c == l (mod 32) then
 * tree32. MIRROR: the dot_mirror order with fma(x, x, acc). */
void orc_rmsnorm(int schedule, const float *gamma, const float *x, float *out,
    size_t width, size_t tokens)
{
    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < tokens; t++) {
        const float *row = x + t * width;
        float ss;
        if (schedule == ORC_REF) {
            float lanes[32] = {0};
            for (size_t c = 0; c < width; c++) {
                lanes[c % 32] += row[c] * row[c];
            }
            ss = tree32(lanes);
        } else {
            ss = dot_mirror(row, row, width);
        }
        float r = 1.0f / sqrtf(ss / (float)width + 1e-5f);
        for (size_t c = 0; c < width; c++) {
            out[t * width + c] = gamma[c] * (row[c] * r);
        }
    }
}

/* Split-half rotation, src/metal_kernels.metal:59-78. */
void orc_rope(const float *x, const float *cosine, const float *sine,
    const float *qfactor, float *out, size_t width, size_t tokens)
{
    for (size_t t = 0; t < tokens; t++) {
        for (size_t i = 0; i < width; i++) {
            size_t index = t * width + i;
            size_t column = i % 128;
            float rotated = column < 64 ? -x[index + 64] : x[index - 64];
            float value = x[index] * cosine[t * 128 + column] + rotated * sine[t * 128 + column];
            if (qfactor) {
                value *= qfactor[t];
            }
            out[index] = value;
        }
    }
}

void orc_silu_mul(int schedule, const float *gate, const float *up, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        float s = schedule == ORC_REF ? orc_silu_ref(gate[i]) : orc_silu_mirror(gate[i]);
        out[i] = s * up[i];
    }
}

#define ORC_SCORE_SCALE 0.08838834764831845f

/* Reference-literal attention for one (token, head), src/metal_kernels.metal:
 * 80-132: lane partials of q*k over d == l (mod 32), tree32, times 1/sqrt(128);
 * max; e = exp(s - max) with lane partial sums over p == l (mod 32), tree32;
 * P = e / total; out[d] = sum_p P*V in position order. */
static void attend_ref(const float *q, const float *keys, const float *values,
    size_t head_stride, size_t pos_stride, size_t kvh, size_t n, float *scores, float *out)
{
    const float *k0 = keys + kvh * head_stride;
    const float *v0 = values + kvh * head_stride;
    float maximum = -INFINITY;
    for (size_t p = 0; p < n; p++) {
        float lanes[32] = {0};
        for (int d = 0; d < 128; d++) {
            lanes[d % 32] += q[d] * k0[p * pos_stride + d];
        }
        float s = tree32(lanes) * ORC_SCORE_SCALE;
        scores[p] = s;
        maximum = fmaxf(maximum, s);
    }
    float lanes[32] = {0};
    for (size_t p = 0; p < n; p++) {
        float e = expf(scores[p] - maximum);
        scores[p] = e;
        lanes[p % 32] += e;
    }
    float total = tree32(lanes);
    for (size_t p = 0; p < n; p++) {
        scores[p] = scores[p] / total;
    }
    for (int d = 0; d < 128; d++) {
        float sum = 0;
        for (size_t p = 0; p < n; p++) {
            sum += scores[p] * v0[p * pos_stride + d];
        }
        out[d] = sum;
    }
}

/* Device-mirror attention for one (token, head), 64-position blocks b:
 *   c_i = chain over d in [32i, 32i+32) of fma(q_d, k_pd) from 0 (i = 0..3);
 *   s_p = fl(((c_0 + c_1) + (c_2 + c_3)) * 1/sqrt(128));
 *   m_b = max of the block's s_p; e_p = orc_expf(s_p - m_b);
 *   T_b = tree64(e, zero-padded); A_b[d] = chain over the block's valid p of
 *   fma(e_p, v_pd, acc) from 0;
 *   M = max_b m_b; f_b = orc_expf(m_b - M);
 *   groups of 8 consecutive blocks: S_g[d] = chain fma(f_b, A_b[d]) and
 *   U_g = chain fma(f_b, T_b), both from 0 in block order;
 *   A = S_0 + S_1 + ..., T = U_0 + U_1 + ... left to right; out[d] = A[d] / T.
 * It is evaluated in tiled phases so each K/V block is read
 * once per tile of query rows rather than once per row: per (kv head, block),
 * a transposed copy of the K block feeds the four heads' score chains 64
 * positions at a time, then the block partials (m_b, T_b, A_b) are formed with
 * the V block hot in cache; the combine runs per (row, head). Every value goes
 * through the same operations in the same order as the per-row statement. */
#define ORC_ROWS 32
static void attention_mirror(const float *q, const float *keys, const float *values,
    size_t head_stride, size_t pos_stride, size_t prefix, size_t count, float *out)
{
    for (size_t t0 = 0; t0 < count; t0 += ORC_ROWS) {
        const size_t tn = count - t0 < ORC_ROWS ? count - t0 : ORC_ROWS;
        const size_t nmax = prefix + t0 + tn;
        const size_t nb = (nmax + 63) / 64;
        float *bmax = malloc(tn * ORC_HEADS * nb * sizeof(float));
        float *btotal = malloc(tn * ORC_HEADS * nb * sizeof(float));
        float *bacc = malloc(tn * ORC_HEADS * nb * 128 * sizeof(float));
        #pragma omp parallel for schedule(dynamic) collapse(2)
        for (size_t kvh = 0; kvh < ORC_KV_HEADS; kvh++) {
            for (size_t b = 0; b < nb; b++) {
                const float *k0 = keys + kvh * head_stride;
                const float *v0 = values + kvh * head_stride;
                float kt[128][64];
                for (size_t l = 0; l < 64; l++) {
                    size_t p = b * 64 + l;
                    for (int d = 0; d < 128; d++) {
                        kt[d][l] = p < nmax ? k0[p * pos_stride + d] : 0.0f;
                    }
                }
                for (size_t tt = 0; tt < tn; tt++) {
                    const size_t n = prefix + t0 + tt + 1;
                    if (b * 64 >= n) {
                        continue;
                    }
                    const size_t valid = n - b * 64 < 64 ? n - b * 64 : 64;
                    for (size_t hh = 0; hh < 4; hh++) {
                        const size_t h = kvh * 4 + hh, row = (tt * ORC_HEADS + h) * nb + b;
                        const float *qv = q + (t0 + tt) * ORC_QUERY + h * ORC_HEAD_DIM;
                        float c[4][64], s[64];
                        for (int i = 0; i < 4; i++) {
                            for (int l = 0; l < 64; l++) {
                                c[i][l] = 0.0f;
                            }
                            for (int d = 32 * i; d < 32 * i + 32; d++) {
                                for (int l = 0; l < 64; l++) {
                                    c[i][l] = fmaf(qv[d], kt[d][l], c[i][l]);
                                }
                            }
                        }
                        float block_max = -INFINITY;
                        for (size_t l = 0; l < 64; l++) {
                            s[l] = ((c[0][l] + c[1][l]) + (c[2][l] + c[3][l])) * ORC_SCORE_SCALE;
                            if (l < valid) {
                                block_max = fmaxf(block_max, s[l]);
                            }
                        }
                        float lanes[64];
                        float *acc = bacc + row * 128;
                        for (int d = 0; d < 128; d++) {
                            acc[d] = 0.0f;
                        }
                        for (size_t l = 0; l < 64; l++) {
                            lanes[l] = 0.0f;
                            if (l < valid) {
                                float e = orc_expf(s[l] - block_max);
                                const float *v = v0 + (b * 64 + l) * pos_stride;
                                lanes[l] = e;
                                for (int d = 0; d < 128; d++) {
                                    acc[d] = fmaf(e, v[d], acc[d]);
                                }
                            }
                        }
                        bmax[row] = block_max;
                        btotal[row] = tree64(lanes);
                    }
                }
            }
        }
        #pragma omp parallel for schedule(static) collapse(2)
        for (size_t tt = 0; tt < tn; tt++) {
            for (size_t h = 0; h < ORC_HEADS; h++) {
                const size_t n = prefix + t0 + tt + 1, nbr = (n + 63) / 64;
                const size_t base = (tt * ORC_HEADS + h) * nb;
                float maximum = -INFINITY;
                for (size_t b = 0; b < nbr; b++) {
                    maximum = fmaxf(maximum, bmax[base + b]);
                }
                float total = 0.0f, sum[128] = {0};
                for (size_t g = 0; g * 8 < nbr; g++) {
                    float group_total = 0.0f, group[128] = {0};
                    for (size_t b = g * 8; b < g * 8 + 8 && b < nbr; b++) {
                        float f = orc_expf(bmax[base + b] - maximum);
                        group_total = fmaf(f, btotal[base + b], group_total);
                        for (int d = 0; d < 128; d++) {
                            group[d] = fmaf(f, bacc[(base + b) * 128 + d], group[d]);
                        }
                    }
                    if (g == 0) {
                        total = group_total;
                        memcpy(sum, group, sizeof sum);
                    } else {
                        total = total + group_total;
                        for (int d = 0; d < 128; d++) {
                            sum[d] = sum[d] + group[d];
                        }
                    }
                }
                float *oh = out + (t0 + tt) * ORC_QUERY + h * ORC_HEAD_DIM;
                for (int d = 0; d < 128; d++) {
                    oh[d] = sum[d] / total;
                }
            }
        }
        free(bmax);
        free(btotal);
        free(bacc);
    }
}

void orc_attention(int schedule, const float *q, const float *keys, const float *values,
    size_t head_stride, size_t pos_stride, size_t prefix, size_t count, float *out)
{
    if (schedule != ORC_REF) {
        attention_mirror(q, keys, values, head_stride, pos_stride, prefix, count, out);
        return;
    }
    #pragma omp parallel
    {
        float *scores = malloc((prefix + count) * sizeof(float));
        #pragma omp for schedule(dynamic) collapse(2)
        for (size_t t = 0; t < count; t++) {
            for (size_t h = 0; h < ORC_HEADS; h++) {
                size_t n = prefix + t + 1;
                const float *qh = q + t * ORC_QUERY + h * ORC_HEAD_DIM;
                float *oh = out + t * ORC_QUERY + h * ORC_HEAD_DIM;
                attend_ref(qh, keys, values, head_stride, pos_stride, h / 4, n, scores, oh);
            }
        }
        free(scores);
    }
}
