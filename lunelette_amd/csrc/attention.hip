// Causal GQA attention over the resident FP32 KV cache, split across
// workgroups by 64-position blocks (src/metal_kernels.metal:80-132 computes the
// same softmax(q.k/sqrt(128)).V with one SIMD group walking every position).
//
//   k_attn_scores : (block, kv_head, token) -> s_p for the 4 query heads that
//                   share the kv head (K tile staged once in LDS), block max.
//   k_attn_pv     : global max over block maxima, e_p = exp(s_p - M), block
//                   sum by the 64-lane tree, block partial A_b[d] = sum e_p v_pd.
//   k_attn_combine: blocks -> 256-position tiles -> tiles, in order; out = A/T.
//
// KV layout [kv_head][capacity][128] per layer keeps each block's K or V tile
// one contiguous 32 KiB read. Positions at or beyond length+t+1 are never read
// into arithmetic.
#include "lh_device.h"
#include "lh_internal.h"

namespace lh {

__global__ void __launch_bounds__(256)
k_attn_scores(const float* __restrict__ q, const float* __restrict__ kcache,
    const lh_step_params* __restrict__ params, uint32_t capacity, float* __restrict__ S,
    float* __restrict__ BM)
{
    __shared__ float Kt[LH_ATTN_BLOCK][LH_HEAD_DIM + 1];
    __shared__ float qs[4][LH_HEAD_DIM];
    const uint32_t b = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const uint32_t n = params->length + t + 1;
    if (b * LH_ATTN_BLOCK >= n) {
        return;
    }
    const uint32_t valid = n - b * LH_ATTN_BLOCK < LH_ATTN_BLOCK ? n - b * LH_ATTN_BLOCK : LH_ATTN_BLOCK;
    const float* kb = kcache + lh_kv_index(capacity, 0, kvh, (uint64_t)b * LH_ATTN_BLOCK);
    for (uint32_t i = threadIdx.x; i < LH_ATTN_BLOCK * 32; i += 256) {
        const uint32_t r = i >> 5, c4 = i & 31;
        if (r < valid) {
            float4 v = reinterpret_cast<const float4*>(kb + (size_t)r * LH_HEAD_DIM)[c4];
            Kt[r][4 * c4 + 0] = v.x;
            Kt[r][4 * c4 + 1] = v.y;
            Kt[r][4 * c4 + 2] = v.z;
            Kt[r][4 * c4 + 3] = v.w;
        }
    }
    for (uint32_t i = threadIdx.x; i < 4 * LH_HEAD_DIM; i += 256) {
        qs[i >> 7][i & 127] = q[(size_t)t * LH_QUERY + kvh * 4 * LH_HEAD_DIM + i];
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t h = kvh * 4 + wave;
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    float s = -__builtin_inff();
    if (lane < valid) {
        float acc = 0.0f;
#pragma unroll 8
        for (int d = 0; d < LH_HEAD_DIM; d++) {
            acc = __builtin_fmaf(qs[wave][d], Kt[lane][d], acc);
        }
        s = acc * LH_SCORE_SCALE;
        S[((size_t)t * LH_HEADS + h) * capacity + b * LH_ATTN_BLOCK + lane] = s;
    }
    const float m = wave_max64(s);
    if (lane == 0) {
        BM[((size_t)t * LH_HEADS + h) * nbc + b] = m;
    }
}

__global__ void __launch_bounds__(256)
k_attn_pv(const float* __restrict__ S, const float* __restrict__ BM,
    const float* __restrict__ vcache, const lh_step_params* __restrict__ params,
    uint32_t capacity, float* __restrict__ PT, float* __restrict__ PA)
{
    __shared__ float Vt[LH_ATTN_BLOCK][LH_HEAD_DIM];
    __shared__ float es[4][LH_ATTN_BLOCK];
    const uint32_t b = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const uint32_t n = params->length + t + 1;
    if (b * LH_ATTN_BLOCK >= n) {
        return;
    }
    const uint32_t valid = n - b * LH_ATTN_BLOCK < LH_ATTN_BLOCK ? n - b * LH_ATTN_BLOCK : LH_ATTN_BLOCK;
    const uint32_t nb = (n + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    const float* vb = vcache + lh_kv_index(capacity, 0, kvh, (uint64_t)b * LH_ATTN_BLOCK);
    for (uint32_t i = threadIdx.x; i < LH_ATTN_BLOCK * 32; i += 256) {
        const uint32_t r = i >> 5, c4 = i & 31;
        if (r < valid) {
            reinterpret_cast<float4*>(&Vt[r][0])[c4] =
                reinterpret_cast<const float4*>(vb + (size_t)r * LH_HEAD_DIM)[c4];
        }
    }
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t h = kvh * 4 + wave;
    const size_t th = (size_t)t * LH_HEADS + h;
    float m = -__builtin_inff();
    for (uint32_t j = lane; j < nb; j += 64) {
        m = fmaxf(m, BM[th * nbc + j]);
    }
    m = wave_max64(m);
    float e = 0.0f;
    if (lane < valid) {
        e = expf_cw(S[th * capacity + b * LH_ATTN_BLOCK + lane] - m);
    }
    es[wave][lane] = e;
    const float total = wave_tree64(e);
    if (lane == 0) {
        PT[th * nbc + b] = total;
    }
    __syncthreads();
    float a0 = 0.0f, a1 = 0.0f;
    const uint32_t d0 = 2 * lane;
    for (uint32_t j = 0; j < valid; j++) {
        const float ej = es[wave][j];
        const float2 v = *reinterpret_cast<const float2*>(&Vt[j][d0]);
        a0 = __builtin_fmaf(ej, v.x, a0);
        a1 = __builtin_fmaf(ej, v.y, a1);
    }
    float2* pa = reinterpret_cast<float2*>(PA + (th * nbc + b) * LH_HEAD_DIM + d0);
    *pa = make_float2(a0, a1);
}

// grid (32 heads, count), block 64.
__global__ void __launch_bounds__(64)
k_attn_combine(const float* __restrict__ PT, const float* __restrict__ PA,
    const lh_step_params* __restrict__ params, uint32_t capacity, float* __restrict__ out)
{
    const uint32_t h = blockIdx.x, t = blockIdx.y;
    const uint32_t n = params->length + t + 1;
    const uint32_t nb = (n + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    const size_t th = (size_t)t * LH_HEADS + h;
    const uint32_t d0 = 2 * threadIdx.x;
    float T = 0.0f, A0 = 0.0f, A1 = 0.0f;
    for (uint32_t tile = 0; tile * LH_ATTN_TILE < nb; tile++) {
        const uint32_t b0 = tile * LH_ATTN_TILE;
        float tT = PT[th * nbc + b0];
        float2 tA = *reinterpret_cast<const float2*>(PA + (th * nbc + b0) * LH_HEAD_DIM + d0);
        for (uint32_t b = b0 + 1; b < b0 + LH_ATTN_TILE && b < nb; b++) {
            const float2 a = *reinterpret_cast<const float2*>(PA + (th * nbc + b) * LH_HEAD_DIM + d0);
            tT = tT + PT[th * nbc + b];
            tA.x = tA.x + a.x;
            tA.y = tA.y + a.y;
        }
        if (tile == 0) {
            T = tT;
            A0 = tA.x;
            A1 = tA.y;
        } else {
            T = T + tT;
            A0 = A0 + tA.x;
            A1 = A1 + tA.y;
        }
    }
    float2* o = reinterpret_cast<float2*>(out + (size_t)t * LH_QUERY + h * LH_HEAD_DIM + d0);
    *o = make_float2(A0 / T, A1 / T);
}

// Embedding gather with exact BF16 widening (src/metal_runtime.m:388-395 copies
// the FP32-expanded row). grid (count), block 256.
__global__ void __launch_bounds__(256)
k_embed(const uint16_t* __restrict__ E, const lh_step_params* __restrict__ params,
    float* __restrict__ x)
{
    const uint32_t t = blockIdx.x;
    const uint16_t* row = E + (size_t)params->tokens[t].id * LH_HIDDEN;
    for (uint32_t c = threadIdx.x; c < LH_HIDDEN; c += 256) {
        x[(size_t)t * LH_HIDDEN + c] = bf16_to_f32(row[c]);
    }
}

}  // namespace lh

using namespace lh;

extern "C" int lh_launch_attention(const float* q, const float* kcache_layer,
    const float* vcache_layer, const lh_step_params* params, uint32_t count,
    uint32_t max_positions, uint32_t capacity, float* S, float* BM, float* PT, float* PA,
    float* out, hipStream_t s)
{
    if (!count || capacity % LH_ATTN_BLOCK || max_positions > capacity || !max_positions) {
        return -1;
    }
    const uint32_t blocks = (max_positions + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    dim3 grid(blocks, LH_KV_HEADS, count);
    hipLaunchKernelGGL(k_attn_scores, grid, dim3(256), 0, s, q, kcache_layer, params, capacity, S, BM);
    hipLaunchKernelGGL(k_attn_pv, grid, dim3(256), 0, s, S, BM, vcache_layer, params, capacity, PT, PA);
    hipLaunchKernelGGL(k_attn_combine, dim3(LH_HEADS, count), dim3(64), 0, s, PT, PA, params,
        capacity, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_embed(const uint16_t* E, const lh_step_params* params, uint32_t count,
    float* x, hipStream_t s)
{
    hipLaunchKernelGGL(k_embed, dim3(count), dim3(256), 0, s, E, params, x);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
