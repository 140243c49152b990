// Elementwise operators for the unfused (one operator per kernel) path and
// the kernel-level ABI: element (add / SiLU / multiply), RoPE, RoPE + KV append,
// and checks of the device FP8 decode and exp.
#include "lh_device.h"
#include "lh_internal.h"

namespace lh {

// src/metal_kernels.metal:46-57.
__global__ void k_element(int mode, const float* __restrict__ a, const float* __restrict__ b,
    float* __restrict__ out, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    const float v = a[i];
    out[i] = mode == 0 ? v + b[i] : (mode == 1 ? silu(v) : v * b[i]);
}

// Streaming-read measurement: `words` 16-byte words from src, wave w reading
// the contiguous range [w, w+1) * words / waves with U non-temporal loads in
// flight per lane, folded by XOR so that no load is dead; a lane writes sink
// only if its fold equals a value chosen so that it practically never does.
typedef uint32_t rf_u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ void __launch_bounds__(256)
k_read_floor(const rf_u32x4* __restrict__ src, size_t words, uint32_t* __restrict__ sink)
{
    const size_t waves = (size_t)gridDim.x * 4;
    const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    const size_t per_wave = words / waves;   // a multiple of 64 * U
    const rf_u32x4* p = src + wave * per_wave + lane;
    uint32_t acc = 0;
    for (size_t i = 0; i < per_wave; i += 64 * U) {
        rf_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            v[u] = __builtin_nontemporal_load(p + i + 64 * u);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
    }
    if (acc == 0x9e3779b9u) {
        sink[wave] = acc;
    }
}

// SiLU(gate)*up in one pass.
__global__ void k_silu_mul(const float* __restrict__ gate, const float* __restrict__ up,
    float* __restrict__ out, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        out[i] = silu(gate[i]) * up[i];
    }
}

__device__ __forceinline__ float rope_at(const float* row, const float* cosine, const float* sine,
    uint32_t i)
{
    const uint32_t column = i & 127u;
    const float rotated = column < 64 ? -row[i + 64] : row[i - 64];
    return row[i] * cosine[column] + rotated * sine[column];
}

// src/metal_kernels.metal:59-78 with per-token cos/sin rows [tokens][128].
__global__ void k_rope(const float* __restrict__ x, const float* __restrict__ cosine,
    const float* __restrict__ sine, const float* __restrict__ qfactor, float* __restrict__ out,
    uint32_t width, uint32_t tokens)
{
    const size_t index = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (index >= (size_t)width * tokens) {
        return;
    }
    const uint32_t t = (uint32_t)(index / width), i = (uint32_t)(index % width);
    float v = rope_at(x + (size_t)t * width, cosine + t * 128, sine + t * 128, i);
    if (qfactor) {
        v = v * qfactor[t];
    }
    out[index] = v;
}

// Unfused tail of the q|k|v projection: RoPE Q (with the query factor) into
// qout, RoPE K and raw V appended to the cache (src/metal_encode.m:137-153).
// q_raw [count][4096], k_raw/v_raw [count][1024]; grid (count), block 256.
__global__ void k_rope_append(const float* __restrict__ q_raw, const float* __restrict__ k_raw,
    const float* __restrict__ v_raw, const lh_step_params* __restrict__ params,
    float* __restrict__ qout, float* __restrict__ kcache, float* __restrict__ vcache,
    uint32_t capacity)
{
    const uint32_t t = blockIdx.x;
    const lh_token_params* tp = &params->tokens[t];
    const uint32_t position = params->length + t;
    const float* qr = q_raw + (size_t)t * LH_QUERY;
    const float* kr = k_raw + (size_t)t * LH_KV;
    const float* vr = v_raw + (size_t)t * LH_KV;
    for (uint32_t i = threadIdx.x; i < LH_QUERY; i += blockDim.x) {
        qout[(size_t)t * LH_QUERY + i] = rope_at(qr, tp->cosine, tp->sine, i) * tp->qfactor;
    }
    for (uint32_t k = threadIdx.x; k < LH_KV; k += blockDim.x) {
        kcache[lh_k_index(capacity, 0, k >> 7, position, k & 127u)] =
            rope_at(kr, tp->cosine, tp->sine, k);
        vcache[lh_kv_index(capacity, 0, k >> 7, position) + (k & 127u)] = vr[k];
    }
}

__global__ void k_fp8_decode(const uint8_t* __restrict__ codes, float* __restrict__ out, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float four[4];
        fp8x4_to_f32(codes[i], four);
        out[i] = four[0];
    }
}

__global__ void k_expf(const float* __restrict__ x, float* __restrict__ out, size_t n)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        out[i] = expf_cw(x[i]);
    }
}

}  // namespace lh

using namespace lh;

static inline dim3 grid_for(size_t n)
{
    return dim3((unsigned)((n + 255) / 256));
}

extern "C" int lh_launch_element(int mode, const float* a, const float* b, float* out, size_t n,
    hipStream_t s)
{
    hipLaunchKernelGGL(k_element, grid_for(n), dim3(256), 0, s, mode, a, b, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_silu_mul(const float* gate, const float* up, float* out, size_t n,
    hipStream_t s)
{
    hipLaunchKernelGGL(k_silu_mul, grid_for(n), dim3(256), 0, s, gate, up, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_rope(const float* x, const float* cosine, const float* sine,
    const float* qfactor, float* out, uint32_t width, uint32_t tokens, hipStream_t s)
{
    hipLaunchKernelGGL(k_rope, grid_for((size_t)width * tokens), dim3(256), 0, s, x, cosine, sine,
        qfactor, out, width, tokens);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_rope_append(const float* q_raw, const float* k_raw, const float* v_raw,
    const lh_step_params* params, uint32_t count, float* q, float* kcache_layer,
    float* vcache_layer, uint32_t capacity, hipStream_t s)
{
    hipLaunchKernelGGL(k_rope_append, dim3(count), dim3(256), 0, s, q_raw, k_raw, v_raw, params,
        q, kcache_layer, vcache_layer, capacity);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_fp8_decode(const uint8_t* codes, float* out, size_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_fp8_decode, grid_for(n), dim3(256), 0, s, codes, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_expf(const float* x, float* out, size_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_expf, grid_for(n), dim3(256), 0, s, x, out, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_read_floor(const void* src, size_t bytes, uint32_t grid, uint32_t unroll,
    uint32_t* sink, hipStream_t s)
{
    const rf_u32x4* w = static_cast<const rf_u32x4*>(src);
    const size_t words = bytes / 16;
    switch (unroll) {
    case 1: hipLaunchKernelGGL(k_read_floor<1>, dim3(grid), dim3(256), 0, s, w, words, sink); break;
    case 2: hipLaunchKernelGGL(k_read_floor<2>, dim3(grid), dim3(256), 0, s, w, words, sink); break;
    case 4: hipLaunchKernelGGL(k_read_floor<4>, dim3(grid), dim3(256), 0, s, w, words, sink); break;
    case 8: hipLaunchKernelGGL(k_read_floor<8>, dim3(grid), dim3(256), 0, s, w, words, sink); break;
    default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
