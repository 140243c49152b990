// Decode / precise-path projections for gfx950. Every output row is a
// canonical row dot (lh_schedule.h): lane l of a wave owns 16 consecutive
// columns of each 1024-column chunk, loads them with one 16-byte load per
// 16 FP8 codes (32 B for BF16, 64 B for FP32), decodes in registers, chains
// fused multiply-adds, and the chunk reduces by the fixed 64-lane tree. Chunks
// are spread over the waves of a workgroup and summed in chunk order.
//
// The FP8 element is w = fl(dec(code) * scale) exactly as the reference's
// weight() (src/metal_kernels.metal:136-144), so compact FP8 and resident FP32
// weights give identical bits. The reference sums fl(w*x) with per-lane Kahan
// (:153-177); here the product and sum are one fused multiply-add.
#include "lh_device.h"
#include "lh_internal.h"

namespace lh {

enum { K_FP8 = 0, K_BF16 = 1, K_F32 = 2 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int KIND> struct WVec;
template <> struct WVec<K_FP8> { u32x4 v[1]; };
template <> struct WVec<K_BF16> { u32x4 v[2]; };
template <> struct WVec<K_F32> { u32x4 v[4]; };

template <int KIND> constexpr int elem_bytes() { return KIND == K_FP8 ? 1 : (KIND == K_BF16 ? 2 : 4); }

// Vector load of the 16 elements a lane owns at column `col` of `row`.
template <int KIND>
__device__ __forceinline__ void load_w(WVec<KIND>& w, const void* base, size_t row, uint32_t cols,
    uint32_t col)
{
    const u32x4* p = reinterpret_cast<const u32x4*>(
        static_cast<const char*>(base) + (row * cols + col) * elem_bytes<KIND>());
#pragma unroll
    for (int i = 0; i < (int)(sizeof(WVec<KIND>) / 16); i++) {
        w.v[i] = __builtin_nontemporal_load(p + i);
    }
}

// Decode the 16 elements held in `w` to FP32 weights (scaled for FP8).
template <int KIND, bool LUT>
__device__ __forceinline__ void decode16(const WVec<KIND>& w, float scale, const float* lut,
    float out[16])
{
    if constexpr (KIND == K_FP8) {
        const uint32_t words[4] = {w.v[0].x, w.v[0].y, w.v[0].z, w.v[0].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float d[4];
            if constexpr (LUT) {
                d[0] = lut[words[i] & 255u];
                d[1] = lut[(words[i] >> 8) & 255u];
                d[2] = lut[(words[i] >> 16) & 255u];
                d[3] = lut[words[i] >> 24];
            } else {
                fp8x4_to_f32(words[i], d);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                out[4 * i + j] = d[j] * scale;
            }
        }
    } else if constexpr (KIND == K_BF16) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t words[4] = {w.v[i].x, w.v[i].y, w.v[i].z, w.v[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                out[8 * i + 2 * j] = __uint_as_float(words[j] << 16);
                out[8 * i + 2 * j + 1] = __uint_as_float(words[j] & 0xffff0000u);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            out[4 * i + 0] = __uint_as_float(w.v[i].x);
            out[4 * i + 1] = __uint_as_float(w.v[i].y);
            out[4 * i + 2] = __uint_as_float(w.v[i].z);
            out[4 * i + 3] = __uint_as_float(w.v[i].w);
        }
    }
}

// Scalar element fetch for unaligned shapes (partial lanes only).
template <int KIND, bool LUT>
__device__ __forceinline__ float load_elem(const void* base, size_t index, float scale,
    const float* lut)
{
    if constexpr (KIND == K_FP8) {
        uint32_t code = static_cast<const uint8_t*>(base)[index];
        float d;
        if constexpr (LUT) {
            d = lut[code];
        } else {
            float four[4];
            fp8x4_to_f32(code, four);
            d = four[0];
        }
        return d * scale;
    } else if constexpr (KIND == K_BF16) {
        return __uint_as_float((uint32_t)static_cast<const uint16_t*>(base)[index] << 16);
    } else {
        return static_cast<const float*>(base)[index];
    }
}

__device__ __forceinline__ float chain16(const float w[16], const float x[16])
{
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        acc = __builtin_fmaf(w[j], x[j], acc);
    }
    return acc;
}

__device__ __forceinline__ void load_x16(const float* x, float out[16])
{
    const float4* p = reinterpret_cast<const float4*>(x);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 v = p[i];
        out[4 * i + 0] = v.x;
        out[4 * i + 1] = v.y;
        out[4 * i + 2] = v.z;
        out[4 * i + 3] = v.w;
    }
}

// Unscaled E4M3FN table for the lookup strategy, filled from the arithmetic
// decode so both strategies agree bit for bit.
__device__ __forceinline__ void fill_lut(float* lut)
{
    for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
        float four[4];
        fp8x4_to_f32(i, four);
        lut[i] = four[0];
    }
}

// Canonical RMSNorm prologue for a 3-chunk (3072-wide) row held as one chunk
// per wave: every thread ends with r; lane values are normalized in place.
template <int NW>
__device__ __forceinline__ void rmsnorm_chunk_prologue(float xs[16], const float* gamma,
    uint32_t col, float* lds_ss, uint32_t nchunks, uint32_t width)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        acc = __builtin_fmaf(xs[j], xs[j], acc);
    }
    acc = wave_tree64(acc);
    if (lane == 0) {
        lds_ss[wave] = acc;
    }
    __syncthreads();
    float ss = lds_ss[0];
    for (uint32_t c = 1; c < nchunks; c++) {
        ss = ss + lds_ss[c];
    }
    float r = 1.0f / __builtin_sqrtf(ss / (float)width + 1e-5f);
    float g[16];
    load_x16(gamma + col, g);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        xs[j] = g[j] * (xs[j] * r);
    }
}

// ---------------------------------------------------------------------------
// Generic row dots: y[t][r] = (residual ? residual[t][r] : 0 +) dot(W[r], x[t]).
// grid (ceil(rows/R), tokens), block NW waves. VEC requires cols*elem % 16 == 0.
template <int KIND, bool LUT, bool VEC, int NW, int R>
__global__ void __launch_bounds__(NW * 64)
k_matvec(const void* __restrict__ W, float scale, const float* __restrict__ x,
    float* y, const float* residual, uint32_t rows, uint32_t cols)
{
    extern __shared__ float smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t row0 = blockIdx.x * R;
    const uint32_t nch = (cols + LH_CHUNK - 1) / LH_CHUNK;
    float* Q = smem;
    float* lut = smem + R * nch;
    if constexpr (LUT) {
        fill_lut(lut);
        __syncthreads();
    }
    const float* xt = x + (size_t)t * cols;
    for (uint32_t c = wave; c < nch; c += NW) {
        const uint32_t col = c * LH_CHUNK + lane * LH_LANE_COLS;
        const int valid = col >= cols ? 0 : (cols - col >= 16 ? 16 : (int)(cols - col));
        float acc[R];
        if (VEC && valid == 16) {
            float xs[16];
            load_x16(xt + col, xs);
            WVec<KIND> wv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                if (row0 + r < rows) {
                    load_w<KIND>(wv[r], W, row0 + r, cols, col);
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float w[16];
                decode16<KIND, LUT>(wv[r], scale, lut, w);
                acc[r] = row0 + r < rows ? chain16(w, xs) : 0.0f;
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; r++) {
                float a = 0.0f;
                if (row0 + r < rows) {
                    for (int j = 0; j < valid; j++) {
                        float w = load_elem<KIND, LUT>(W, (size_t)(row0 + r) * cols + col + j,
                            scale, lut);
                        a = __builtin_fmaf(w, xt[col + j], a);
                    }
                }
                acc[r] = a;
            }
        }
        // Trees run with the whole wave converged.
#pragma unroll
        for (int r = 0; r < R; r++) {
            float total = wave_tree64(acc[r]);
            if (lane == 0) {
                Q[r * nch + c] = total;
            }
        }
    }
    __syncthreads();
    const uint32_t r = threadIdx.x;
    if (r < R && row0 + r < rows) {
        float v = Q[r * nch];
        for (uint32_t c = 1; c < nch; c++) {
            v = v + Q[r * nch + c];
        }
        const size_t o = (size_t)t * rows + row0 + r;
        y[o] = residual ? residual[o] + v : v;
    }
}

// ---------------------------------------------------------------------------
// Fused RMSNorm -> q|k|v rows -> RoPE (+ query factor on Q) -> Q scratch and
// KV cache append (src/metal_encode.m:129-153). Workgroup g covers one head
// (g/16 of 48: 32 q, 8 k, 8 v) and the four RoPE pairs (i, i+64) for
// i = 4*(g%16) .. +3. grid (768, count), block 192 (one chunk per wave).
template <bool LUT>
__global__ void __launch_bounds__(192)
k_qkv_rope(const uint8_t* __restrict__ Wqkv, float3 scales, const float* __restrict__ gamma,
    const float* __restrict__ xin, const lh_step_params* __restrict__ params,
    float* __restrict__ qout, float* __restrict__ kcache, float* __restrict__ vcache,
    uint32_t capacity)
{
    __shared__ float Q[8][3];
    __shared__ float lds_ss[3];
    __shared__ float lut_s[LUT ? 256 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t head = blockIdx.x >> 4;
    const uint32_t i0 = (blockIdx.x & 15) * 4;
    const float scale = head < 32 ? scales.x : (head < 40 ? scales.y : scales.z);
    if constexpr (LUT) {
        fill_lut(lut_s);
    }
    const uint32_t col = wave * LH_CHUNK + lane * LH_LANE_COLS;
    float xs[16];
    load_x16(xin + (size_t)t * LH_HIDDEN + col, xs);
    WVec<K_FP8> wv[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const uint32_t row = head * 128 + i0 + (r & 3) + (r >= 4 ? 64 : 0);
        load_w<K_FP8>(wv[r], Wqkv, row, LH_HIDDEN, col);
    }
    rmsnorm_chunk_prologue<3>(xs, gamma, col, lds_ss, 3, LH_HIDDEN);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float w[16];
        decode16<K_FP8, LUT>(wv[r], scale, lut_s, w);
        float acc = wave_tree64(chain16(w, xs));
        if (lane == 0) {
            Q[r][wave] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        const uint32_t j = threadIdx.x;
        float lo = Q[j][0];
        lo = lo + Q[j][1];
        lo = lo + Q[j][2];
        float hi = Q[4 + j][0];
        hi = hi + Q[4 + j][1];
        hi = hi + Q[4 + j][2];
        const uint32_t i = i0 + j;
        const lh_token_params* tp = &params->tokens[t];
        const uint32_t position = params->length + t;
        if (head < 40) {
            // column i < 64 rotates with -x[i+64]; column i+64 with x[i].
            float out_lo = lo * tp->cosine[i] + (-hi) * tp->sine[i];
            float out_hi = hi * tp->cosine[i + 64] + lo * tp->sine[i + 64];
            if (head < 32) {
                out_lo = out_lo * tp->qfactor;
                out_hi = out_hi * tp->qfactor;
                float* qh = qout + (size_t)t * LH_QUERY + head * 128;
                qh[i] = out_lo;
                qh[i + 64] = out_hi;
            } else {
                float* kr = kcache + lh_kv_index(capacity, 0, head - 32, position);
                kr[i] = out_lo;
                kr[i + 64] = out_hi;
            }
        } else {
            float* vr = vcache + lh_kv_index(capacity, 0, head - 40, position);
            vr[i] = lo;
            vr[i + 64] = hi;
        }
    }
}

// Fused RMSNorm -> gate and up rows -> SiLU(gate)*up (src/metal_encode.m:162-171).
// grid (2304, count), block 192; workgroup g covers inner rows 4g..4g+3.
template <bool LUT>
__global__ void __launch_bounds__(192)
k_gateup_silu(const uint8_t* __restrict__ Wgate, const uint8_t* __restrict__ Wup, float2 scales,
    const float* __restrict__ gamma, const float* __restrict__ xin, float* __restrict__ gated)
{
    __shared__ float Q[8][3];
    __shared__ float lds_ss[3];
    __shared__ float lut_s[LUT ? 256 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t row0 = blockIdx.x * 4;
    if constexpr (LUT) {
        fill_lut(lut_s);
    }
    const uint32_t col = wave * LH_CHUNK + lane * LH_LANE_COLS;
    float xs[16];
    load_x16(xin + (size_t)t * LH_HIDDEN + col, xs);
    WVec<K_FP8> wv[8];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        load_w<K_FP8>(wv[r], Wgate, row0 + r, LH_HIDDEN, col);
        load_w<K_FP8>(wv[4 + r], Wup, row0 + r, LH_HIDDEN, col);
    }
    rmsnorm_chunk_prologue<3>(xs, gamma, col, lds_ss, 3, LH_HIDDEN);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float w[16];
        decode16<K_FP8, LUT>(wv[r], r < 4 ? scales.x : scales.y, lut_s, w);
        float acc = wave_tree64(chain16(w, xs));
        if (lane == 0) {
            Q[r][wave] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        const uint32_t j = threadIdx.x;
        float g = Q[j][0];
        g = g + Q[j][1];
        g = g + Q[j][2];
        float u = Q[4 + j][0];
        u = u + Q[4 + j][1];
        u = u + Q[4 + j][2];
        gated[(size_t)t * LH_INNER + row0 + j] = silu(g) * u;
    }
}

// Fused final RMSNorm -> tied BF16 head (src/metal_encode.m:204-210): the
// embedding stays BF16 in HBM and widens exactly in registers.
// grid (VOCAB/8), block 192.
__global__ void __launch_bounds__(192)
k_head(const uint16_t* __restrict__ E, const float* __restrict__ gamma,
    const float* __restrict__ xrow, float* __restrict__ logits)
{
    __shared__ float Q[8][3];
    __shared__ float lds_ss[3];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.x * 8;
    const uint32_t col = wave * LH_CHUNK + lane * LH_LANE_COLS;
    float xs[16];
    load_x16(xrow + col, xs);
    WVec<K_BF16> wv[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        load_w<K_BF16>(wv[r], E, row0 + r, LH_HIDDEN, col);
    }
    rmsnorm_chunk_prologue<3>(xs, gamma, col, lds_ss, 3, LH_HIDDEN);
#pragma unroll
    for (int r = 0; r < 8; r++) {
        float w[16];
        decode16<K_BF16, false>(wv[r], 1.0f, nullptr, w);
        float acc = wave_tree64(chain16(w, xs));
        if (lane == 0) {
            Q[r][wave] = acc;
        }
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        const uint32_t r = threadIdx.x;
        float v = Q[r][0];
        v = v + Q[r][1];
        v = v + Q[r][2];
        logits[row0 + r] = v;
    }
}

// Standalone canonical RMSNorm (tests and the multi-token MFMA path).
// grid (tokens), block 64*ceil(width/1024) up to 16 waves.
__global__ void __launch_bounds__(1024)
k_rmsnorm(const float* __restrict__ gamma, const float* __restrict__ x, float* __restrict__ out,
    uint32_t width)
{
    __shared__ float lds_ss[16];
    __shared__ float r_s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x;
    const uint32_t nch = (width + LH_CHUNK - 1) / LH_CHUNK;
    const float* row = x + (size_t)t * width;
    const uint32_t col = wave * LH_CHUNK + lane * LH_LANE_COLS;
    float acc = 0.0f;
    for (uint32_t j = 0; j < 16 && col + j < width; j++) {
        acc = __builtin_fmaf(row[col + j], row[col + j], acc);
    }
    acc = wave_tree64(acc);
    if (lane == 0) {
        lds_ss[wave] = acc;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = lds_ss[0];
        for (uint32_t c = 1; c < nch; c++) {
            ss = ss + lds_ss[c];
        }
        r_s = 1.0f / __builtin_sqrtf(ss / (float)width + 1e-5f);
    }
    __syncthreads();
    const float r = r_s;
    for (uint32_t c = threadIdx.x; c < width; c += blockDim.x) {
        out[(size_t)t * width + c] = gamma[c] * (row[c] * r);
    }
}

}  // namespace lh

using namespace lh;

// ---------------------------------------------------------------------------
// Launchers (C ABI, internal).

template <int KIND, bool LUT, bool VEC>
static int launch_matvec(const void* W, float scale, const float* x, float* y,
    const float* residual, uint32_t rows, uint32_t cols, uint32_t tokens, hipStream_t s)
{
    constexpr int NW = 4, R = 4;
    const uint32_t nch = (cols + LH_CHUNK - 1) / LH_CHUNK;
    const size_t lds = (R * nch + (LUT ? 256 : 0)) * sizeof(float);
    dim3 grid((rows + R - 1) / R, tokens);
    hipLaunchKernelGGL((k_matvec<KIND, LUT, VEC, NW, R>), grid, dim3(NW * 64), lds, s,
        W, scale, x, y, residual, rows, cols);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_matvec(int kind, int lookup, const void* W, float scale,
    const float* x, float* y, const float* residual, uint32_t rows, uint32_t cols,
    uint32_t tokens, hipStream_t s)
{
    if (!W || !x || !y || !rows || !cols || !tokens || tokens > 65535 || rows > 0x7fffffffu) {
        return -1;
    }
    const size_t esize = kind == K_FP8 ? 1 : (kind == K_BF16 ? 2 : 4);
    const bool vec = ((size_t)cols * esize) % 16 == 0 && ((uintptr_t)W % 16) == 0 &&
        ((uintptr_t)x % 16) == 0;
    if (kind == K_FP8) {
        if (lookup) {
            return vec ? launch_matvec<K_FP8, true, true>(W, scale, x, y, residual, rows, cols, tokens, s)
                       : launch_matvec<K_FP8, true, false>(W, scale, x, y, residual, rows, cols, tokens, s);
        }
        return vec ? launch_matvec<K_FP8, false, true>(W, scale, x, y, residual, rows, cols, tokens, s)
                   : launch_matvec<K_FP8, false, false>(W, scale, x, y, residual, rows, cols, tokens, s);
    }
    if (kind == K_BF16) {
        return vec ? launch_matvec<K_BF16, false, true>(W, 1.0f, x, y, residual, rows, cols, tokens, s)
                   : launch_matvec<K_BF16, false, false>(W, 1.0f, x, y, residual, rows, cols, tokens, s);
    }
    if (kind == K_F32) {
        return vec ? launch_matvec<K_F32, false, true>(W, 1.0f, x, y, residual, rows, cols, tokens, s)
                   : launch_matvec<K_F32, false, false>(W, 1.0f, x, y, residual, rows, cols, tokens, s);
    }
    return -1;
}

extern "C" int lh_launch_qkv_rope(int lookup, const uint8_t* Wqkv, float sq, float sk, float sv,
    const float* gamma, const float* x, const lh_step_params* params, uint32_t count,
    float* q, float* kcache_layer, float* vcache_layer, uint32_t capacity, hipStream_t s)
{
    dim3 grid(48 * 16, count);
    float3 scales = make_float3(sq, sk, sv);
    if (lookup) {
        hipLaunchKernelGGL(k_qkv_rope<true>, grid, dim3(192), 0, s, Wqkv, scales, gamma, x, params,
            q, kcache_layer, vcache_layer, capacity);
    } else {
        hipLaunchKernelGGL(k_qkv_rope<false>, grid, dim3(192), 0, s, Wqkv, scales, gamma, x, params,
            q, kcache_layer, vcache_layer, capacity);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_gateup_silu(int lookup, const uint8_t* Wgate, const uint8_t* Wup,
    float sg, float su, const float* gamma, const float* x, uint32_t count, float* gated,
    hipStream_t s)
{
    dim3 grid(LH_INNER / 4, count);
    float2 scales = make_float2(sg, su);
    if (lookup) {
        hipLaunchKernelGGL(k_gateup_silu<true>, grid, dim3(192), 0, s, Wgate, Wup, scales, gamma, x, gated);
    } else {
        hipLaunchKernelGGL(k_gateup_silu<false>, grid, dim3(192), 0, s, Wgate, Wup, scales, gamma, x, gated);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_head(const uint16_t* E, const float* gamma, const float* xrow,
    float* logits, hipStream_t s)
{
    hipLaunchKernelGGL(k_head, dim3(LH_VOCAB / 8), dim3(192), 0, s, E, gamma, xrow, logits);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_rmsnorm(const float* gamma, const float* x, float* out, uint32_t width,
    uint32_t tokens, hipStream_t s)
{
    if (!width || width > 16 * LH_CHUNK || !tokens) {
        return -1;
    }
    const uint32_t nch = (width + LH_CHUNK - 1) / LH_CHUNK;
    hipLaunchKernelGGL(k_rmsnorm, dim3(tokens), dim3(64 * nch), 0, s, gamma, x, out, width);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
