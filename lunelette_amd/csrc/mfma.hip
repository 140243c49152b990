// Multi-token (chunked prefill) projections on the gfx950 matrix cores, the
// PREFILL_MPS path (replaces convert_fp8 + MPSMatrixMultiplication,
// src/metal_encode.m:94-110, src/metal_mps.m:26-111).
//
// C[m][n] = scale * sum_k X[m][k] * dec(W[n][k]).
// - W stays FP8 in HBM; each lane converts its 32 codes per 64-column step to
//   BF16 in registers (v_cvt_scalef32_pk_bf16_fp8 with unit scale is exact:
//   every E4M3FN value has at most 4 significant bits).
// - X (FP32 activations) is pre-split by k_split into hi + mid + lo BF16 so
//   that X == hi + mid + lo exactly; every MFMA product is exact in FP32 and
//   the three partial products accumulate in FP32.
// - One wave per workgroup computes two 32x32 output tiles with
//   v_mfma_f32_32x32x16_bf16 over the whole K range (no LDS, no barriers).
//   Lane l supplies A[m0 + l%32][k..k+8) and B[k..k+8)[n0 + l%32]; K is
//   permuted so lane half g = l/32 reads 32 contiguous columns per 64-column
//   step (one 32-byte weight load per tile).
// - Workgroup ids are mapped so the token tiles that share a weight slab run
//   on the same XCD (round-robin dispatch over 8 XCDs) and share its L2.
// - The scale is applied once in the epilogue (MFMA accumulation order is the
//   hardware's, so this path is tolerance-checked, not bit-mirrored).
#include "lh_device.h"
#include "lh_internal.h"
#include "lh_layer.h"

#include <stdlib.h>

namespace lh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NSPLIT = 3;
constexpr int TM = 32;   // tokens per tile
constexpr int TN = 32;   // weight rows per tile
constexpr int BK = 64;   // columns per main-loop step

// Exact split of x into hi + mid + lo BF16 (truncations; the residuals are
// exact in FP32 because each step removes the leading 8 significant bits).
__device__ __forceinline__ void split3(float x, uint16_t out[3])
{
    const uint32_t xb = __float_as_uint(x);
    const uint32_t hb = xb & 0xffff0000u;
    const float r1 = x - __uint_as_float(hb);
    const uint32_t mb = __float_as_uint(r1) & 0xffff0000u;
    const float r2 = r1 - __uint_as_float(mb);
    out[0] = (uint16_t)(hb >> 16);
    out[1] = (uint16_t)(mb >> 16);
    out[2] = (uint16_t)(__float_as_uint(r2) >> 16);
}

// xs[p][m][k] for p < 3 from FP32 rows, optionally RMS-normalized with the
// canonical schedule first (so the MFMA path sees the same normalized values
// as the decode path). grid (count), block 64*ceil(width/1024) (<= 16 waves).
__global__ void __launch_bounds__(1024)
k_split(const float* __restrict__ gamma, const float* __restrict__ x, uint16_t* __restrict__ xs,
    uint32_t width, uint32_t stride_tokens)
{
    __shared__ float lds_ss[16];
    __shared__ float r_s;
    const uint32_t t = blockIdx.x;
    const float* row = x + (size_t)t * width;
    float r = 1.0f;
    if (gamma) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const uint32_t nch = (width + LH_CHUNK - 1) / LH_CHUNK;
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
        r = r_s;
    }
    const size_t plane = (size_t)stride_tokens * width;
    for (uint32_t c = threadIdx.x; c < width; c += blockDim.x) {
        const float v = gamma ? gamma[c] * (row[c] * r) : row[c];
        uint16_t parts[3];
        split3(v, parts);
        const size_t at = (size_t)t * width + c;
        xs[at] = parts[0];
        xs[plane + at] = parts[1];
        xs[2 * plane + at] = parts[2];
    }
}

// Convert 8 FP8 codes (two dwords) to a BF16x8 B operand.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t lo, uint32_t hi)
{
    auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    auto c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    auto d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    bf16x8 out;
    out[0] = a[0]; out[1] = a[1]; out[2] = b[0]; out[3] = b[1];
    out[4] = c[0]; out[5] = c[1]; out[6] = d[0]; out[7] = d[1];
    return out;
}

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p)
{
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
    return __builtin_bit_cast(bf16x8, v);
}

// Accumulate two 32x32 tiles (weight rows w0[], w1[] start pointers of row
// n0 + l%32 of each tile) over columns [k_begin, k_end) for token tile m0.
__device__ __forceinline__ void mma_two_tiles(const uint8_t* w0, const uint8_t* w1,
    const uint16_t* xs, size_t plane, uint32_t K, uint32_t m, uint32_t k_begin, uint32_t k_end,
    floatx16& c0, floatx16& c1)
{
    const int lane = threadIdx.x & 63;
    const uint32_t g = lane >> 5;
    const uint16_t* xrow = xs + (size_t)m * K;
    for (uint32_t k0 = k_begin; k0 < k_end; k0 += BK) {
        const uint32_t kk = k0 + 32 * g;
        const u32x4 wa0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w0 + kk));
        const u32x4 wa1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w0 + kk + 16));
        const u32x4 wb0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w1 + kk));
        const u32x4 wb1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w1 + kk + 16));
        bf16x8 xa[NSPLIT][4];
#pragma unroll
        for (int p = 0; p < NSPLIT; p++) {
#pragma unroll
            for (int s = 0; s < 4; s++) {
                xa[p][s] = load_bf16x8(xrow + p * plane + kk + 8 * s);
            }
        }
        const bf16x8 ba[4] = {fp8x8_to_bf16(wa0.x, wa0.y), fp8x8_to_bf16(wa0.z, wa0.w),
                              fp8x8_to_bf16(wa1.x, wa1.y), fp8x8_to_bf16(wa1.z, wa1.w)};
        const bf16x8 bb[4] = {fp8x8_to_bf16(wb0.x, wb0.y), fp8x8_to_bf16(wb0.z, wb0.w),
                              fp8x8_to_bf16(wb1.x, wb1.y), fp8x8_to_bf16(wb1.z, wb1.w)};
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int p = NSPLIT - 1; p >= 0; p--) {
                c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[p][s], ba[s], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[p][s], bb[s], c1, 0, 0, 0);
            }
        }
    }
}

// Tile coordinates: workgroup b -> (row tile r, token tile t) with the token
// tiles of one row tile on the same XCD. rows_tiles must be a multiple of 8.
__device__ __forceinline__ void tile_of(uint32_t b, uint32_t token_tiles, uint32_t& r, uint32_t& t)
{
    const uint32_t xcd = b & 7u, q = b >> 3;
    t = q % token_tiles;
    r = (q / token_tiles) * 8u + xcd;
}

// Output row of accumulator element e for this lane (D layout of
// v_mfma_f32_32x32x16_bf16: row (e/4)*8 + (l/32)*4 + e%4, column l%32).
__device__ __forceinline__ uint32_t out_row(int e)
{
    const int lane = threadIdx.x & 63;
    return (uint32_t)((e >> 2) * 8 + (lane >> 5) * 4 + (e & 3));
}

// q|k|v with RoPE + query factor + KV append. Row tile r in [0, 96): head
// r/2, half-pair r%2 -> tiles rows head*128 + 32*(r%2) + [0,32) and +64.
__global__ void __launch_bounds__(64)
k_gemm_qkv_rope(const uint8_t* __restrict__ Wqkv, float3 scales, const uint16_t* __restrict__ xs,
    uint32_t count, uint32_t stride_tokens, const lh_step_params* __restrict__ params,
    float* __restrict__ qout, float* __restrict__ kcache, float* __restrict__ vcache,
    uint32_t capacity)
{
    const uint32_t token_tiles = (count + TM - 1) / TM;
    uint32_t r, t;
    tile_of(blockIdx.x, token_tiles, r, t);
    const int lane = threadIdx.x & 63;
    const uint32_t head = r >> 1;
    const uint32_t i0 = 32 * (r & 1);
    const uint32_t n_lo = head * 128 + i0 + (lane & 31);
    const uint8_t* w0 = Wqkv + (size_t)n_lo * LH_HIDDEN;
    const uint8_t* w1 = Wqkv + (size_t)(n_lo + 64) * LH_HIDDEN;
    floatx16 c0 = {}, c1 = {};
    const size_t plane = (size_t)stride_tokens * LH_HIDDEN;
    mma_two_tiles(w0, w1, xs, plane, LH_HIDDEN, t * TM + (lane & 31), 0, LH_HIDDEN, c0, c1);
    const float scale = head < 32 ? scales.x : (head < 40 ? scales.y : scales.z);
    const uint32_t i = i0 + (lane & 31);
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const uint32_t m = t * TM + out_row(e);
        if (m >= count) {
            continue;
        }
        const float lo = c0[e] * scale;
        const float hi = c1[e] * scale;
        const lh_token_params* tp = &params->tokens[m];
        const uint32_t position = params->length + m;
        if (head < 40) {
            float out_lo = lo * tp->cosine[i] + (-hi) * tp->sine[i];
            float out_hi = hi * tp->cosine[i + 64] + lo * tp->sine[i + 64];
            if (head < 32) {
                out_lo = out_lo * tp->qfactor;
                out_hi = out_hi * tp->qfactor;
                float* qh = qout + (size_t)m * LH_QUERY + head * 128;
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

// gate/up + SiLU*up. Row tile r in [0, 288): inner rows 32r + [0,32).
__global__ void __launch_bounds__(64)
k_gemm_gateup_silu(const uint8_t* __restrict__ Wgate, const uint8_t* __restrict__ Wup,
    float2 scales, const uint16_t* __restrict__ xs, uint32_t count, uint32_t stride_tokens,
    float* __restrict__ gated)
{
    const uint32_t token_tiles = (count + TM - 1) / TM;
    uint32_t r, t;
    tile_of(blockIdx.x, token_tiles, r, t);
    const int lane = threadIdx.x & 63;
    const uint32_t n = 32 * r + (lane & 31);
    floatx16 c0 = {}, c1 = {};
    const size_t plane = (size_t)stride_tokens * LH_HIDDEN;
    mma_two_tiles(Wgate + (size_t)n * LH_HIDDEN, Wup + (size_t)n * LH_HIDDEN, xs, plane, LH_HIDDEN,
        t * TM + (lane & 31), 0, LH_HIDDEN, c0, c1);
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const uint32_t m = t * TM + out_row(e);
        if (m < count) {
            const float g = c0[e] * scales.x;
            const float u = c1[e] * scales.y;
            gated[(size_t)m * LH_INNER + n] = silu(g) * u;
        }
    }
}

// Plain rows with split-K partials: row tile r in [0, rows/64) covers rows
// 64r + [0,32) and 64r + 32 + [0,32); split s of S covers K/S columns.
// partial[s][m][n] (unscaled).
__global__ void __launch_bounds__(64)
k_gemm_rows_partial(const uint8_t* __restrict__ W, uint32_t rows, uint32_t K,
    const uint16_t* __restrict__ xs, uint32_t count, uint32_t stride_tokens, uint32_t splits,
    float* __restrict__ partial)
{
    const uint32_t token_tiles = (count + TM - 1) / TM;
    const uint32_t per_split = rows / 64 * token_tiles;
    const uint32_t s = blockIdx.x / per_split;
    uint32_t r, t;
    tile_of(blockIdx.x % per_split, token_tiles, r, t);
    const int lane = threadIdx.x & 63;
    const uint32_t n = 64 * r + (lane & 31);
    floatx16 c0 = {}, c1 = {};
    const size_t plane = (size_t)stride_tokens * K;
    const uint32_t kspan = K / splits;
    mma_two_tiles(W + (size_t)n * K, W + (size_t)(n + 32) * K, xs, plane, K,
        t * TM + (lane & 31), s * kspan, (s + 1) * kspan, c0, c1);
    float* out = partial + (size_t)s * stride_tokens * rows;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const uint32_t m = t * TM + out_row(e);
        if (m < count) {
            out[(size_t)m * rows + n] = c0[e];
            out[(size_t)m * rows + n + 32] = c1[e];
        }
    }
}

// x[m][n] = x[m][n] + scale * (((p0 + p1) + p2) + ...): deterministic split-K
// combine with the residual add (src/metal_encode.m:160,175); without the
// residual, x[m][n] = scale * (...).
__global__ void k_combine_residual(const float* __restrict__ partial, uint32_t splits,
    uint32_t rows, uint32_t count, uint32_t stride_tokens, float scale, float* __restrict__ x,
    int residual)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)count * rows) {
        return;
    }
    float acc = partial[i];
    for (uint32_t s = 1; s < splits; s++) {
        acc = acc + partial[(size_t)s * stride_tokens * rows + i];
    }
    x[i] = residual ? x[i] + acc * scale : acc * scale;
}

}  // namespace lh

using namespace lh;

static int launched_ok(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        lh_set_error("%s launch failed: %s", what, hipGetErrorString(e));
        return -1;
    }
    return 0;
}

static uint32_t tiles_grid(uint32_t row_tiles, uint32_t count)
{
    return row_tiles * ((count + TM - 1) / TM);
}

// Token stride of the MFMA scratch: whole 32-token tiles, so every A-operand
// row a tile reads lies inside the split buffer.
static uint32_t padded_block(const lh_workspace* ws)
{
    return (uint32_t)((ws->block + TM - 1) / TM * TM);
}

extern "C" int lh_mfma_prepare(lh_workspace* ws)
{
    if (ws->d_split && ws->d_gemm) {
        return 0;
    }
    const size_t B = padded_block(ws);
    if (hipMalloc((void**)&ws->d_split, 3 * B * LH_INNER * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc((void**)&ws->d_gemm, 4 * B * LH_HIDDEN * sizeof(float)) != hipSuccess) {
        lh_set_error("MFMA workspace allocation failed");
        return -1;
    }
    ws->bytes += 3 * B * LH_INNER * sizeof(uint16_t) + 4 * B * LH_HIDDEN * sizeof(float);
    if (hipMemset(ws->d_split, 0, 3 * B * LH_INNER * sizeof(uint16_t)) != hipSuccess) {
        lh_set_error("MFMA workspace clear failed");
        return -1;
    }
    return 0;
}

static int split_rows(const float* gamma, const float* x, uint16_t* xs, uint32_t width,
    uint32_t count, uint32_t stride, hipStream_t s)
{
    const uint32_t nch = (width + LH_CHUNK - 1) / LH_CHUNK;
    hipLaunchKernelGGL(k_split, dim3(count), dim3(64 * nch), 0, s, gamma, x, xs, width, stride);
    return launched_ok("split");
}

static int rows_residual(const uint8_t* W, float scale, uint32_t rows, uint32_t K,
    const uint16_t* xs, uint32_t count, uint32_t stride, float* partial, float* x, hipStream_t s,
    int residual = 1)
{
    const uint32_t splits = K >= 8192 ? 4 : 2;
    const uint32_t grid = tiles_grid(rows / 64, count) * splits;
    hipLaunchKernelGGL(k_gemm_rows_partial, dim3(grid), dim3(64), 0, s, W, rows, K, xs, count,
        stride, splits, partial);
    if (launched_ok("gemm rows")) {
        return -1;
    }
    const size_t n = (size_t)count * rows;
    hipLaunchKernelGGL(k_combine_residual, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
        partial, splits, rows, count, stride, scale, x, residual);
    return launched_ok("split-K combine");
}

// Kernel-level MFMA projection y[t][r] = scale * sum_c dec(W[r][c]) x[t][c]
// (the block-projection seam, src/metal_encode.m:94-110): rows a multiple of
// 512 up to 3072, cols a multiple of 256 up to 9216, tokens <= the
// workspace block.
extern "C" int lh_fp8_gemm(lh_workspace* ws, const uint8_t* d_w, float scale, const float* d_x,
    float* d_y, size_t rows, size_t cols, size_t tokens, void* stream)
{
    if (!ws || !d_w || !d_x || !d_y || !rows || rows % 512 || rows > LH_HIDDEN || !cols ||
        cols % 256 || cols > LH_INNER || !tokens || tokens > ws->block) {
        lh_set_error("fp8_gemm: rows multiple of 512 (<= 3072), cols multiple of 256 (<= 9216), "
            "tokens <= workspace block");
        return -1;
    }
    if (lh_mfma_prepare(ws)) {
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    const uint32_t B = padded_block(ws);
    if (split_rows(NULL, d_x, ws->d_split, (uint32_t)cols, (uint32_t)tokens, B, s)) {
        return -1;
    }
    return rows_residual(d_w, scale, (uint32_t)rows, (uint32_t)cols, ws->d_split,
        (uint32_t)tokens, B, ws->d_gemm, d_y, s, 0);
}

extern "C" int lh_layer_forward_mfma(const lh_layer_weights* w, float* d_x, float* d_keys,
    float* d_values, lh_workspace* ws, hipStream_t s)
{
    if (!w->qkv || !w->o || !w->gate || !w->up || !w->down) {
        lh_set_error("MFMA path needs compact FP8 weights");
        return -1;
    }
    if (lh_mfma_prepare(ws)) {
        return -1;
    }
    const uint32_t n = (uint32_t)ws->count, C = (uint32_t)ws->capacity;
    const uint32_t B = padded_block(ws);
    if (split_rows(w->input_norm, d_x, ws->d_split, LH_HIDDEN, n, B, s)) {
        return -1;
    }
    hipLaunchKernelGGL(k_gemm_qkv_rope, dim3(tiles_grid(96, n)), dim3(64), 0, s, w->qkv,
        make_float3(w->scale[0], w->scale[1], w->scale[2]), ws->d_split, n, B, ws->d_params,
        ws->d_q, d_keys, d_values, C);
    if (launched_ok("gemm qkv") ||
        lh_launch_attention(ws->d_q, d_keys, d_values, ws->d_params, (uint32_t)ws->length, n,
            C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_attn, s) ||
        split_rows(NULL, ws->d_attn, ws->d_split, LH_QUERY, n, B, s) ||
        rows_residual(w->o, w->scale[3], LH_HIDDEN, LH_QUERY, ws->d_split, n, B, ws->d_gemm, d_x,
            s) ||
        split_rows(w->post_norm, d_x, ws->d_split, LH_HIDDEN, n, B, s)) {
        return -1;
    }
    hipLaunchKernelGGL(k_gemm_gateup_silu, dim3(tiles_grid(LH_INNER / 32, n)), dim3(64), 0, s,
        w->gate, w->up, make_float2(w->scale[4], w->scale[5]), ws->d_split, n, B, ws->d_gated);
    if (launched_ok("gemm gate/up") ||
        split_rows(NULL, ws->d_gated, ws->d_split, LH_INNER, n, B, s) ||
        rows_residual(w->down, w->scale[6], LH_HIDDEN, LH_INNER, ws->d_split, n, B, ws->d_gemm,
            d_x, s)) {
        return -1;
    }
    return 0;
}
