// Multi-token (chunked prefill) projections on the gfx950 matrix cores, the
// PREFILL_MPS path (replaces convert_fp8 + MPSMatrixMultiplication,
// src/metal_encode.m:94-110, src/metal_mps.m:26-111).
//
// P[s][m][n] = sum over the split's columns k of X[m][k] * dec(W[n][k]), FP32.
// - X (FP32 activations) reaches the GEMM as planes of 16-bit values, in one
//   of two formats. Three BF16 planes: X == hi + mid + lo exactly (k_split,
//   the q|k|v input). Two FP16 planes of the row, or of a K range of it,
//   scaled by a power of two: X * 2^e == h + l to about 22 significant bits,
//   with 2^e bringing the range's largest magnitude into [2^14, 2^15) so
//   that nothing overflows (the o, gate|up and down inputs); the GEMM or the
//   consumer multiplies the products by 2^-e, exactly. W stays FP8 in HBM and is decoded exactly to
//   BF16 or FP16 (v_cvt_scalef32_pk_{bf16,f16}_fp8, unit scale: every E4M3FN
//   value has at most 4 significant bits and fits either type). The plane
//   products accumulate in FP32.
// - k_gemm_bf16 / k_gemm_f16: a 256-thread workgroup owns 64 tokens x 256
//   weight rows of one K split; each wave owns 64 weight rows and all 64
//   tokens (4 x 4 MFMA tiles). Per 64-column stage the activation tile (64 tokens x P planes,
//   8P KB) goes to LDS by direct loads (global_load_lds_dwordx4) in
//   fragment-major order, so each v_mfma_f32_16x16x32_{bf16,f16} A operand is
//   one conflict-free 16-byte LDS read, shared by the four waves; each wave
//   streams its weight rows straight into registers (16 FP8 codes per lane
//   and row fragment) and converts them there. The next stage's loads are
//   in flight (two LDS buffers, two weight register sets) while the current
//   stage's 32P MFMAs per wave run. Lane group g = lane/16 supplies columns
//   16g .. 16g+15 of the stage to both operands (a K permutation shared by
//   A and B, so the sum is unchanged) as two 8-column k-slices. Two
//   workgroups share a CU (<= 48 KB LDS and <= 256 registers each). Two FP16
//   planes do two thirds of the MFMA work of three BF16 planes (gate|up at
//   256 tokens: 85 against 104 us, the same error against an FP64 product).
//   Measured alternatives: weights through LDS as well (slower on gate|up,
//   equal elsewhere); a third stage in flight (spills at two workgroups per
//   CU); two BF16 planes (16 significant bits, outside the tolerance).
// - Workgroup ids deal the (weight tile, split) columns round-robin to the 8
//   XCDs and run a column's token tiles back to back on one XCD, so the
//   weight tile is read from HBM once per XCD and from L2 after that.
// - k_gemm_f16_stream (gate|up): the same stages over a stream-K partition.
//   The (256-row column, 64-column stage) units are dealt in equal
//   contiguous ranges to groups of one workgroup per token tile on one XCD,
//   two workgroups per CU, so every CU holds the same work: the 1152
//   split-K workgroups of gate|up at 256 tokens ran 2.25 rounds of 512 and
//   left most CUs idle in the last. A group writes a partial per column it
//   covers; k_split_silu sums each column's 2 or 3 in K order.
// - Scales and epilogues live in the consumers: k_qkv_epilogue (scales, RoPE,
//   query factor, KV append), k_split_silu (SiLU(gate)*up feeding the down
//   projection's split) and k_combine_residual (split-K sum in split order,
//   scale, residual). MFMA accumulation order is the hardware's, so this path
//   is tolerance-checked against the oracle, not bit-mirrored.
#include "lh_device.h"
#include "lh_internal.h"
#include "lh_layer.h"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>

namespace lh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t GM = 64;               // tokens per workgroup tile
constexpr uint32_t GN = 256;              // weight rows per workgroup tile (4 waves x 64)
constexpr uint32_t BK = 64;               // columns per pipeline stage
constexpr uint32_t SPLIT_ROWS = 128;      // token stride granule of the split planes
constexpr uint32_t MAX_N = 2 * LH_INNER;  // widest GEMM: gate|up

// Activation plane formats of the GEMM: three exact BF16 planes (hi + mid + lo),
// or two FP16 planes of a row scaled by 2^e (h + l, about 22 significant bits).
enum { PLANES_BF16 = 3, PLANES_F16 = 2 };

__device__ __forceinline__ float4 scale4(float4 v, float s)
{
    return make_float4(v.x * s, v.y * s, v.z * s, v.w * s);
}

__device__ __forceinline__ float absmax4(float4 v)
{
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Sum of S split-K partials in split order ((p0 + p1) + p2) + ..., all loads
// issued before the first add. p points at split 0; stride4 is the split
// stride in float4 units.
template <int S>
__device__ __forceinline__ float4 sum_splits(const float4* __restrict__ p, size_t stride4)
{
    float4 v[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        v[s] = p[s * stride4];
    }
    float4 acc = v[0];
#pragma unroll
    for (int s = 1; s < S; s++) {
        acc.x = acc.x + v[s].x;
        acc.y = acc.y + v[s].y;
        acc.z = acc.z + v[s].z;
        acc.w = acc.w + v[s].w;
    }
    return acc;
}

// sum_splits over the first n (1 <= n <= S) partials only, in the same
// order (n = S: bitwise sum_splits); the rest are neither loaded nor added.
template <int S>
__device__ __forceinline__ float4 sum_segments(const float4* __restrict__ p, size_t stride4,
    uint32_t n)
{
    float4 v[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        v[s] = s == 0 || (uint32_t)s < n ? p[s * stride4] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float4 acc = v[0];
#pragma unroll
    for (int s = 1; s < S; s++) {
        if ((uint32_t)s < n) {
            acc.x = acc.x + v[s].x;
            acc.y = acc.y + v[s].y;
            acc.z = acc.z + v[s].z;
            acc.w = acc.w + v[s].w;
        }
    }
    return acc;
}

// Stream-K partition of a product's (column, stage) units, column = 256
// weight rows, stage = 64 K columns, in column-major order: group g of
// `groups` takes units [begin(g), begin(g + 1)), equal to within one.
__host__ __device__ inline uint32_t stream_begin(uint32_t g, uint32_t units, uint32_t groups)
{
    return (uint32_t)((uint64_t)g * units / groups);
}

// The group whose range holds `unit`.
__host__ __device__ inline uint32_t stream_group(uint32_t unit, uint32_t units, uint32_t groups)
{
    return (uint32_t)((((uint64_t)unit + 1) * groups - 1) / units);
}

// Number of groups (partials) that cover column c of `stages` stages.
__host__ __device__ inline uint32_t stream_segments(uint32_t c, uint32_t stages, uint32_t units,
    uint32_t groups)
{
    return stream_group(c * stages + stages - 1, units, groups) -
        stream_group(c * stages, units, groups) + 1;
}

// Segments of column c (256 rows) of the down projection (3072 rows, 9216
// columns) over `groups` stream-K groups.
__device__ __forceinline__ uint32_t down_segments(uint32_t c, uint32_t groups)
{
    constexpr uint32_t STAGES = LH_INNER / BK, UNITS = LH_HIDDEN / GN * STAGES;
    return stream_segments(c, STAGES, UNITS, groups);
}

// xs[p][m][k] for p < 3 from FP32 rows, no normalization. grid (count,
// ceil(width / 2048)), block 256: thread j of the row takes columns
// 8j .. 8j+7 (width a multiple of 8, rows 16-byte aligned).
__global__ void __launch_bounds__(256)
k_split(const float* __restrict__ x, uint16_t* __restrict__ xs, uint32_t width,
    uint32_t stride_tokens)
{
    const uint32_t t = xs_token(blockIdx.x, gridDim.x), j = blockIdx.y * 256 + threadIdx.x;
    if (8 * j >= width) {
        return;
    }
    const float4* row = reinterpret_cast<const float4*>(x + (size_t)t * width);
    const float4 a = row[2 * j], b = row[2 * j + 1];
    const size_t plane = (size_t)stride_tokens * width;
    store_split4(xs, plane, xs_at(t, 8 * j, width), a);
    store_split4(xs, plane, xs_at(t, 8 * j + 4, width), b);
}

// One token row of 3072 per workgroup: with S > 0, the split-K residual
// combine x[t] = x[t] + scale * (((p0 + p1) + p2) + ...) (the o and down
// projections, src/metal_encode.m:160,175), written back; then the canonical
// RMSNorm of the (updated) row, y = gamma * (x * r) with ss by the row-dot
// schedule (w = x) and r = 1/sqrt(ss/n + 1e-5), the same normalized values the
// decode kernels compute, written as the next GEMM's input planes: with F16,
// scaled by the row's power of two 2^e and split into two FP16 planes, with
// out_scale[t] = 2^-e to undo it on the GEMM's output; otherwise the three
// exact BF16 planes (out_scale unused). The partials carry their own
// groups > 0: the partials are the down projection's stream-K partials of
// that many groups, each column summing only its segments. S = 0
// only normalizes (the first layer's input norm). grid (count), block 768:
// thread i owns columns 4i .. 4i+3.
template <int S, bool F16>
__global__ void __launch_bounds__(768)
k_residual_norm_split(const float* __restrict__ partial, size_t split_stride, float scale,
    float* __restrict__ x, const float* __restrict__ gamma,
    uint16_t* __restrict__ xs, float* __restrict__ out_scale, uint32_t stride_tokens,
    uint32_t groups)
{
    // Row in the [chunk][quad][lane] 16-byte-word layout: lane l's 16 values
    // of chunk c (columns c*1024 + 16l .. +15) are words (4c + q)*64 + l.
    __shared__ float4 row_l[LH_HIDDEN / 4];
    __shared__ float r_s;
    __shared__ float wmax[LH_HIDDEN / 4 / 64];
    const uint32_t t = xs_token(blockIdx.x, gridDim.x), tid = threadIdx.x;
    float4* xr = reinterpret_cast<float4*>(x + (size_t)t * LH_HIDDEN);
    const float4 g = reinterpret_cast<const float4*>(gamma)[tid];
    float4 v = xr[tid];
    if constexpr (S > 0) {
        const float4* pt = reinterpret_cast<const float4*>(partial + (size_t)t * LH_HIDDEN) + tid;
        const float4 acc = groups
            ? sum_segments<S>(pt, split_stride / 4, down_segments(tid / 64, groups))
            : sum_splits<S>(pt, split_stride / 4);
        v.x = v.x + acc.x * scale;
        v.y = v.y + acc.y * scale;
        v.z = v.z + acc.z * scale;
        v.w = v.w + acc.w * scale;
        xr[tid] = v;
    }
    const uint32_t c = tid >> 8, w = tid & 255;
    row_l[(4 * c + (w & 3)) * 64 + (w >> 2)] = v;
    __syncthreads();
    if (tid < 64) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < LH_HIDDEN / 256; k++) {
            const float4 u = row_l[k * 64 + tid];
            acc = __builtin_fmaf(u.x, u.x, acc);
            acc = __builtin_fmaf(u.y, u.y, acc);
            acc = __builtin_fmaf(u.z, u.z, acc);
            acc = __builtin_fmaf(u.w, u.w, acc);
        }
        const float ss = wave_tree64(acc);
        if (tid == 0) {
            r_s = 1.0f / __builtin_sqrtf(ss / (float)LH_HIDDEN + 1e-5f);
        }
    }
    __syncthreads();
    const float r = r_s;
    const float4 y = make_float4(g.x * (v.x * r), g.y * (v.y * r), g.z * (v.z * r), g.w * (v.w * r));
    if constexpr (!F16) {
        store_split4(xs, (size_t)stride_tokens * LH_HIDDEN, xs_at(t, 4 * tid, LH_HIDDEN), y);
        return;
    }
    const float m = wave_max64(absmax4(y));
    if ((tid & 63) == 0) {
        wmax[tid >> 6] = m;
    }
    __syncthreads();
    float mr = wmax[0];
#pragma unroll
    for (int i = 1; i < LH_HIDDEN / 4 / 64; i++) {
        mr = fmaxf(mr, wmax[i]);
    }
    const int e = row_exponent(mr);
    if (tid == 0) {
        out_scale[t] = exp2i(-e);
    }
    store_f16x2_4(xs, (size_t)stride_tokens * LH_HIDDEN, xs_at(t, 4 * tid, LH_HIDDEN),
        scale4(y, exp2i(e)));
}

// Down-projection input: SiLU(s_g * gate) * (s_u * up) (src/metal_encode.m:
// 162-171) from the gate|up GEMM partials P[s][m][0..18432) (gate rows first),
// summed in split order and multiplied by their row scale in_scale[t] (a power
// of two, exact). groups = 0: S equal K splits; otherwise the stream-K
// partials of `groups` groups (gemm_stream_tile), S >= every column's
// segment count. Each of the down projection's DOWN_SPLITS K ranges (576
// columns) gets its own power of two 2^e (its largest magnitude into
// [2^14, 2^15)) before the split into two FP16 planes; out_scale[t][g] = 2^-e,
// which the down projection's GEMM applies to that granule's products. grid
// (count, DOWN_SPLITS), block 192: thread j < 144 owns columns 576g + 4j .. +3.
constexpr uint32_t DOWN_SPLITS = 16;
constexpr uint32_t GROUP4 = LH_INNER / DOWN_SPLITS / 4;   // float4 columns per group: 144

template <int S>
__global__ void __launch_bounds__(192)
k_split_silu(const float* __restrict__ partial, size_t split_stride, float2 scales,
    const float* __restrict__ in_scale, uint16_t* __restrict__ xs,
    float* __restrict__ out_scale, uint32_t stride_tokens, uint32_t groups)
{
    __shared__ float wmax[3];
    const uint32_t t = xs_token(blockIdx.x, gridDim.x), grp = blockIdx.y, j = threadIdx.x;
    const bool active = j < GROUP4;
    // Idle lanes load (and discard) the group's last column: no branch around loads.
    const uint32_t c4 = grp * GROUP4 + (active ? j : GROUP4 - 1);
    const float4* row = reinterpret_cast<const float4*>(partial + (size_t)t * MAX_N) + c4;
    const size_t s4 = split_stride / 4;
    const float ts = in_scale[t], sg = scales.x, su = scales.y;
    // Segments of the gate column (c4 / 64) and of the up column 36 later.
    constexpr uint32_t STAGES = LH_HIDDEN / BK, UNITS = MAX_N / GN * STAGES;
    const uint32_t ng = groups ? stream_segments(c4 / 64, STAGES, UNITS, groups) : S;
    const uint32_t nu = groups ? stream_segments(c4 / 64 + LH_INNER / GN, STAGES, UNITS, groups) : S;
    const float4 g = scale4(sum_segments<S>(row, s4, ng), ts);
    const float4 u = scale4(sum_segments<S>(row + LH_INNER / 4, s4, nu), ts);
    const float4 y = make_float4(silu(g.x * sg) * (u.x * su), silu(g.y * sg) * (u.y * su),
        silu(g.z * sg) * (u.z * su), silu(g.w * sg) * (u.w * su));
    const float m = wave_max64(active ? absmax4(y) : 0.0f);
    if ((j & 63) == 0) {
        wmax[j >> 6] = m;
    }
    __syncthreads();
    const int e = row_exponent(fmaxf(wmax[0], fmaxf(wmax[1], wmax[2])));
    if (j == 0) {
        out_scale[t * DOWN_SPLITS + grp] = exp2i(-e);
    }
    if (active) {
        store_f16x2_4(xs, (size_t)stride_tokens * LH_INNER, xs_at(t, 4 * c4, LH_INNER),
            scale4(y, exp2i(e)));
    }
}

// q|k|v epilogue (src/metal_encode.m:129-153): partials P[s][m][0..6144)
// summed in split order, per-tensor scale, RoPE (column i < 64 rotates with
// -x[i+64], column i+64 with x[i]) and the query factor on Q; Q to qout, K and
// V appended to the cache at position length + m. grid (count, 3), block 256:
// thread j < 768 of the row takes pairs i0 .. i0+3 of head j/16, i0 = 4(j%16).
template <int S>
__global__ void __launch_bounds__(256)
k_qkv_epilogue(const float* __restrict__ partial, size_t split_stride, float3 scales,
    const lh_step_params* __restrict__ params, float* __restrict__ qout,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t capacity)
{
    const uint32_t t = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    const uint32_t head = j >> 4, i0 = (j & 15) * 4;
    const float4* row = reinterpret_cast<const float4*>(partial + (size_t)t * LH_QKV_ROWS);
    const size_t s4 = split_stride / 4;
    const uint32_t n4 = (head * 128 + i0) / 4;
    float4 lo = sum_splits<S>(row + n4, s4), hi = sum_splits<S>(row + n4 + 16, s4);
    const float scale = head < 32 ? scales.x : (head < 40 ? scales.y : scales.z);
    lo = make_float4(lo.x * scale, lo.y * scale, lo.z * scale, lo.w * scale);
    hi = make_float4(hi.x * scale, hi.y * scale, hi.z * scale, hi.w * scale);
    const uint32_t position = params->length + t;
    if (head >= 40) {
        float4* vr = reinterpret_cast<float4*>(vcache + lh_kv_index(capacity, 0, head - 40, position));
        vr[i0 / 4] = lo;
        vr[i0 / 4 + 16] = hi;
        return;
    }
    const lh_token_params* tp = &params->tokens[t];
    const float4 cl = *reinterpret_cast<const float4*>(tp->cosine + i0);
    const float4 ch = *reinterpret_cast<const float4*>(tp->cosine + i0 + 64);
    const float4 sl = *reinterpret_cast<const float4*>(tp->sine + i0);
    const float4 sh = *reinterpret_cast<const float4*>(tp->sine + i0 + 64);
    float4 out_lo, out_hi;
    out_lo.x = lo.x * cl.x + (-hi.x) * sl.x;
    out_lo.y = lo.y * cl.y + (-hi.y) * sl.y;
    out_lo.z = lo.z * cl.z + (-hi.z) * sl.z;
    out_lo.w = lo.w * cl.w + (-hi.w) * sl.w;
    out_hi.x = hi.x * ch.x + lo.x * sh.x;
    out_hi.y = hi.y * ch.y + lo.y * sh.y;
    out_hi.z = hi.z * ch.z + lo.z * sh.z;
    out_hi.w = hi.w * ch.w + lo.w * sh.w;
    if (head < 32) {
        const float f = tp->qfactor;
        float4* qh = reinterpret_cast<float4*>(qout + (size_t)t * LH_QUERY + head * 128);
        qh[i0 / 4] = make_float4(out_lo.x * f, out_lo.y * f, out_lo.z * f, out_lo.w * f);
        qh[i0 / 4 + 16] = make_float4(out_hi.x * f, out_hi.y * f, out_hi.z * f, out_hi.w * f);
    } else {
        *reinterpret_cast<float4*>(kcache + lh_k_index(capacity, 0, head - 32, position, i0)) =
            out_lo;
        *reinterpret_cast<float4*>(kcache + lh_k_index(capacity, 0, head - 32, position, i0 + 64)) =
            out_hi;
    }
}

// FP8 -> BF16 (or FP16) weight fragments, exact either way: the 16 codes of
// u (row bytes 16g .. 16g+15 of the step) give the two 8-column k-slices
// h = 0 (bytes 0..7) and h = 1.
__device__ __forceinline__ void fp8x16_to_bf16x8x2(u32x4 u, bf16x8& lo, bf16x8& hi)
{
    u32x4 a, b;
    a.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.x, 1.0f, false));
    a.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.x, 1.0f, true));
    a.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.y, 1.0f, false));
    a.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.y, 1.0f, true));
    b.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.z, 1.0f, false));
    b.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.z, 1.0f, true));
    b.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.w, 1.0f, false));
    b.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(u.w, 1.0f, true));
    lo = __builtin_bit_cast(bf16x8, a);
    hi = __builtin_bit_cast(bf16x8, b);
}

__device__ __forceinline__ void fp8x16_to_f16x8x2(u32x4 u, f16x8& lo, f16x8& hi)
{
    u32x4 a, b;
    a.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.x, 1.0f, false));
    a.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.x, 1.0f, true));
    a.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.y, 1.0f, false));
    a.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.y, 1.0f, true));
    b.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.z, 1.0f, false));
    b.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.z, 1.0f, true));
    b.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.w, 1.0f, false));
    b.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(u.w, 1.0f, true));
    lo = __builtin_bit_cast(f16x8, a);
    hi = __builtin_bit_cast(f16x8, b);
}

// One 64-column stage of a wave's 64 tokens x 16 NF weight rows: A fragments
// (mf, p, h) from the stage's LDS buffer, read one (p, h) group of four ahead
// of its MFMAs; each fragment feeds the NF weight fragments of w (this
// lane's 16 FP8 codes of rows 16 nf + lane % 16, columns 16 (lane / 16) ..
// +15 of the stage).
template <int P, int NF>
__device__ __forceinline__ void gemm_stage(const uint8_t* buf, const u32x4 (&w)[NF], uint32_t lane,
    floatx4 (&acc)[4][NF])
{
    using V = typename std::conditional<P == PLANES_BF16, bf16x8, f16x8>::type;
    V b[NF][2];
#pragma unroll
    for (int nf = 0; nf < NF; nf++) {
        if constexpr (P == PLANES_BF16) {
            fp8x16_to_bf16x8x2(w[nf], b[nf][0], b[nf][1]);
        } else {
            fp8x16_to_f16x8x2(w[nf], b[nf][0], b[nf][1]);
        }
    }
    V ac[4], an[4];
    // Groups j: k-slice h = j / P, planes from the smallest (p = P - 1) up.
    auto read_group = [&](int j, V (&dst)[4]) {
        const int h = j / P, p = (P - 1) - j % P;
#pragma unroll
        for (int mf = 0; mf < 4; mf++) {
            dst[mf] = __builtin_bit_cast(V, *reinterpret_cast<const u32x4*>(
                buf + ((mf * P + p) * 2 + h) * 1024 + 16 * lane));
        }
    };
    read_group(0, ac);
#pragma unroll
    for (int j = 0; j < 2 * P; j++) {
        // Wait for this group's reads (LDS only: s_waitcnt lgkmcnt(0) with
        // vmcnt and expcnt at their maxima, so the next stage's global loads
        // stay in flight) before the next group's are issued. The
        // compiler's own wait would come after them and wait for both.
        __builtin_amdgcn_s_waitcnt(0xc07f);
        if (j < 2 * P - 1) {
            read_group(j + 1, an);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mf = 0; mf < 4; mf++) {
#pragma unroll
            for (int nf = 0; nf < NF; nf++) {
                if constexpr (P == PLANES_BF16) {
                    acc[mf][nf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[mf],
                        b[nf][j / P], acc[mf][nf], 0, 0, 0);
                } else {
                    acc[mf][nf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ac[mf],
                        b[nf][j / P], acc[mf][nf], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mf = 0; mf < 4; mf++) {
            ac[mf] = an[mf];
        }
    }
}

template <int NF>
__device__ __forceinline__ void zero_tile(floatx4 (&acc)[4][NF])
{
#pragma unroll
    for (int mf = 0; mf < 4; mf++) {
#pragma unroll
        for (int nf = 0; nf < NF; nf++) {
            acc[mf][nf] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

// The wave's 64 x 64 tile into o[m][n0 + ..] for token rows m0.. < count.
// D layout of v_mfma_f32_16x16x32_{bf16,f16}: lane l holds rows 4*(l/16) + r,
// column l%16 of each 16x16 tile.
template <int NF>
__device__ __forceinline__ void store_tile(const floatx4 (&acc)[4][NF], float* __restrict__ o,
    uint32_t N, uint32_t m0, uint32_t n0, uint32_t count, uint32_t lane)
{
    const uint32_t g = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int mf = 0; mf < 4; mf++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = m0 + 16 * mf + 4 * g + r;
            if (m < count) {
#pragma unroll
                for (int nf = 0; nf < NF; nf++) {
                    o[(size_t)m * N + n0 + 16 * nf + l16] = acc[mf][nf][r];
                }
            }
        }
    }
}

// store_tile, or with add the tile added to what the same lanes stored there
// before (each element is read back only by the lane that wrote it).
template <int NF>
__device__ __forceinline__ void fold_tile(const floatx4 (&acc)[4][NF], float* __restrict__ o,
    uint32_t N, uint32_t m0, uint32_t n0, uint32_t count, uint32_t lane, bool add)
{
    if (!add) {
        store_tile<NF>(acc, o, N, m0, n0, count, lane);
        return;
    }
    const uint32_t g = lane >> 4, l16 = lane & 15;
#pragma unroll
    for (int mf = 0; mf < 4; mf++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = m0 + 16 * mf + 4 * g + r;
            if (m < count) {
#pragma unroll
                for (int nf = 0; nf < NF; nf++) {
                    float* const e = o + (size_t)m * N + n0 + 16 * nf + l16;
                    *e = *e + acc[mf][nf][r];
                }
            }
        }
    }
}

// P activation planes (PLANES_BF16 or PLANES_F16) of the same layout
// xs[p][m][k]. Each wave owns 16 NF weight rows, the workgroup 64 NF (256 or
// 192). grid: n_tiles * m_tiles * splits workgroups of 256 threads, two
// resident per CU; (n_tiles * splits) a multiple of 8. W0 holds rows
// [0, boundary), W1 rows [boundary, N) (gate|up as two tensors); boundary a
// multiple of 64 NF.
// out: P[s][m][n] with split stride stride_tokens * N; token rows >= count
// are not written (their activation rows, < m_tiles * 64 <= stride_tokens,
// are read).
//
// With gscale, the planes of token m's K split s carry the power of two
// 1/gscale[m][s] (row stride `splits`; the attention's output for the o
// projection): the split's products are multiplied by gscale[m][s] (exact)
// before the store, so the partials leave unscaled.
template <int P, int NF>
__device__ __forceinline__ void gemm_tile(const uint8_t* __restrict__ W0,
    const uint8_t* __restrict__ W1, uint32_t boundary, uint32_t N, uint32_t K,
    const uint16_t* __restrict__ xs, uint32_t stride_tokens, uint32_t count, uint32_t m_tiles,
    uint32_t splits, const float* __restrict__ gscale, float* __restrict__ out)
{
    constexpr uint32_t WN = 16 * NF, TN = 4 * WN;   // weight rows per wave, per workgroup
    static_assert(P == PLANES_BF16 || P == PLANES_F16, "plane format");
    constexpr uint32_t A_FRAGS = 4 * P * 2;   // 1 KB activation fragments per stage
    constexpr uint32_t PW = A_FRAGS / 4;      // fragments each wave loads
    __shared__ __attribute__((aligned(1024))) uint8_t As0[A_FRAGS * 1024];
    __shared__ __attribute__((aligned(1024))) uint8_t As1[A_FRAGS * 1024];
    // (weight tile, split) columns are dealt round-robin to the 8 XCDs; each
    // XCD runs a column's token tiles back to back, so they share its
    // weight tile in L2.
    const uint32_t xcd = blockIdx.x & 7u, q = blockIdx.x >> 3;
    const uint32_t mt = q % m_tiles, col = (q / m_tiles) * 8u + xcd;
    const uint32_t s = col % splits, nt = col / splits;
    const uint32_t kps = K / splits, k0 = s * kps, steps = kps / BK;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = lane >> 4, l16 = lane & 15;
    const uint32_t m0 = mt * GM, n0 = nt * TN + wave * WN;
    const uint8_t* Wt = n0 < boundary ? W0 + (size_t)n0 * K : W1 + (size_t)(n0 - boundary) * K;
    const uint8_t* wrow = Wt + (size_t)l16 * K + k0 + 16 * g;
    const size_t plane = (size_t)stride_tokens * K;
    // This wave's PW A fragments of each stage: f = PW*wave + i,
    // f = (mf*P + p)*2 + h.
    const uint16_t* asrc[PW];
#pragma unroll
    for (int i = 0; i < (int)PW; i++) {
        const uint32_t f = PW * wave + i, mf = f / (2 * P), p = (f / 2) % P, h = f % 2;
        asrc[i] = xs + p * plane + xs_at(m0 + 16 * mf, k0 + 8 * h, K) + 8 * lane;
    }
    // One contiguous 1 KiB fragment per load (xs_at): stage dk / 64 further
    // on is 1024 elements further on.
    auto load_a = [&](uint32_t dk, uint8_t* buf) {
#pragma unroll
        for (int i = 0; i < (int)PW; i++) {
            __builtin_amdgcn_global_load_lds(asrc[i] + (dk / BK) * 1024, buf + (PW * wave + i) * 1024,
                16, 0, 0);
        }
    };
    u32x4 wr[NF];
    auto load_w = [&](uint32_t dk) {
#pragma unroll
        for (int nf = 0; nf < NF; nf++) {
            wr[nf] = *reinterpret_cast<const u32x4*>(wrow + (size_t)16 * nf * K + dk);
        }
    };
    floatx4 acc[4][NF];
    zero_tile<NF>(acc);
    // Double-buffered stages: the next stage's activation (direct to LDS) and
    // weight loads are issued after the barrier that ends every read of the
    // LDS buffer they overwrite, and complete (s_waitcnt 0 + barrier) before
    // its MFMAs.
    u32x4 wc[NF];
    load_a(0, As0);
    load_w(0);
    for (uint32_t st = 0; st < steps; st += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int nf = 0; nf < NF; nf++) {
            wc[nf] = wr[nf];
        }
        if (st + 1 < steps) {
            load_a((st + 1) * BK, As1);
            load_w((st + 1) * BK);
        }
        gemm_stage<P, NF>(As0, wc, lane, acc);
        if (st + 1 >= steps) {
            break;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int nf = 0; nf < NF; nf++) {
            wc[nf] = wr[nf];
        }
        if (st + 2 < steps) {
            load_a((st + 2) * BK, As0);
            load_w((st + 2) * BK);
        }
        gemm_stage<P, NF>(As1, wc, lane, acc);
    }
    if (gscale) {
        // Rows past count read a stale factor and are not stored.
#pragma unroll
        for (int mf = 0; mf < 4; mf++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float f = gscale[(size_t)(m0 + 16 * mf + 4 * g + r) * splits + s];
#pragma unroll
                for (int nf = 0; nf < NF; nf++) {
                    acc[mf][nf][r] *= f;
                }
            }
        }
    }
    store_tile<NF>(acc, out + (size_t)s * stride_tokens * N, N, m0, n0, count, lane);
}

// gemm_tile over a stream-K partition: grid 8 * gpx * m_tiles workgroups of
// 256 threads (two resident per CU), `8 * gpx` groups of m_tiles workgroups,
// one per 64-token tile, on one XCD so that they share each weight tile in
// L2. A workgroup runs its group's units back to back, the next unit's loads
// in flight during the current one across column boundaries, and writes one
// partial per column it covers, into slot (group - first group of the
// column): P[slot][m][n], slot stride stride_tokens * N. A column's
// segments are its slots 0 .. stream_segments - 1, in K order; higher slots
// are not written for it. Every workgroup holds the same work to within one
// unit, so the launch has no partial last round.
//
// With gscale, the planes of token m's K granule j (K / GRANULES columns)
// carry the power of two 1/gscale[m][j] (k_split_silu): the accumulator is
// kept in units of the current granule's planes, multiplied by
// gscale[m][j] / gscale[m][j+1] where a segment crosses into the next
// granule and by gscale[m][j] before it is stored, so the partials are
// unscaled. The factors are powers of two (exact products); the workgroup's
// 64 x GRANULES factors are staged in LDS before the first stage.
// The accumulator holds at most about 2^38 in its granule's units (576
// products of a plane value below 2^15 and a weight below 2^9), so a ratio
// above 2^64 could overflow it (a granule whose largest value is more than
// 2^64 below its predecessor's, e.g. SiLU of very negative gates). Where a
// lane's rows meet such a ratio, its wave folds the unscaled accumulator into
// the column's partial in memory instead and restarts from zero; the column's
// last store then adds to what was folded (each lane re-reads only what it
// wrote itself).
constexpr float WIDE_RATIO = 0x1p64f;
constexpr uint32_t GRANULES = 16;
static_assert(GRANULES == DOWN_SPLITS, "the down input's scale granules");

template <int P>
__device__ __forceinline__ void gemm_stream_tile(const uint8_t* __restrict__ W0,
    const uint8_t* __restrict__ W1, uint32_t boundary, uint32_t N, uint32_t K,
    const uint16_t* __restrict__ xs, uint32_t stride_tokens, uint32_t count, uint32_t m_tiles,
    uint32_t gpx, const float* __restrict__ gscale, float* __restrict__ out)
{
    static_assert(P == PLANES_BF16 || P == PLANES_F16, "plane format");
    constexpr uint32_t A_FRAGS = 4 * P * 2;
    constexpr uint32_t PW = A_FRAGS / 4;
    __shared__ __attribute__((aligned(1024))) uint8_t As0[A_FRAGS * 1024];
    __shared__ __attribute__((aligned(1024))) uint8_t As1[A_FRAGS * 1024];
    __shared__ float4 gs[GM * GRANULES / 4];
    const uint32_t xcd = blockIdx.x & 7u, q = blockIdx.x >> 3;
    const uint32_t mt = q % m_tiles, groups = 8 * gpx, G = xcd * gpx + q / m_tiles;
    const uint32_t stages = K / BK, units = N / GN * stages, gstages = stages / GRANULES;
    const uint32_t u0 = stream_begin(G, units, groups), u1 = stream_begin(G + 1, units, groups);
    if (u0 >= u1) {
        return;
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = lane >> 4, l16 = lane & 15;
    const uint32_t m0 = mt * GM;
    if (gscale) {
        // Rows past count take 1 (their products are never stored).
        const float4 v = reinterpret_cast<const float4*>(gscale + (size_t)m0 * GRANULES)[tid];
        gs[tid] = m0 + tid / 4 < count ? v : make_float4(1.f, 1.f, 1.f, 1.f);
    }
    const size_t plane = (size_t)stride_tokens * K;
    const uint16_t* abase[PW];
#pragma unroll
    for (int i = 0; i < (int)PW; i++) {
        const uint32_t f = PW * wave + i, mf = f / (2 * P), p = (f / 2) % P, h = f % 2;
        abase[i] = xs + p * plane + xs_at(m0 + 16 * mf, 8 * h, K) + 8 * lane;
    }
    auto load_a = [&](uint32_t u, uint8_t* buf) {
        const uint32_t st = u % stages;
#pragma unroll
        for (int i = 0; i < (int)PW; i++) {
            __builtin_amdgcn_global_load_lds(abase[i] + st * 1024, buf + (PW * wave + i) * 1024, 16,
                0, 0);
        }
    };
    u32x4 wr[4];
    auto load_w = [&](uint32_t u) {
        const uint32_t nt = u / stages, n0 = nt * GN + wave * 64;
        const uint8_t* Wt = n0 < boundary ? W0 + (size_t)n0 * K : W1 + (size_t)(n0 - boundary) * K;
        const uint8_t* wrow = Wt + (size_t)l16 * K + (u - nt * stages) * BK + 16 * g;
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            wr[nf] = *reinterpret_cast<const u32x4*>(wrow + (size_t)16 * nf * K);
        }
    };
    floatx4 acc[4][4];
    zero_tile<4>(acc);
    // Whether this wave has folded part of the current column into memory.
    bool folded = false;
    // A column's partial leaves after its last stage or the range's last unit.
    auto finish = [&](uint32_t u) {
        const uint32_t nt = u / stages, st = u - nt * stages;
        const bool last = u + 1 == u1 || st + 1 == stages;
        float* const dst = out + (size_t)(G - stream_group(nt * stages, units, groups)) *
            stride_tokens * N;
        if (gscale && (last || (st + 1) % gstages == 0)) {
            const uint32_t j = st / gstages;
            const float* gf = reinterpret_cast<const float*>(gs);
            bool wide = false;
            if (!last) {
#pragma unroll
                for (int mf = 0; mf < 4; mf++) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float* row = gf + (16 * mf + 4 * g + r) * GRANULES;
                        wide = wide || row[j] > WIDE_RATIO * row[j + 1];
                    }
                }
                wide = __builtin_amdgcn_ballot_w64(wide) != 0;
            }
#pragma unroll
            for (int mf = 0; mf < 4; mf++) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float* row = gf + (16 * mf + 4 * g + r) * GRANULES;
                    const float f = last || wide ? row[j] : row[j] / row[j + 1];
#pragma unroll
                    for (int nf = 0; nf < 4; nf++) {
                        acc[mf][nf][r] *= f;
                    }
                }
            }
            if (wide) {
                fold_tile<4>(acc, dst, N, m0, nt * GN + wave * 64, count, lane, folded);
                folded = true;
                zero_tile<4>(acc);
            }
        }
        if (last) {
            fold_tile<4>(acc, dst, N, m0, nt * GN + wave * 64, count, lane, folded);
            folded = false;
            zero_tile<4>(acc);
        }
    };
    // The same double-buffered stages as gemm_tile, over units.
    u32x4 wc[4];
    load_a(u0, As0);
    load_w(u0);
    for (uint32_t u = u0; u < u1; u += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            wc[nf] = wr[nf];
        }
        if (u + 1 < u1) {
            load_a(u + 1, As1);
            load_w(u + 1);
        }
        gemm_stage<P, 4>(As0, wc, lane, acc);
        finish(u);
        if (u + 1 >= u1) {
            break;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            wc[nf] = wr[nf];
        }
        if (u + 2 < u1) {
            load_a(u + 2, As0);
            load_w(u + 2);
        }
        gemm_stage<P, 4>(As1, wc, lane, acc);
        finish(u + 1);
    }
}

// The two plane formats as kernels (a kernel template's host stub would have
// to instantiate the FP16 body on the host).
__global__ void __launch_bounds__(256, 2)
k_gemm_bf16(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1, uint32_t boundary,
    uint32_t N, uint32_t K, const uint16_t* __restrict__ xs, uint32_t stride_tokens,
    uint32_t count, uint32_t m_tiles, uint32_t splits, float* __restrict__ out)
{
    gemm_tile<PLANES_BF16, 4>(W0, W1, boundary, N, K, xs, stride_tokens, count, m_tiles, splits,
        nullptr, out);
}

// 192-row workgroup tiles (48 rows per wave): q|k|v at 4 K splits and o at
// 8 make 512 workgroups, every two-per-CU slot, where 256-row tiles leave a
// quarter of them empty.
__global__ void __launch_bounds__(256, 2)
k_gemm_bf16_n3(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1, uint32_t boundary,
    uint32_t N, uint32_t K, const uint16_t* __restrict__ xs, uint32_t stride_tokens,
    uint32_t count, uint32_t m_tiles, uint32_t splits, float* __restrict__ out)
{
    gemm_tile<PLANES_BF16, 3>(W0, W1, boundary, N, K, xs, stride_tokens, count, m_tiles, splits,
        nullptr, out);
}

__global__ void __launch_bounds__(256, 2)
k_gemm_f16(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1, uint32_t boundary,
    uint32_t N, uint32_t K, const uint16_t* __restrict__ xs, uint32_t stride_tokens,
    uint32_t count, uint32_t m_tiles, uint32_t splits, const float* __restrict__ gscale,
    float* __restrict__ out)
{
    gemm_tile<PLANES_F16, 4>(W0, W1, boundary, N, K, xs, stride_tokens, count, m_tiles, splits,
        gscale, out);
}

__global__ void __launch_bounds__(256, 2)
k_gemm_f16_n3(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1, uint32_t boundary,
    uint32_t N, uint32_t K, const uint16_t* __restrict__ xs, uint32_t stride_tokens,
    uint32_t count, uint32_t m_tiles, uint32_t splits, const float* __restrict__ gscale,
    float* __restrict__ out)
{
    gemm_tile<PLANES_F16, 3>(W0, W1, boundary, N, K, xs, stride_tokens, count, m_tiles, splits,
        gscale, out);
}

__global__ void __launch_bounds__(256, 2)
k_gemm_f16_stream(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1,
    uint32_t boundary, uint32_t N, uint32_t K, const uint16_t* __restrict__ xs,
    uint32_t stride_tokens, uint32_t count, uint32_t m_tiles, uint32_t gpx,
    const float* __restrict__ gscale, float* __restrict__ out)
{
    gemm_stream_tile<PLANES_F16>(W0, W1, boundary, N, K, xs, stride_tokens, count, m_tiles, gpx,
        gscale, out);
}

// x[i] = x[i] + scale * (((p0 + p1) + p2) + ...) (deterministic split-K
// combine with the residual add, src/metal_encode.m:160,175); without the
// residual, x[i] = scale * (...). Partials P[s][i] with split stride
// split_stride, or (groups > 0) the down projection's stream-K partials,
// each column's segments only; i runs over count * rows in float4 units
// (rows4 = rows / 4 per token). grid ceil(count * rows / 1024), block 256.
template <int S>
__global__ void __launch_bounds__(256)
k_combine_residual(const float* __restrict__ partial, size_t split_stride, size_t n4, float scale,
    uint32_t rows4, float* __restrict__ x, int residual, uint32_t groups)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) {
        return;
    }
    const float4* pi = reinterpret_cast<const float4*>(partial) + i;
    const float4 acc = groups
        ? sum_segments<S>(pi, split_stride / 4, down_segments((uint32_t)(i % rows4) / 64, groups))
        : sum_splits<S>(pi, split_stride / 4);
    float4* xr = reinterpret_cast<float4*>(x) + i;
    float4 v = make_float4(acc.x * scale, acc.y * scale, acc.z * scale, acc.w * scale);
    if (residual) {
        const float4 o = *xr;
        v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
    }
    *xr = v;
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

// Token stride of the MFMA scratch: whole 128-token tiles, so every
// activation row a tile reads lies inside the split buffer.
static uint32_t padded_block(const lh_workspace* ws)
{
    return (uint32_t)((ws->block + SPLIT_ROWS - 1) / SPLIT_ROWS * SPLIT_ROWS);
}

// Partial buffer: four 18432-wide splits per token (or more, narrower ones).
static size_t partial_floats(uint32_t B)
{
    return (size_t)4 * B * MAX_N;
}

// Bytes of the activation planes: three BF16 (or two FP16) planes of up to
// 9216 columns per token. The scales of the FP16 planes follow them: one per
// token for the gate|up input, DOWN_SPLITS per token for the down input (the
// same slots first hold the o input's eight per token, one per kv head).
static size_t plane_bytes(size_t B)
{
    return 3 * B * LH_INNER * sizeof(uint16_t);
}

static float* token_scales(const lh_workspace* ws)
{
    return reinterpret_cast<float*>(reinterpret_cast<char*>(ws->d_split) +
        plane_bytes(padded_block(ws)));
}

static float* group_scales(const lh_workspace* ws)
{
    return token_scales(ws) + padded_block(ws);
}

extern "C" int lh_mfma_prepare(lh_workspace* ws)
{
    if (ws->d_split && ws->d_gemm) {
        return 0;
    }
    const size_t B = padded_block(ws);
    const size_t split_bytes = plane_bytes(B) + (1 + DOWN_SPLITS) * B * sizeof(float);
    const size_t gemm_bytes = partial_floats((uint32_t)B) * sizeof(float);
    if (lh_dev_malloc((void**)&ws->d_split, split_bytes) != hipSuccess ||
        lh_dev_malloc((void**)&ws->d_gemm, gemm_bytes) != hipSuccess) {
        lh_set_error("MFMA workspace allocation failed");
        return -1;
    }
    ws->bytes += split_bytes + gemm_bytes;
    // Token rows past the executed count are read by the last tile (their
    // products are never stored); start them at zero.
    if (hipMemset(ws->d_split, 0, split_bytes) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        lh_set_error("MFMA workspace clear failed");
        return -1;
    }
    return 0;
}

// Calls f(std::integral_constant<int, S>) for the split count S, which the
// elementwise kernels take as a template argument so that every partial load
// issues before the first add. S = 0 (no partials) only where ZERO is set;
// counts above MAXS are rejected (and not instantiated).
template <bool ZERO = false, int MAXS = 16, typename F>
static int with_splits(uint32_t splits, const char* what, F&& f)
{
    switch (splits) {
    case 0:
        if constexpr (ZERO) {
            f(std::integral_constant<int, 0>{});
            break;
        }
        lh_set_error("%s: no partials", what);
        return -1;
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 8:
        if constexpr (MAXS >= 8) {
            f(std::integral_constant<int, 8>{});
            break;
        }
        lh_set_error("%s: unsupported split count %u", what, splits);
        return -1;
    case 16:
        if constexpr (MAXS >= 16) {
            f(std::integral_constant<int, 16>{});
            break;
        }
        lh_set_error("%s: unsupported split count %u", what, splits);
        return -1;
    default:
        lh_set_error("%s: unsupported split count %u", what, splits);
        return -1;
    }
    return launched_ok(what);
}

static int split_rows(const float* x, uint16_t* xs, uint32_t width, uint32_t count,
    uint32_t stride, hipStream_t s)
{
    hipLaunchKernelGGL(k_split, dim3(count, (width / 8 + 255) / 256), dim3(256), 0, s, x, xs,
        width, stride);
    return launched_ok("split");
}

// x = x + scale * sum of `splits` partials (groups > 0: the down projection's
// stream-K partials; 0 splits: x unchanged), then
// the RMSNorm of x with gamma as the next GEMM's input planes in xs: two FP16
// planes with their row scales in out_scale, or (out_scale NULL) three BF16
// planes; rows of 3072.
static int residual_norm_split(const float* partial, uint32_t splits, uint32_t stride,
    float scale, float* x, const float* gamma, uint16_t* xs, float* out_scale, uint32_t count,
    hipStream_t s, uint32_t groups = 0)
{
    return with_splits<true>(splits, "residual norm split", [&](auto S) {
        if (out_scale) {
            hipLaunchKernelGGL((k_residual_norm_split<decltype(S)::value, true>), dim3(count),
                dim3(768), 0, s, partial, (size_t)stride * LH_HIDDEN, scale, x, gamma, xs,
                out_scale, stride, groups);
        } else {
            hipLaunchKernelGGL((k_residual_norm_split<decltype(S)::value, false>), dim3(count),
                dim3(768), 0, s, partial, (size_t)stride * LH_HIDDEN, scale, x, gamma, xs,
                out_scale, stride, groups);
        }
    });
}

// P[s][m][n] for n < N over `splits` equal K ranges from `planes` activation
// planes (PLANES_BF16 or PLANES_F16). N and boundary multiples of 256, K a
// multiple of 64*splits, (N/256 * splits) a multiple of 8.
static int gemm(int planes, const uint8_t* W0, const uint8_t* W1, uint32_t boundary, uint32_t N,
    uint32_t K, const uint16_t* xs, uint32_t stride, uint32_t count, uint32_t splits, float* out,
    hipStream_t s, const float* gscale = nullptr, uint32_t nf = 4)
{
    const uint32_t tn = 64 * nf;   // weight rows per workgroup
    const uint32_t n_tiles = N / tn;
    const uint32_t m_tiles = (count + GM - 1) / GM;
    if (!count || !splits || (nf != 3 && nf != 4) || N % tn || (n_tiles * splits) % 8 ||
        K % (BK * splits) || boundary % tn || m_tiles * GM > stride ||
        (size_t)splits * stride * N > partial_floats(stride)) {
        lh_set_error("gemm: unsupported shape N=%u K=%u splits=%u", N, K, splits);
        return -1;
    }
    const dim3 grid(n_tiles * m_tiles * splits);
    if (planes == PLANES_BF16) {
        hipLaunchKernelGGL(nf == 4 ? k_gemm_bf16 : k_gemm_bf16_n3, grid, dim3(256), 0, s,
            W0, W1 ? W1 : W0, boundary, N, K, xs, stride, count, m_tiles, splits, out);
    } else {
        hipLaunchKernelGGL(nf == 4 ? k_gemm_f16 : k_gemm_f16_n3, grid, dim3(256), 0, s,
            W0, W1 ? W1 : W0, boundary, N, K, xs, stride, count, m_tiles, splits, gscale, out);
    }
    return launched_ok("gemm");
}

// The FP16-plane product over a stream-K partition (gemm_stream_tile): the
// most groups per XCD (<= 64 / m_tiles, two workgroups per CU) whose
// partials fit the partial buffer and the consumer's MAXS slots. Returns the
// slot count in *slots and the group count in *groups.
template <uint32_t MAXS>
static int gemm_stream(const uint8_t* W0, const uint8_t* W1, uint32_t boundary, uint32_t N,
    uint32_t K, const uint16_t* xs, uint32_t stride, uint32_t count, const float* gscale,
    float* out, uint32_t* slots, uint32_t* groups, hipStream_t s)
{
    const uint32_t n_tiles = N / GN;
    const uint32_t m_tiles = (count + GM - 1) / GM;
    if (!count || N % GN || K % BK || boundary % GN || m_tiles * GM > stride || m_tiles > 64 ||
        (gscale && K % (BK * GRANULES))) {
        lh_set_error("stream gemm: unsupported shape N=%u K=%u count=%u", N, K, count);
        return -1;
    }
    const uint32_t stages = K / BK, units = n_tiles * stages;
    for (uint32_t gpx = 64 / m_tiles; gpx > 0; gpx--) {
        const uint32_t ng = 8 * gpx;
        uint32_t most = 0;
        for (uint32_t c = 0; c < n_tiles; c++) {
            most = std::max(most, stream_segments(c, stages, units, ng));
        }
        if (most > MAXS || (size_t)most * stride * N > partial_floats(stride)) {
            continue;
        }
        hipLaunchKernelGGL(k_gemm_f16_stream, dim3(ng * m_tiles), dim3(256), 0, s, W0,
            W1 ? W1 : W0, boundary, N, K, xs, stride, count, m_tiles, gpx, gscale, out);
        *slots = most;
        *groups = ng;
        return launched_ok("stream gemm");
    }
    lh_set_error("stream gemm: no partition fits N=%u K=%u count=%u", N, K, count);
    return -1;
}

static int combine(const float* partial, uint32_t splits, uint32_t rows, uint32_t count,
    uint32_t stride, float scale, float* x, int residual, hipStream_t s, uint32_t groups = 0)
{
    const size_t n4 = (size_t)count * rows / 4;
    return with_splits(splits, "split-K combine", [&](auto S) {
        hipLaunchKernelGGL(k_combine_residual<decltype(S)::value>,
            dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, partial,
            (size_t)stride * rows, n4, scale, rows / 4, x, residual, groups);
    });
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
    const uint32_t B = padded_block(ws), n = (uint32_t)tokens;
    // Deepest K split (<= 16) that divides the 64-column stages.
    const uint32_t stages = (uint32_t)cols / BK;
    const uint32_t splits = stages % 16 == 0 ? 16 : (stages % 8 == 0 ? 8 : 4);
    if (split_rows(d_x, ws->d_split, (uint32_t)cols, n, B, s) ||
        gemm(PLANES_BF16, d_w, NULL, (uint32_t)rows, (uint32_t)rows, (uint32_t)cols, ws->d_split,
            B, n, splits, ws->d_gemm, s)) {
        return -1;
    }
    return combine(ws->d_gemm, splits, (uint32_t)rows, n, B, scale, d_y, 0, s);
}

// One layer over ws->count tokens. input_split: ws->d_split already holds the
// BF16 planes of input_norm(x) (the previous layer's last kernel wrote them);
// next_norm: the last kernel also writes them for the following layer (NULL:
// plain residual combine). The o, gate|up and down inputs travel as two
// FP16 planes with power-of-two scales (per token and kv head for o, per
// token for gate|up, per token and 576-column K granule for down). The q|k|v
// input stays in three exact BF16 planes: its error reaches the attention
// scores, which the softmax amplifies (at scores of a few hundred, two FP16
// planes put the layer of 256 tokens after a 4096-token prefix at 1.2e-3 of
// the row maximum, over the 1e-3 tolerance).
extern "C" int lh_layer_forward_mfma(const lh_layer_weights* w, float* d_x, float* d_keys,
    float* d_values, lh_workspace* ws, int input_split, const float* next_norm, hipStream_t s)
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
    float* P = ws->d_gemm;
    uint16_t* xs = ws->d_split;
    float* scale_a = token_scales(ws);
    float* scale_b = group_scales(ws);
    // K splits (measured at 256 tokens): q|k|v 4, o 8, down 16; gate|up is
    // stream-K.
    // q|k|v: 6144 rows, 3072 columns; scales, RoPE and the KV append in the
    // epilogue.
    const uint32_t sq = 4;
    if ((!input_split &&
            residual_norm_split(NULL, 0, B, 1.0f, d_x, w->input_norm, xs, NULL, n, s)) ||
        gemm(PLANES_BF16, w->qkv, NULL, LH_QKV_ROWS, LH_QKV_ROWS, LH_HIDDEN, xs, B, n, sq, P, s,
            nullptr, 3) ||
        with_splits(sq, "qkv epilogue", [&](auto S) {
            hipLaunchKernelGGL(k_qkv_epilogue<decltype(S)::value>, dim3(n, 3), dim3(256), 0, s,
                P, (size_t)B * LH_QKV_ROWS, make_float3(w->scale[0], w->scale[1], w->scale[2]),
                ws->d_params, ws->d_q, d_keys, d_values, C);
        })) {
        return -1;
    }
    // Attention writes the o projection's input as two FP16 planes with a
    // power-of-two scale per (token, kv head): the kv head's four query heads
    // are one of o's eight 512-column K splits, whose products the GEMM
    // scales back. o: 3072 rows, 4096 columns; residual, post-norm and the
    // gate|up input after it.
    const uint32_t so = LH_KV_HEADS;
    if (lh_launch_attention_mfma(ws->d_q, d_keys, d_values, ws->d_params, (uint32_t)ws->length,
            n, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_attn, xs, B, scale_b, s) ||
        launched_ok("attention") ||
        gemm(PLANES_F16, w->o, NULL, LH_HIDDEN, LH_HIDDEN, LH_QUERY, xs, B, n, so, P, s,
            scale_b, 3) ||
        residual_norm_split(P, so, B, w->scale[3], d_x, w->post_norm, xs, scale_a, n, s)) {
        return -1;
    }
    // gate|up: 18432 rows, 3072 columns, stream-K (at 256 tokens 128 groups of
    // 27 stages, at most 3 partials per column); SiLU(gate)*up as the down
    // projection's input.
    uint32_t sg = 0, groups = 0;
    if (gemm_stream<4>(w->gate, w->up, LH_INNER, MAX_N, LH_HIDDEN, xs, B, n, NULL, P, &sg,
            &groups, s) ||
        with_splits<false, 4>(sg, "silu split", [&](auto S) {
            hipLaunchKernelGGL(k_split_silu<decltype(S)::value>, dim3(n, DOWN_SPLITS), dim3(192),
                0, s, P, (size_t)B * MAX_N, make_float2(w->scale[4], w->scale[5]), scale_a, xs,
                scale_b, B, groups);
        })) {
        return -1;
    }
    // down: 3072 rows, 9216 columns, stream-K (at 256 tokens 128 groups of
    // 13-14 stages, 11-12 partials per column) with the input's granule
    // scales applied in the GEMM; residual (and the next layer's input
    // planes).
    uint32_t sd = 0, dgroups = 0;
    if (gemm_stream<16>(w->down, NULL, LH_HIDDEN, LH_HIDDEN, LH_INNER, xs, B, n, scale_b, P, &sd,
            &dgroups, s)) {
        return -1;
    }
    // Segment counts vary by column: sum with the 16-slot kernels.
    sd = 16;
    return next_norm
        ? residual_norm_split(P, sd, B, w->scale[6], d_x, next_norm, xs, NULL, n, s, dgroups)
        : combine(P, sd, LH_HIDDEN, n, B, w->scale[6], d_x, 1, s, dgroups);
}
