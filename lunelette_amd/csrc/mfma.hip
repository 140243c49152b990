// Multi-token (chunked prefill) projections on the gfx950 matrix cores, the
// PREFILL_MPS path (replaces convert_fp8 + MPSMatrixMultiplication,
// src/metal_encode.m:94-110, src/metal_mps.m:26-111).
//
// P[s][m][n] = sum over the split's columns k of X[m][k] * dec(W[n][k]), FP32.
// - X (FP32 activations) is pre-split by k_split into hi + mid + lo BF16 planes
//   so that X == hi + mid + lo exactly; W stays FP8 in HBM and is decoded to
//   BF16 exactly (v_cvt_scalef32_pk_bf16_fp8, unit scale: every E4M3FN value
//   has at most 4 significant bits). Every MFMA product is exact; the three
//   plane products accumulate in FP32.
// - k_gemm: a 256-thread workgroup owns 64 tokens x 256 weight rows of one K
//   split; each wave owns 64 weight rows and all 64 tokens (4 x 4 MFMA
//   tiles). Per 64-column stage the activation tile (64 tokens x 3 planes,
//   24 KB) goes to LDS by direct loads (global_load_lds_dwordx4) in
//   fragment-major order, so each v_mfma_f32_16x16x32_bf16 A operand is one
//   conflict-free 16-byte LDS read, shared by the four waves; each wave
//   streams its weight rows straight into registers (16 FP8 codes per lane
//   and row fragment) and converts them there. The next stage's loads are
//   in flight (two LDS buffers, two weight register sets) while the current
//   stage's 96 MFMAs per wave run. Lane group g = lane/16 supplies columns
//   16g .. 16g+15 of the stage to both operands (a K permutation shared by
//   A and B, so the sum is unchanged) as two 8-column k-slices. Two
//   workgroups share a CU (48 KB LDS and <= 256 registers each). Measured
//   alternatives: weights through LDS as well (slower on gate|up, equal
//   elsewhere); a third stage in flight (spills at two workgroups per CU).
// - Workgroup ids deal the (weight tile, split) columns round-robin to the 8
//   XCDs and run a column's token tiles back to back on one XCD, so the
//   weight tile is read from HBM once per XCD and from L2 after that.
// - Scales and epilogues live in the consumers: k_qkv_epilogue (scales, RoPE,
//   query factor, KV append), k_split_silu (SiLU(gate)*up feeding the down
//   projection's split) and k_combine_residual (split-K sum in split order,
//   scale, residual). MFMA accumulation order is the hardware's, so this path
//   is tolerance-checked against the oracle, not bit-mirrored.
#include "lh_device.h"
#include "lh_internal.h"
#include "lh_layer.h"

#include <stdlib.h>

#include <type_traits>

namespace lh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NSPLIT = 3;                 // BF16 planes per activation
constexpr uint32_t GM = 64;               // tokens per workgroup tile
constexpr uint32_t GN = 256;              // weight rows per workgroup tile (4 waves x 64)
constexpr uint32_t BK = 64;               // columns per pipeline stage
constexpr uint32_t A_FRAGS = 4 * 3 * 2;   // 1 KB activation fragments per stage
constexpr uint32_t SPLIT_ROWS = 128;      // token stride granule of the split planes
constexpr uint32_t MAX_N = 2 * LH_INNER;  // widest GEMM: gate|up

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

// xs[p][m][k] for p < 3 from FP32 rows, no normalization. grid (count,
// ceil(width / 2048)), block 256: thread j of the row takes columns
// 8j .. 8j+7 (width a multiple of 8, rows 16-byte aligned).
__global__ void __launch_bounds__(256)
k_split(const float* __restrict__ x, uint16_t* __restrict__ xs, uint32_t width,
    uint32_t stride_tokens)
{
    const uint32_t t = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    if (8 * j >= width) {
        return;
    }
    const float4* row = reinterpret_cast<const float4*>(x + (size_t)t * width);
    const float4 a = row[2 * j], b = row[2 * j + 1];
    const size_t plane = (size_t)stride_tokens * width, at = (size_t)t * width + 8 * j;
    store_split4(xs, plane, at, a);
    store_split4(xs, plane, at + 4, b);
}

// One token row of 3072 per workgroup: with S > 0, the split-K residual
// combine x[t] = x[t] + scale * (((p0 + p1) + p2) + ...) (the o and down
// projections, src/metal_encode.m:160,175), written back; then the canonical
// RMSNorm of the (updated) row, y = gamma * (x * r) with ss by the row-dot
// schedule (w = x) and r = 1/sqrt(ss/n + 1e-5), the same normalized values the
// decode kernels compute, split into the hi/mid/lo planes of xs for the next
// GEMM. S = 0 only normalizes (the first layer's input norm). grid (count),
// block 768: thread i owns columns 4i .. 4i+3.
template <int S>
__global__ void __launch_bounds__(768)
k_residual_norm_split(const float* __restrict__ partial, size_t split_stride, float scale,
    float* __restrict__ x, const float* __restrict__ gamma, uint16_t* __restrict__ xs,
    uint32_t stride_tokens)
{
    // Row in the [chunk][quad][lane] 16-byte-word layout: lane l's 16 values
    // of chunk c (columns c*1024 + 16l .. +15) are words (4c + q)*64 + l.
    __shared__ float4 row_l[LH_HIDDEN / 4];
    __shared__ float r_s;
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    float4* xr = reinterpret_cast<float4*>(x + (size_t)t * LH_HIDDEN);
    const float4 g = reinterpret_cast<const float4*>(gamma)[tid];
    float4 v = xr[tid];
    if constexpr (S > 0) {
        const float4 acc = sum_splits<S>(
            reinterpret_cast<const float4*>(partial + (size_t)t * LH_HIDDEN) + tid,
            split_stride / 4);
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
    store_split4(xs, (size_t)stride_tokens * LH_HIDDEN, (size_t)t * LH_HIDDEN + 4 * tid,
        make_float4(g.x * (v.x * r), g.y * (v.y * r), g.z * (v.z * r), g.w * (v.w * r)));
}

// Down-projection input: SiLU(s_g * gate) * (s_u * up) (src/metal_encode.m:
// 162-171) from the gate|up GEMM partials P[s][m][0..18432) (gate rows first),
// summed in split order, split into BF16 planes. grid (count, 5), block 256:
// thread j < 1152 of the row takes inner columns 8j .. 8j+7.
template <int S>
__global__ void __launch_bounds__(256)
k_split_silu(const float* __restrict__ partial, size_t split_stride, float2 scales,
    uint16_t* __restrict__ xs, uint32_t stride_tokens)
{
    const uint32_t t = blockIdx.x, j = blockIdx.y * 256 + threadIdx.x;
    if (8 * j >= LH_INNER) {
        return;
    }
    const float4* row = reinterpret_cast<const float4*>(partial + (size_t)t * MAX_N) + 2 * j;
    const size_t s4 = split_stride / 4;
    const float4 g0 = sum_splits<S>(row, s4), g1 = sum_splits<S>(row + 1, s4);
    const float4 u0 = sum_splits<S>(row + LH_INNER / 4, s4);
    const float4 u1 = sum_splits<S>(row + LH_INNER / 4 + 1, s4);
    const float sg = scales.x, su = scales.y;
    const size_t plane = (size_t)stride_tokens * LH_INNER, at = (size_t)t * LH_INNER + 8 * j;
    store_split4(xs, plane, at,
        make_float4(silu(g0.x * sg) * (u0.x * su), silu(g0.y * sg) * (u0.y * su),
            silu(g0.z * sg) * (u0.z * su), silu(g0.w * sg) * (u0.w * su)));
    store_split4(xs, plane, at + 4,
        make_float4(silu(g1.x * sg) * (u1.x * su), silu(g1.y * sg) * (u1.y * su),
            silu(g1.z * sg) * (u1.z * su), silu(g1.w * sg) * (u1.w * su)));
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
        float4* kr = reinterpret_cast<float4*>(kcache + lh_kv_index(capacity, 0, head - 32, position));
        kr[i0 / 4] = out_lo;
        kr[i0 / 4 + 16] = out_hi;
    }
}

// FP8 -> BF16 weight fragments: the 16 codes of u (row bytes 16g .. 16g+15
// of the step) give the two 8-column k-slices h = 0 (bytes 0..7) and h = 1.
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

// grid: n_tiles * m_tiles * splits workgroups of 256 threads, two resident per
// CU; (n_tiles * splits) a multiple of 8. W0 holds rows [0, boundary), W1
// rows [boundary, N) (gate|up as two tensors); boundary a multiple of 256.
// out: P[s][m][n] with split stride stride_tokens * N; token rows >= count
// are not written (their activation rows, < m_tiles * 64 <= stride_tokens,
// are read).
__global__ void __launch_bounds__(256, 2)
k_gemm(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1, uint32_t boundary,
    uint32_t N, uint32_t K, const uint16_t* __restrict__ xs, uint32_t stride_tokens,
    uint32_t count, uint32_t m_tiles, uint32_t splits, float* __restrict__ out)
{
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
    const uint32_t m0 = mt * GM, n0 = nt * GN + wave * 64;
    const uint8_t* Wt = n0 < boundary ? W0 + (size_t)n0 * K : W1 + (size_t)(n0 - boundary) * K;
    const uint8_t* wrow = Wt + (size_t)l16 * K + k0 + 16 * g;
    const size_t plane = (size_t)stride_tokens * K;
    // This wave's six A fragments of each stage: f = 6*wave + i, f = (mf*3 + p)*2 + h.
    const uint16_t* asrc[6];
#pragma unroll
    for (int i = 0; i < 6; i++) {
        const uint32_t f = 6 * wave + i, mf = f / 6, p = (f / 2) % 3, h = f % 2;
        asrc[i] = xs + p * plane + (size_t)(m0 + 16 * mf + l16) * K + k0 + 16 * g + 8 * h;
    }
    auto load_a = [&](uint32_t dk, uint8_t* buf) {
#pragma unroll
        for (int i = 0; i < 6; i++) {
            __builtin_amdgcn_global_load_lds(asrc[i] + dk, buf + (6 * wave + i) * 1024, 16, 0, 0);
        }
    };
    u32x4 wr[4];
    auto load_w = [&](uint32_t dk) {
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            wr[nf] = *reinterpret_cast<const u32x4*>(wrow + (size_t)16 * nf * K + dk);
        }
    };
    floatx4 acc[4][4];
#pragma unroll
    for (int mf = 0; mf < 4; mf++) {
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            acc[mf][nf] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    // One stage: A fragments (mf, p, h) read from LDS one (p, h) group of four
    // ahead of its MFMAs; each fragment feeds the four weight fragments.
    auto compute = [&](const uint8_t* buf, const u32x4 (&w)[4]) {
        bf16x8 b[4][2];
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            fp8x16_to_bf16x8x2(w[nf], b[nf][0], b[nf][1]);
        }
        bf16x8 ac[4], an[4];
        auto read_group = [&](int j, bf16x8 (&dst)[4]) {
            const int h = j / 3, p = 2 - j % 3;
#pragma unroll
            for (int mf = 0; mf < 4; mf++) {
                dst[mf] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                    buf + ((mf * 3 + p) * 2 + h) * 1024 + 16 * lane));
            }
        };
        read_group(0, ac);
#pragma unroll
        for (int j = 0; j < 6; j++) {
            if (j < 5) {
                read_group(j + 1, an);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mf = 0; mf < 4; mf++) {
#pragma unroll
                for (int nf = 0; nf < 4; nf++) {
                    acc[mf][nf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[mf], b[nf][j / 3],
                        acc[mf][nf], 0, 0, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mf = 0; mf < 4; mf++) {
                ac[mf] = an[mf];
            }
        }
    };
    // Double-buffered stages: the next stage's activation (direct to LDS) and
    // weight loads are issued after the barrier that ends every read of the
    // LDS buffer they overwrite, and complete (s_waitcnt 0 + barrier) before
    // its MFMAs.
    u32x4 wc[4];
    load_a(0, As0);
    load_w(0);
    for (uint32_t st = 0; st < steps; st += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            wc[nf] = wr[nf];
        }
        if (st + 1 < steps) {
            load_a((st + 1) * BK, As1);
            load_w((st + 1) * BK);
        }
        compute(As0, wc);
        if (st + 1 >= steps) {
            break;
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int nf = 0; nf < 4; nf++) {
            wc[nf] = wr[nf];
        }
        if (st + 2 < steps) {
            load_a((st + 2) * BK, As0);
            load_w((st + 2) * BK);
        }
        compute(As1, wc);
    }
    // D layout of v_mfma_f32_16x16x32_bf16: lane l holds rows 4*(l/16) + r,
    // column l%16 of each 16x16 tile.
    float* o = out + (size_t)s * stride_tokens * N;
#pragma unroll
    for (int mf = 0; mf < 4; mf++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = m0 + 16 * mf + 4 * g + r;
            if (m < count) {
#pragma unroll
                for (int nf = 0; nf < 4; nf++) {
                    o[(size_t)m * N + nt * GN + wave * 64 + 16 * nf + l16] = acc[mf][nf][r];
                }
            }
        }
    }
}

// x[i] = x[i] + scale * (((p0 + p1) + p2) + ...) (deterministic split-K
// combine with the residual add, src/metal_encode.m:160,175); without the
// residual, x[i] = scale * (...). Partials P[s][i] with split stride
// split_stride; i runs over count * rows in float4 units. grid
// ceil(count * rows / 1024), block 256.
template <int S>
__global__ void __launch_bounds__(256)
k_combine_residual(const float* __restrict__ partial, size_t split_stride, size_t n4, float scale,
    float* __restrict__ x, int residual)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) {
        return;
    }
    const float4 acc = sum_splits<S>(reinterpret_cast<const float4*>(partial) + i, split_stride / 4);
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

extern "C" int lh_mfma_prepare(lh_workspace* ws)
{
    if (ws->d_split && ws->d_gemm) {
        return 0;
    }
    const size_t B = padded_block(ws);
    const size_t split_bytes = 3 * B * LH_INNER * sizeof(uint16_t);
    const size_t gemm_bytes = partial_floats((uint32_t)B) * sizeof(float);
    if (hipMalloc((void**)&ws->d_split, split_bytes) != hipSuccess ||
        hipMalloc((void**)&ws->d_gemm, gemm_bytes) != hipSuccess) {
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
// issues before the first add. S = 0 (no partials) only where ZERO is set.
template <bool ZERO = false, typename F>
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
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 8: f(std::integral_constant<int, 8>{}); break;
    case 16: f(std::integral_constant<int, 16>{}); break;
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

// x = x + scale * sum of `splits` partials (0: x unchanged), then the RMSNorm
// of x with gamma split into xs; rows of 3072.
static int residual_norm_split(const float* partial, uint32_t splits, uint32_t stride,
    float scale, float* x, const float* gamma, uint16_t* xs, uint32_t count, hipStream_t s)
{
    return with_splits<true>(splits, "residual norm split", [&](auto S) {
        hipLaunchKernelGGL(k_residual_norm_split<decltype(S)::value>, dim3(count), dim3(768), 0, s,
            partial, (size_t)stride * LH_HIDDEN, scale, x, gamma, xs, stride);
    });
}

// P[s][m][n] for n < N over `splits` equal K ranges. N and boundary multiples
// of 256, K a multiple of 64*splits, (N/256 * splits) a multiple of 8.
static int gemm(const uint8_t* W0, const uint8_t* W1, uint32_t boundary, uint32_t N, uint32_t K,
    const uint16_t* xs, uint32_t stride, uint32_t count, uint32_t splits, float* out,
    hipStream_t s)
{
    const uint32_t n_tiles = N / GN;
    const uint32_t m_tiles = (count + GM - 1) / GM;
    if (!count || !splits || N % GN || (n_tiles * splits) % 8 || K % (BK * splits) ||
        boundary % GN || m_tiles * GM > stride ||
        (size_t)splits * stride * N > partial_floats(stride)) {
        lh_set_error("gemm: unsupported shape N=%u K=%u splits=%u", N, K, splits);
        return -1;
    }
    hipLaunchKernelGGL(k_gemm, dim3(n_tiles * m_tiles * splits), dim3(256), 0, s, W0,
        W1 ? W1 : W0, boundary, N, K, xs, stride, count, m_tiles, splits, out);
    return launched_ok("gemm");
}

static int combine(const float* partial, uint32_t splits, uint32_t rows, uint32_t count,
    uint32_t stride, float scale, float* x, int residual, hipStream_t s)
{
    const size_t n4 = (size_t)count * rows / 4;
    return with_splits(splits, "split-K combine", [&](auto S) {
        hipLaunchKernelGGL(k_combine_residual<decltype(S)::value>,
            dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, partial,
            (size_t)stride * rows, n4, scale, x, residual);
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
        gemm(d_w, NULL, (uint32_t)rows, (uint32_t)rows, (uint32_t)cols, ws->d_split, B, n,
            splits, ws->d_gemm, s)) {
        return -1;
    }
    return combine(ws->d_gemm, splits, (uint32_t)rows, n, B, scale, d_y, 0, s);
}

// One layer over ws->count tokens. input_split: ws->d_split already holds the
// BF16 split of input_norm(x) (the previous layer's last kernel wrote it);
// next_norm: the last kernel also writes the split of next_norm(x) for the
// following layer (NULL: plain residual combine).
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
    // K splits (measured at 256 tokens): gate|up 4 (the partial buffer's
    // limit), q|k|v 8, o 8, down 16.
    // q|k|v: 6144 rows, 3072 columns; scales, RoPE and the KV append in the
    // epilogue.
    const uint32_t sq = 8;
    if ((!input_split &&
            residual_norm_split(NULL, 0, B, 1.0f, d_x, w->input_norm, xs, n, s)) ||
        gemm(w->qkv, NULL, LH_QKV_ROWS, LH_QKV_ROWS, LH_HIDDEN, xs, B, n, sq, P, s) ||
        with_splits(sq, "qkv epilogue", [&](auto S) {
            hipLaunchKernelGGL(k_qkv_epilogue<decltype(S)::value>, dim3(n, 3), dim3(256), 0, s,
                P, (size_t)B * LH_QKV_ROWS, make_float3(w->scale[0], w->scale[1], w->scale[2]),
                ws->d_params, ws->d_q, d_keys, d_values, C);
        })) {
        return -1;
    }
    // Attention writes the o projection's input split; o: 3072 rows, 4096
    // columns; residual, post-norm and the gate|up split after it.
    const uint32_t so = 8;
    if (lh_launch_attention_mfma(ws->d_q, d_keys, d_values, ws->d_params, (uint32_t)ws->length,
            n, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_attn, xs, B, s) ||
        launched_ok("attention") ||
        gemm(w->o, NULL, LH_HIDDEN, LH_HIDDEN, LH_QUERY, xs, B, n, so, P, s) ||
        residual_norm_split(P, so, B, w->scale[3], d_x, w->post_norm, xs, n, s)) {
        return -1;
    }
    // gate|up: 18432 rows, 3072 columns; SiLU(gate)*up in the down
    // projection's split.
    const uint32_t sg = 4;
    if (gemm(w->gate, w->up, LH_INNER, MAX_N, LH_HIDDEN, xs, B, n, sg, P, s) ||
        with_splits(sg, "silu split", [&](auto S) {
            hipLaunchKernelGGL(k_split_silu<decltype(S)::value>, dim3(n, 5), dim3(256), 0, s, P,
                (size_t)B * MAX_N, make_float2(w->scale[4], w->scale[5]), xs, B);
        })) {
        return -1;
    }
    // down: 3072 rows, 9216 columns, residual (and the next layer's input
    // split).
    const uint32_t sd = 16;
    if (gemm(w->down, NULL, LH_HIDDEN, LH_HIDDEN, LH_INNER, xs, B, n, sd, P, s)) {
        return -1;
    }
    return next_norm ? residual_norm_split(P, sd, B, w->scale[6], d_x, next_norm, xs, n, s)
                     : combine(P, sd, LH_HIDDEN, n, B, w->scale[6], d_x, 1, s);
}
