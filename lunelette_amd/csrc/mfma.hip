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
// - k_gemm: a 256-thread workgroup owns 128 tokens x 16*NF weight rows of one
//   K split. Each 64-column step, the workgroup converts its weight tile once
//   into a double-buffered BF16 LDS tile (row stride 72 BF16, so the 16 rows a
//   fragment load touches fall in different banks; the next step's tile is
//   fetched during this step's MFMAs), while each wave loads its 32 tokens'
//   activation planes straight into v_mfma_f32_16x16x32_bf16 operand
//   registers. Lane group g = lane/16 supplies columns 16g .. 16g+15 of the
//   step to both operands (a K permutation shared by A and B, so the sum is
//   unchanged) as two 8-column MFMA k-slices. Register use stays under 256 so
//   two workgroups share a CU and hide each other's loads, conversions and
//   barriers; the grids hold about 512 workgroups (split-K where N is small).
// - Workgroup ids map the (token tile, split) work of one weight tile onto one
//   XCD (dispatch is round-robin over the 8 XCDs), so the tile's second read
//   comes from that XCD's L2.
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
constexpr uint32_t BM = 128;              // tokens per workgroup tile (4 waves x 32)
constexpr uint32_t BK = 64;               // columns per main-loop step
constexpr uint32_t LDS_STRIDE = BK + 8;   // BF16 elements per LDS weight row
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

// Eight FP8 codes (two dwords) -> eight BF16 at out (16-byte aligned), exact.
__device__ __forceinline__ void fp8x8_to_bf16(uint32_t lo, uint32_t hi, uint16_t* out)
{
    const auto a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const auto b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const auto c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const auto d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    u32x4 v;
    v.x = __builtin_bit_cast(uint32_t, a);
    v.y = __builtin_bit_cast(uint32_t, b);
    v.z = __builtin_bit_cast(uint32_t, c);
    v.w = __builtin_bit_cast(uint32_t, d);
    *reinterpret_cast<u32x4*>(out) = v;
}

// grid: n_tiles * m_tiles * splits workgroups of 256 threads (n_tiles a
// multiple of 8), two resident per CU so one workgroup's loads, conversions
// and barriers overlap the other's MFMAs. W0 holds rows [0, boundary), W1 rows
// [boundary, N) (gate|up as two tensors); boundary is a multiple of 16*NF.
// out: P[s][m][n] with split stride stride_tokens * N; token rows >= count
// are not written.
template <int NF>
__global__ void __launch_bounds__(256, 2)
k_gemm(const uint8_t* __restrict__ W0, const uint8_t* __restrict__ W1, uint32_t boundary,
    uint32_t N, uint32_t K, const uint16_t* __restrict__ xs, uint32_t stride_tokens,
    uint32_t count, uint32_t m_tiles, uint32_t splits, float* __restrict__ out)
{
    constexpr uint32_t BN = 16 * NF;
    constexpr uint32_t CHUNKS = BN * (BK / 16);   // 16-code chunks per step
    constexpr uint32_t BCH = (CHUNKS + 255) / 256;
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDS_STRIDE];

    const uint32_t xcd = blockIdx.x & 7u, q = blockIdx.x >> 3;
    const uint32_t inner = m_tiles * splits;
    const uint32_t nt = (q / inner) * 8u + xcd;
    const uint32_t mt = (q % inner) % m_tiles, s = (q % inner) / m_tiles;
    const uint32_t kps = K / splits;
    const uint32_t k0 = s * kps, steps = kps / BK;
    const uint32_t n0 = nt * BN;
    const uint8_t* Wt = n0 < boundary ? W0 + (size_t)n0 * K : W1 + (size_t)(n0 - boundary) * K;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = lane >> 4, l16 = lane & 15;
    const uint32_t m_base = mt * BM + wave * 32;
    const size_t plane = (size_t)stride_tokens * K;
    const uint16_t* arow0 = xs + (size_t)(m_base + l16) * K + 16 * g + k0;
    const uint16_t* arow1 = arow0 + (size_t)16 * K;

    // Weight chunk c (row c/4, 16 codes at column 16*(c%4) of the step): the
    // loads are unconditional (threads past the tile reload its last chunk),
    // only the LDS store is predicated.
    const uint8_t* bsrc[BCH];
    uint32_t bdst[BCH];
    bool bown[BCH];
#pragma unroll
    for (uint32_t i = 0; i < BCH; i++) {
        const uint32_t c = tid + 256 * i;
        const uint32_t cc = c < CHUNKS ? c : CHUNKS - 1;
        bsrc[i] = Wt + (size_t)(cc >> 2) * K + 16 * (cc & 3) + k0;
        bdst[i] = (cc >> 2) * LDS_STRIDE + 16 * (cc & 3);
        bown[i] = c < CHUNKS;
    }
    u32x4 bw[BCH];
    auto load_b = [&](uint32_t dk) {
#pragma unroll
        for (uint32_t i = 0; i < BCH; i++) {
            bw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bsrc[i] + dk));
        }
    };
    auto store_b = [&](uint32_t stage) {
#pragma unroll
        for (uint32_t i = 0; i < BCH; i++) {
            if (bown[i]) {
                uint16_t* dst = &Bs[stage][bdst[i]];
                fp8x8_to_bf16(bw[i].x, bw[i].y, dst);
                fp8x8_to_bf16(bw[i].z, bw[i].w, dst + 8);
            }
        }
    };
    bf16x8 a[2][NSPLIT][2];
    auto load_a = [&](uint32_t dk) {
#pragma unroll
        for (int p = 0; p < NSPLIT; p++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                a[0][p][h] = __builtin_bit_cast(bf16x8,
                    *reinterpret_cast<const u32x4*>(arow0 + p * plane + dk + 8 * h));
                a[1][p][h] = __builtin_bit_cast(bf16x8,
                    *reinterpret_cast<const u32x4*>(arow1 + p * plane + dk + 8 * h));
            }
        }
    };
    floatx4 acc[2][NF];
#pragma unroll
    for (int mf = 0; mf < 2; mf++) {
#pragma unroll
        for (int nf = 0; nf < NF; nf++) {
            acc[mf][nf] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    load_b(0);
    store_b(0);
    __syncthreads();
    for (uint32_t step = 0; step < steps; step++) {
        const bool more = step + 1 < steps;
        load_a(step * BK);
        if (more) {
            load_b((step + 1) * BK);
        }
        const uint16_t* bs = &Bs[step & 1][l16 * LDS_STRIDE + 16 * g];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            bf16x8 b[NF];
#pragma unroll
            for (int nf = 0; nf < NF; nf++) {
                b[nf] = __builtin_bit_cast(bf16x8,
                    *reinterpret_cast<const u32x4*>(bs + nf * 16 * LDS_STRIDE + 8 * h));
            }
#pragma unroll
            for (int nf = 0; nf < NF; nf++) {
#pragma unroll
                for (int mf = 0; mf < 2; mf++) {
#pragma unroll
                    for (int p = NSPLIT - 1; p >= 0; p--) {
                        acc[mf][nf] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mf][p][h], b[nf],
                            acc[mf][nf], 0, 0, 0);
                    }
                }
            }
        }
        if (more) {
            store_b((step + 1) & 1);
        }
        __syncthreads();
    }
    // D layout of v_mfma_f32_16x16x32_bf16: lane l holds rows 4*(l/16) + r,
    // column l%16 of each 16x16 tile.
    float* o = out + (size_t)s * stride_tokens * N;
#pragma unroll
    for (int mf = 0; mf < 2; mf++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = m_base + 16 * mf + 4 * g + r;
            if (m < count) {
#pragma unroll
                for (int nf = 0; nf < NF; nf++) {
                    o[(size_t)m * N + n0 + 16 * nf + l16] = acc[mf][nf][r];
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
    return (uint32_t)((ws->block + BM - 1) / BM * BM);
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

// P[s][m][n] for n < N over `splits` equal K ranges. N / (16*NF) must be a
// multiple of 8, K a multiple of 64*splits, boundary a multiple of 16*NF.
template <int NF>
static int gemm(const uint8_t* W0, const uint8_t* W1, uint32_t boundary, uint32_t N, uint32_t K,
    const uint16_t* xs, uint32_t stride, uint32_t count, uint32_t splits, float* out,
    hipStream_t s)
{
    const uint32_t n_tiles = N / (16 * NF);
    const uint32_t m_tiles = (count + BM - 1) / BM;
    if (!count || N % (16 * NF) || n_tiles % 8 || K % (BK * splits) || boundary % (16 * NF) ||
        m_tiles * BM > stride || (size_t)splits * stride * N > partial_floats(stride)) {
        lh_set_error("gemm: unsupported shape N=%u K=%u splits=%u", N, K, splits);
        return -1;
    }
    hipLaunchKernelGGL(k_gemm<NF>, dim3(n_tiles * m_tiles * splits), dim3(256), 0, s, W0,
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

// K splits giving about 512 workgroups: `base` for two token tiles, twice as
// deep for one.
static uint32_t splits_for(uint32_t count, uint32_t base)
{
    return count > BM ? base : 2 * base;
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
    const uint32_t splits = splits_for(n, 1);
    if (split_rows(d_x, ws->d_split, (uint32_t)cols, n, B, s) ||
        gemm<4>(d_w, NULL, (uint32_t)rows, (uint32_t)rows, (uint32_t)cols, ws->d_split, B, n,
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
    // q|k|v: 6144 rows in tiles of 96, 3072 columns; scales, RoPE and the KV
    // append in the epilogue.
    const uint32_t sq = splits_for(n, 4);
    if ((!input_split &&
            residual_norm_split(NULL, 0, B, 1.0f, d_x, w->input_norm, xs, n, s)) ||
        gemm<6>(w->qkv, NULL, LH_QKV_ROWS, LH_QKV_ROWS, LH_HIDDEN, xs, B, n, sq, P, s) ||
        with_splits(sq, "qkv epilogue", [&](auto S) {
            hipLaunchKernelGGL(k_qkv_epilogue<decltype(S)::value>, dim3(n, 3), dim3(256), 0, s,
                P, (size_t)B * LH_QKV_ROWS, make_float3(w->scale[0], w->scale[1], w->scale[2]),
                ws->d_params, ws->d_q, d_keys, d_values, C);
        })) {
        return -1;
    }
    // Attention writes the o projection's input split; o: 3072 rows in tiles
    // of 96, 4096 columns; residual, post-norm and the gate|up split after it.
    const uint32_t so = splits_for(n, 8);
    if (lh_launch_attention_mfma(ws->d_q, d_keys, d_values, ws->d_params, (uint32_t)ws->length,
            n, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_attn, xs, B, s) ||
        launched_ok("attention") ||
        gemm<6>(w->o, NULL, LH_HIDDEN, LH_HIDDEN, LH_QUERY, xs, B, n, so, P, s) ||
        residual_norm_split(P, so, B, w->scale[3], d_x, w->post_norm, xs, n, s)) {
        return -1;
    }
    // gate|up: 18432 rows in tiles of 144, 3072 columns; SiLU(gate)*up in the
    // down projection's split.
    const uint32_t sg = splits_for(n, 2);
    if (gemm<9>(w->gate, w->up, LH_INNER, MAX_N, LH_HIDDEN, xs, B, n, sg, P, s) ||
        with_splits(sg, "silu split", [&](auto S) {
            hipLaunchKernelGGL(k_split_silu<decltype(S)::value>, dim3(n, 5), dim3(256), 0, s, P,
                (size_t)B * MAX_N, make_float2(w->scale[4], w->scale[5]), xs, B);
        })) {
        return -1;
    }
    // down: 3072 rows in tiles of 96, 9216 columns, residual (and the next
    // layer's input split).
    const uint32_t sd = splits_for(n, 8);
    if (gemm<6>(w->down, NULL, LH_HIDDEN, LH_HIDDEN, LH_INNER, xs, B, n, sd, P, s)) {
        return -1;
    }
    return next_norm ? residual_norm_split(P, sd, B, w->scale[6], d_x, next_norm, xs, n, s)
                     : combine(P, sd, LH_HIDDEN, n, B, w->scale[6], d_x, 1, s);
}
