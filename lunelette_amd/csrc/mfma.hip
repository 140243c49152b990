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

namespace lh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NSPLIT = 3;                 // BF16 planes per activation
constexpr uint32_t BM = 128;              // tokens per workgroup tile (4 waves x 32)
constexpr uint32_t BK = 64;               // columns per main-loop step
constexpr uint32_t LDS_STRIDE = BK + 8;   // BF16 elements per LDS weight row
constexpr uint32_t MAX_N = 2 * LH_INNER;  // widest GEMM: gate|up

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

__device__ __forceinline__ void store_split(uint16_t* xs, size_t plane, size_t at, float v)
{
    uint16_t parts[3];
    split3(v, parts);
    xs[at] = parts[0];
    xs[plane + at] = parts[1];
    xs[2 * plane + at] = parts[2];
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
        store_split(xs, plane, (size_t)t * width + c, v);
    }
}

// Down-projection input: SiLU(s_g * gate) * (s_u * up) (src/metal_encode.m:
// 162-171) from the gate|up GEMM partials P[s][m][0..18432) (gate rows first),
// summed in split order, split into BF16 planes. grid (count), block 256.
__global__ void __launch_bounds__(256)
k_split_silu(const float* __restrict__ partial, uint32_t splits, size_t split_stride,
    float2 scales, uint16_t* __restrict__ xs, uint32_t stride_tokens)
{
    const uint32_t t = blockIdx.x;
    const size_t plane = (size_t)stride_tokens * LH_INNER;
    const float* row = partial + (size_t)t * MAX_N;
    for (uint32_t i = threadIdx.x; i < LH_INNER; i += 256) {
        float g = row[i], u = row[LH_INNER + i];
        for (uint32_t s = 1; s < splits; s++) {
            g = g + row[s * split_stride + i];
            u = u + row[s * split_stride + LH_INNER + i];
        }
        store_split(xs, plane, (size_t)t * LH_INNER + i, silu(g * scales.x) * (u * scales.y));
    }
}

// q|k|v epilogue (src/metal_encode.m:129-153): partials P[s][m][0..6144)
// summed in split order, per-tensor scale, RoPE (column i < 64 rotates with
// -x[i+64], column i+64 with x[i]) and the query factor on Q; Q to qout, K and
// V appended to the cache at position length + m. grid (count), block 256.
__global__ void __launch_bounds__(256)
k_qkv_epilogue(const float* __restrict__ partial, uint32_t splits, size_t split_stride,
    float3 scales, const lh_step_params* __restrict__ params, float* __restrict__ qout,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t capacity)
{
    const uint32_t t = blockIdx.x;
    const float* row = partial + (size_t)t * LH_QKV_ROWS;
    const lh_token_params* tp = &params->tokens[t];
    const uint32_t position = params->length + t;
    for (uint32_t pair = threadIdx.x; pair < LH_QKV_ROWS / 2; pair += 256) {
        const uint32_t head = pair >> 6, i = pair & 63;
        const uint32_t n = head * 128 + i;
        float lo = row[n], hi = row[n + 64];
        for (uint32_t s = 1; s < splits; s++) {
            lo = lo + row[s * split_stride + n];
            hi = hi + row[s * split_stride + n + 64];
        }
        const float scale = head < 32 ? scales.x : (head < 40 ? scales.y : scales.z);
        lo = lo * scale;
        hi = hi * scale;
        if (head < 40) {
            const float out_lo = lo * tp->cosine[i] + (-hi) * tp->sine[i];
            const float out_hi = hi * tp->cosine[i + 64] + lo * tp->sine[i + 64];
            if (head < 32) {
                float* qh = qout + (size_t)t * LH_QUERY + head * 128;
                qh[i] = out_lo * tp->qfactor;
                qh[i + 64] = out_hi * tp->qfactor;
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

// x[m][n] = x[m][n] + scale * (((p0 + p1) + p2) + ...): deterministic split-K
// combine with the residual add (src/metal_encode.m:160,175); without the
// residual, x[m][n] = scale * (...). Partials P[s][m][n] with split stride
// stride_tokens * rows.
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

static int split_rows(const float* gamma, const float* x, uint16_t* xs, uint32_t width,
    uint32_t count, uint32_t stride, hipStream_t s)
{
    const uint32_t nch = (width + LH_CHUNK - 1) / LH_CHUNK;
    hipLaunchKernelGGL(k_split, dim3(count), dim3(64 * nch), 0, s, gamma, x, xs, width, stride);
    return launched_ok("split");
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
    const size_t n = (size_t)count * rows;
    hipLaunchKernelGGL(k_combine_residual, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
        partial, splits, rows, count, stride, scale, x, residual);
    return launched_ok("split-K combine");
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
    if (split_rows(NULL, d_x, ws->d_split, (uint32_t)cols, n, B, s) ||
        gemm<4>(d_w, NULL, (uint32_t)rows, (uint32_t)rows, (uint32_t)cols, ws->d_split, B, n,
            splits, ws->d_gemm, s)) {
        return -1;
    }
    return combine(ws->d_gemm, splits, (uint32_t)rows, n, B, scale, d_y, 0, s);
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
    float* P = ws->d_gemm;
    // q|k|v: 6144 rows in tiles of 96, 3072 columns.
    const uint32_t sq = splits_for(n, 4);
    if (split_rows(w->input_norm, d_x, ws->d_split, LH_HIDDEN, n, B, s) ||
        gemm<6>(w->qkv, NULL, LH_QKV_ROWS, LH_QKV_ROWS, LH_HIDDEN, ws->d_split, B, n, sq, P, s)) {
        return -1;
    }
    hipLaunchKernelGGL(k_qkv_epilogue, dim3(n), dim3(256), 0, s, P, sq,
        (size_t)B * LH_QKV_ROWS, make_float3(w->scale[0], w->scale[1], w->scale[2]),
        ws->d_params, ws->d_q, d_keys, d_values, C);
    // o: 3072 rows in tiles of 96, 4096 columns, residual.
    const uint32_t so = splits_for(n, 8);
    if (launched_ok("qkv epilogue") ||
        lh_launch_attention_mfma(ws->d_q, d_keys, d_values, ws->d_params, (uint32_t)ws->length,
            n, C, ws->d_PM, ws->d_PT, ws->d_PA, ws->d_attn, s) ||
        split_rows(NULL, ws->d_attn, ws->d_split, LH_QUERY, n, B, s) ||
        gemm<6>(w->o, NULL, LH_HIDDEN, LH_HIDDEN, LH_QUERY, ws->d_split, B, n, so, P, s) ||
        combine(P, so, LH_HIDDEN, n, B, w->scale[3], d_x, 1, s)) {
        return -1;
    }
    // gate|up: 18432 rows in tiles of 144, 3072 columns; SiLU(gate)*up in the
    // down projection's split.
    const uint32_t sg = splits_for(n, 2);
    if (split_rows(w->post_norm, d_x, ws->d_split, LH_HIDDEN, n, B, s) ||
        gemm<9>(w->gate, w->up, LH_INNER, MAX_N, LH_HIDDEN, ws->d_split, B, n, sg, P, s)) {
        return -1;
    }
    hipLaunchKernelGGL(k_split_silu, dim3(n), dim3(256), 0, s, P, sg, (size_t)B * MAX_N,
        make_float2(w->scale[4], w->scale[5]), ws->d_split, B);
    // down: 3072 rows in tiles of 96, 9216 columns, residual.
    const uint32_t sd = splits_for(n, 8);
    if (launched_ok("silu split") ||
        gemm<6>(w->down, NULL, LH_HIDDEN, LH_HIDDEN, LH_INNER, ws->d_split, B, n, sd, P, s) ||
        combine(P, sd, LH_HIDDEN, n, B, w->scale[6], d_x, 1, s)) {
        return -1;
    }
    return 0;
}
