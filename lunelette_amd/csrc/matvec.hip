// Decode / precise-path projections for gfx950. Every output row is a
// canonical row dot (lh_schedule.h): lane l of one wave owns columns
// [16l, 16l+16) of every 1024-column chunk, issues one 16-byte load per 16 FP8
// codes (32 B for BF16, 64 B for FP32) for all of its rows up front, decodes in
// registers with v_cvt_pk_f32_fp8, chains one fused multiply-add per element
// across all its chunks, and the 64 lane sums reduce by one fixed tree. The
// per-tensor scale multiplies the row total once.
//
// One wave owns whole rows. The workgroup stages the input row once in LDS;
// where a norm precedes the projection (q|k|v, gate/up, head) the workgroup
// applies the canonical RMSNorm there before any dot. The q|k|v and gate/up
// kernels split each output pair (RoPE halves, gate and up) over two waves
// and join the two dots through LDS.
#include "lh_attention_blocks.h"
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

// acc = fma(w_j, x_j, acc) for the lane's 16 columns in order; FP8 codes are
// decoded unscaled (exact), BF16 widened exactly, FP32 used as stored.
template <int KIND, bool LUT>
__device__ __forceinline__ float chain16(const WVec<KIND>& w, const float x[16], const float* lut,
    float acc)
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
                acc = __builtin_fmaf(d[j], x[4 * i + j], acc);
            }
        }
    } else if constexpr (KIND == K_BF16) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t words[4] = {w.v[i].x, w.v[i].y, w.v[i].z, w.v[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc = __builtin_fmaf(__uint_as_float(words[j] << 16), x[8 * i + 2 * j], acc);
                acc = __builtin_fmaf(__uint_as_float(words[j] & 0xffff0000u), x[8 * i + 2 * j + 1],
                    acc);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            acc = __builtin_fmaf(__uint_as_float(w.v[i].x), x[4 * i + 0], acc);
            acc = __builtin_fmaf(__uint_as_float(w.v[i].y), x[4 * i + 1], acc);
            acc = __builtin_fmaf(__uint_as_float(w.v[i].z), x[4 * i + 2], acc);
            acc = __builtin_fmaf(__uint_as_float(w.v[i].w), x[4 * i + 3], acc);
        }
    }
    return acc;
}

template <int KIND, bool LUT>
__device__ __forceinline__ float load_elem(const void* base, size_t index, const float* lut)
{
    if constexpr (KIND == K_FP8) {
        const uint32_t code = static_cast<const uint8_t*>(base)[index];
        if constexpr (LUT) {
            return lut[code];
        } else {
            float four[4];
            fp8x4_to_f32(code, four);
            return four[0];
        }
    } else if constexpr (KIND == K_BF16) {
        return __uint_as_float((uint32_t)static_cast<const uint16_t*>(base)[index] << 16);
    } else {
        return static_cast<const float*>(base)[index];
    }
}

__device__ __forceinline__ void load_x16(const float* x, float out[16])
{
    const float4* p = reinterpret_cast<const float4*>(x);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = p[i];
        out[4 * i + 0] = v.x;
        out[4 * i + 1] = v.y;
        out[4 * i + 2] = v.z;
        out[4 * i + 3] = v.w;
    }
}

// Unscaled E4M3FN table (the lookup strategy), filled from the arithmetic
// decode so both strategies agree bit for bit.
__device__ __forceinline__ void fill_lut(float* lut)
{
    for (uint32_t i = threadIdx.x; i < 256; i += blockDim.x) {
        float four[4];
        fp8x4_to_f32(i, four);
        lut[i] = four[0];
    }
}

// Workgroup-shared input row in LDS, laid out [chunk][quad][lane] as 16-byte
// words: lane l's 16 values of chunk c (columns c*1024 + 16l .. +15) are the
// words (4c + q)*64 + l, q = 0..3, so a wave reads a chunk with four
// conflict-free 16-byte loads. Staging is split around the weight loads:
// stage_load issues the row loads first, since vector loads retire in issue
// order; stage_commit writes LDS.
__device__ __forceinline__ uint32_t staged_word(int i, uint32_t tid)
{
    // float4 index tid + 256*i of the row is chunk i, lane tid/4, quad tid%4
    return (4 * i + (tid & 3)) * 64 + (tid >> 2);
}

template <int NCH>
__device__ __forceinline__ void stage_load(const float* row, float4 (&xv)[NCH])
{
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        xv[i] = reinterpret_cast<const float4*>(row)[tid + 256 * i];
    }
}

template <int NCH>
__device__ __forceinline__ void stage_commit(const float4 (&xv)[NCH], float4* xl)
{
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        xl[staged_word(i, tid)] = xv[i];
    }
    __syncthreads();
}

// Norm-prologue staging of a 3072-wide row for a T-thread workgroup. Thread
// tid loads the 8-byte units h = tid + T*u of the row and of gamma (unit h is
// columns 2h, 2h+1, half h&1 of 16-byte word h/2), so every thread count that
// divides 1536 needs no guards. norm_commit stores the units in the LDS layout
// above; wave 0 forms the canonical r from LDS; every thread then writes
// gamma * (x * r) over its own units. Three barriers; the last one publishes the
// normalized row (and anything else the workgroup stored before it).
template <int T>
__device__ __forceinline__ void norm_load(const float* row, const float* gamma,
    float2 (&xv)[1536 / T], float2 (&gv)[1536 / T])
{
    static_assert(1536 % T == 0, "thread count must divide the row's 8-byte units");
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < 1536 / T; u++) {
        xv[u] = reinterpret_cast<const float2*>(row)[tid + T * u];
        gv[u] = reinterpret_cast<const float2*>(gamma)[tid + T * u];
    }
}

__device__ __forceinline__ float2* staged_unit(float4* xl, uint32_t h)
{
    const uint32_t w = h >> 1;
    return reinterpret_cast<float2*>(xl + staged_word(w >> 8, w & 255)) + (h & 1);
}

template <int T>
__device__ __forceinline__ void norm_commit(const float2 (&xv)[1536 / T],
    const float2 (&gv)[1536 / T], float4* xl, float* r_s)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63;
#pragma unroll
    for (int u = 0; u < 1536 / T; u++) {
        *staged_unit(xl, tid + T * u) = xv[u];
    }
    __syncthreads();
    if ((tid >> 6) == 0) {
        float acc = 0.0f;
#pragma unroll 2
        for (int w = 0; w < 12; w++) {
            const float4 v = xl[w * 64 + lane];
            acc = __builtin_fmaf(v.x, v.x, acc);
            acc = __builtin_fmaf(v.y, v.y, acc);
            acc = __builtin_fmaf(v.z, v.z, acc);
            acc = __builtin_fmaf(v.w, v.w, acc);
        }
        const float ss = wave_lane0(wave_tree64(acc));
        if (lane == 0) {
            *r_s = 1.0f / __builtin_sqrtf(ss / (float)LH_HIDDEN + 1e-5f);
        }
    }
    __syncthreads();
    const float r = *r_s;
#pragma unroll
    for (int u = 0; u < 1536 / T; u++) {
        *staged_unit(xl, tid + T * u) = make_float2(gv[u].x * (xv[u].x * r), gv[u].y * (xv[u].y * r));
    }
    __syncthreads();
}

// Issue the lane's loads for R rows (row-major, NCH*1024 columns) before any
// other memory traffic of the wave, so weight latency overlaps the input-row
// loads and the RMSNorm prologue.
template <int KIND, int NCH, int R>
__device__ __forceinline__ void issue_rows(const void* W, const uint32_t (&rows)[R],
    WVec<KIND> (&wv)[R][NCH])
{
    const int lane = threadIdx.x & 63;
    constexpr uint32_t K = NCH * LH_CHUNK;
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            load_w<KIND>(wv[r][c], W, rows[r], K, c * LH_CHUNK + lane * LH_LANE_COLS);
        }
    }
}

// R canonical dots (unscaled) of the issued rows against the staged input
// row; lane 0 holds the wave totals. The R chains are interleaved element by
// element (each row's own order is unchanged) for instruction-level
// parallelism.
template <int KIND, bool LUT, int NCH, int R>
__device__ __forceinline__ void dot_rows(const WVec<KIND> (&wv)[R][NCH], const float4* xl,
    const float* lut, float (&out)[R])
{
    const uint32_t lane = threadIdx.x & 63;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        acc[r] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        float xs[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = xl[(c * 4 + q) * 64 + lane];
            xs[4 * q] = v.x;
            xs[4 * q + 1] = v.y;
            xs[4 * q + 2] = v.z;
            xs[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            acc[r] = chain16<KIND, LUT>(wv[r][c], xs, lut, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        out[r] = wave_tree64(acc[r]);
    }
}

// A wave's run of RW rows (rows[j], any order) with DEPTH rows of loads in
// flight: start() issues the first DEPTH rows; run() then, before each row's
// dot, issues the row DEPTH ahead into the slot the previous dot freed, and
// dots one row at a time in issue order. The compiler's waits follow issue
// order, so each dot starts as soon as its own row has landed, and after the
// last bytes arrive only one row's dot remains (where dot_rows over three rows
// at once waits for the last of the three). Scheduling barriers keep each
// row's loads between the dots around them: the scheduler otherwise hoists
// later rows' loads above a dot, which pushes that dot's waits back to
// vmcnt(0) and drains the wave's queue on every row.
template <int KIND, int NCH, int RW, int DEPTH>
struct RowStream {
    static constexpr int SLOTS = DEPTH + 1;
    WVec<KIND> wv[SLOTS][NCH];

    __device__ __forceinline__ void issue(const void* W, uint32_t row, int slot)
    {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            load_w<KIND>(wv[slot][c], W, row, NCH * LH_CHUNK, c * LH_CHUNK + lane * LH_LANE_COLS);
        }
    }

    __device__ __forceinline__ void start(const void* W, const uint32_t (&rows)[RW])
    {
#pragma unroll
        for (int j = 0; j < DEPTH && j < RW; j++) {
            issue(W, rows[j], j % SLOTS);
        }
    }

    // Unscaled canonical dots of the RW rows; lane 0 holds the totals.
    template <bool LUT>
    __device__ __forceinline__ void run(const void* W, const uint32_t (&rows)[RW],
        const float4* xl, const float* lut, float (&dots)[RW])
    {
#pragma unroll
        for (int j = 0; j < RW; j++) {
            if (j + DEPTH < RW) {
                issue(W, rows[j + DEPTH], (j + DEPTH) % SLOTS);
            }
            __builtin_amdgcn_sched_barrier(0);
            float d[1];
            dot_rows<KIND, LUT, NCH, 1>(
                *reinterpret_cast<const WVec<KIND>(*)[1][NCH]>(&wv[j % SLOTS]), xl, lut, d);
            dots[j] = d[0];
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// ---------------------------------------------------------------------------
// Model-shape row dots: y[t][row] = (RES ? residual[t][row] + : ) s * dot.
// Wave w of workgroup b owns rows R*(4b + w) .. +R. grid (rows/(4R), tokens).
template <int KIND, bool LUT, int NCH, int R, bool RES>
__global__ void __launch_bounds__(256)
k_rows(const void* __restrict__ W, float scale, const float* __restrict__ x, float* y,
    const float* residual, uint32_t rows)
{
    __shared__ float lut_s[LUT ? 256 : 1];
    __shared__ float4 xin_s[NCH * 4 * 64];
    if constexpr (LUT) {
        fill_lut(lut_s);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t row0 = (blockIdx.x * 4 + wave) * R;
    float4 xv[NCH];
    stage_load<NCH>(x + (size_t)t * NCH * LH_CHUNK, xv);
    uint32_t rr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        rr[r] = row0 + r;
    }
    // FP8 rows stream with one row of loads in flight ahead of the row being
    // dotted (RowStream); with all R rows requested at once the model's o
    // and down projections ran 6% and 8% slower. Other kinds keep every row
    // in flight.
    constexpr bool STREAM = KIND == K_FP8 && R > 1;
    RowStream<KIND, NCH, R, 1> stream;
    WVec<KIND> wv[STREAM ? 1 : R][NCH];
    if constexpr (STREAM) {
        stream.start(W, rr);
    } else {
        issue_rows<KIND, NCH, R>(W, rr, wv);
    }
    stage_commit<NCH>(xv, xin_s);
    // The epilogue's residual values are requested now, after the row is
    // staged, so they return behind the weights instead of costing a memory
    // round trip after the dots. Written as assembly because the compiler
    // sinks an ordinary load to its use. Loads complete in issue order, so
    // the compiler's own waits for the weights, which do not count these,
    // stay sufficient: for a row issued before them they wait longer, for a
    // row issued after them exactly. The values are read only after waiting
    // for all loads.
    float res[R];
    if constexpr (RES) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float* p = residual + (size_t)t * rows + row0 + r;
            asm volatile("global_load_dword %0, %1, off" : "=v"(res[r]) : "v"(p) : "memory");
        }
    }
    float dots[R];
    if constexpr (STREAM) {
        stream.template run<LUT>(W, rr, xin_s, lut_s, dots);
    } else {
        dot_rows<KIND, LUT, NCH, R>(wv, xin_s, lut_s, dots);
    }
    if constexpr (RES) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            asm volatile("s_waitcnt vmcnt(0)" : "+v"(res[r]) : : "memory");
        }
    }
    float out[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = dots[r] * scale;
        out[r] = RES ? res[r] + v : v;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            y[(size_t)t * rows + row0 + r] = out[r];
        }
    }
}

// Generic shapes (kernel-level ABI): one wave per row, chunks in a loop,
// vector loads where the lane's 16 columns are whole and aligned.
template <int KIND, bool LUT, bool VEC>
__global__ void __launch_bounds__(256)
k_rows_generic(const void* __restrict__ W, float scale, const float* __restrict__ x, float* y,
    const float* residual, uint32_t rows, uint32_t cols)
{
    __shared__ float lut_s[LUT ? 256 : 1];
    if constexpr (LUT) {
        fill_lut(lut_s);
        __syncthreads();
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.y;
    const uint32_t row = blockIdx.x * 4 + wave;
    if (row >= rows) {
        return;
    }
    const float* xt = x + (size_t)t * cols;
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < cols; c0 += LH_CHUNK) {
        const uint32_t col = c0 + lane * LH_LANE_COLS;
        const int valid = col >= cols ? 0 : (cols - col >= 16 ? 16 : (int)(cols - col));
        if (VEC && valid == 16) {
            float xs[16];
            load_x16(xt + col, xs);
            WVec<KIND> wv;
            load_w<KIND>(wv, W, row, cols, col);
            acc = chain16<KIND, LUT>(wv, xs, lut_s, acc);
        } else {
            for (int j = 0; j < valid; j++) {
                acc = __builtin_fmaf(load_elem<KIND, LUT>(W, (size_t)row * cols + col + j, lut_s),
                    xt[col + j], acc);
            }
        }
    }
    const float total = wave_tree64(acc);
    if (lane == 0) {
        const size_t o = (size_t)t * rows + row;
        const float v = total * scale;
        y[o] = residual ? residual[o] + v : v;
    }
}

// ---------------------------------------------------------------------------
// RMSNorm -> q|k|v -> RoPE (+ query factor on Q) -> Q scratch and KV append
// (src/metal_encode.m:129-153). The 48 heads (32 q, 8 k, 8 v) hold 64 RoPE
// pairs each, rows head*128 + i and + 64. A workgroup owns six pairs: waves 0
// and 1 dot the three lower rows (i) of pairs 3k .. 3k+2 of its six, waves 2
// and 3 the matching upper rows (i + 64), and the scaled dots meet in LDS,
// where threads 0..5 rotate one pair each. The row loads of all four waves
// are issued before any weight load (the first barrier), so the RMSNorm
// prologue is not queued behind weight misses.
template <bool LUT>
struct QkvShared {
    float lut[LUT ? 256 : 1];
    float4 xin[3 * 4 * 64];
    float prod[2][6];
    float r;
};

// Pair m of a workgroup's six: g * 6 + m in head order, or (BYKV) item
// g * 6 + m of kv head kvh's 384 pairs (its four query heads, then its key
// head, then its value head).
template <bool BYKV>
__device__ __forceinline__ uint32_t qkv_pair(uint32_t g, uint32_t kvh, uint32_t m)
{
    const uint32_t li = g * 6 + m;
    if constexpr (!BYKV) {
        return li;
    }
    return li < 256 ? kvh * 256 + li
        : li < 320 ? (32 + kvh) * 64 + (li - 256) : (40 + kvh) * 64 + (li - 320);
}

template <bool LUT, bool BYKV>
__device__ __forceinline__ void qkv_rope_body(const uint8_t* __restrict__ Wqkv, float3 scales,
    const float* __restrict__ gamma, const float* __restrict__ xin,
    const lh_step_params* __restrict__ params, float* __restrict__ qout,
    float* __restrict__ kcache, float* __restrict__ vcache, uint32_t capacity, uint32_t g,
    uint32_t kvh, uint32_t t, QkvShared<LUT>& sh)
{
    constexpr int T = 256;
    if constexpr (LUT) {
        fill_lut(sh.lut);  // published by the barriers below, before any dot
    }
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const bool upper = wave >= 2;
    const uint32_t k0 = 3 * (wave & 1);
    float2 xv[1536 / T], gv[1536 / T];
    norm_load<T>(xin + (size_t)t * LH_HIDDEN, gamma, xv, gv);
    __syncthreads();
    uint32_t rr[3];
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const uint32_t pair = qkv_pair<BYKV>(g, kvh, k0 + j);
        rr[j] = (pair >> 6) * 128 + (pair & 63) + (upper ? 64 : 0);
    }
    WVec<K_FP8> wv[3][3];
    issue_rows<K_FP8, 3, 3>(Wqkv, rr, wv);
    norm_commit<T>(xv, gv, sh.xin, &sh.r);
    float dots[3];
    dot_rows<K_FP8, LUT, 3, 3>(wv, sh.xin, sh.lut, dots);
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const uint32_t head = qkv_pair<BYKV>(g, kvh, k0 + j) >> 6;
            const float scale = head < 32 ? scales.x : (head < 40 ? scales.y : scales.z);
            sh.prod[upper][k0 + j] = dots[j] * scale;
        }
    }
    __syncthreads();
    if (tid < 6) {
        const lh_token_params* tp = &params->tokens[t];
        const uint32_t position = params->length + t;
        const uint32_t pair = qkv_pair<BYKV>(g, kvh, tid), head = pair >> 6, i = pair & 63;
        const float lo = sh.prod[0][tid];
        const float hi = sh.prod[1][tid];
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
                kcache[lh_k_index(capacity, 0, head - 32, position, i)] = out_lo;
                kcache[lh_k_index(capacity, 0, head - 32, position, i + 64)] = out_hi;
            }
        } else {
            float* vr = vcache + lh_kv_index(capacity, 0, head - 40, position);
            vr[i] = lo;
            vr[i + 64] = hi;
        }
    }
}

// grid (512, count), block 256: workgroup x owns pairs 6x .. 6x+5.
template <bool LUT>
__global__ void __launch_bounds__(256)
k_qkv_rope(const uint8_t* __restrict__ Wqkv, float3 scales, const float* __restrict__ gamma,
    const float* __restrict__ xin, const lh_step_params* __restrict__ params,
    float* __restrict__ qout, float* __restrict__ kcache, float* __restrict__ vcache,
    uint32_t capacity)
{
    __shared__ QkvShared<LUT> sh;
    qkv_rope_body<LUT, false>(Wqkv, scales, gamma, xin, params, qout, kcache, vcache, capacity,
        blockIdx.x, 0, blockIdx.y, sh);
}

// One decode token's q|k|v projection and attention blocks in one launch
// (src/metal_encode.m:129-153 then :154-160). Workgroups 0..511 are the q|k|v
// projection, workgroup j * 8 + kvh owning pairs 6j .. 6j+5 of kv head kvh;
// once its rows are stored (acknowledged by the L2) each stores its flag,
// flags[kvh * 64 + j] = (epoch, XCD), with a plain store: an atomic per
// workgroup on shared words costs microseconds, the flags nothing.
// Workgroups 512 + b * 8 + kvh are attention block b of kv head kvh:
// they load their K/V tiles while the projection streams its weights, wait
// for their kv head's 64 producers, then load q and the new row. Ids that
// agree mod 8 run on one XCD, so the producers' stores and the waiting blocks
// meet in that XCD's L2. The dispatcher starts a launch's workgroups in id
// order on each XCD, so every producer has started before any block waits.
// COMBINE: up to 16 blocks, the last block of each kv head combines;
// otherwise each block flags its partials in bflags and 128 combiner
// workgroups follow the blocks (id 512 + 8 * nblk + (4 * (h % 4) + qd) * 8 +
// h / 4, on kv head h / 4's XCD). epoch: nonzero, new for every launch on
// these flags; the blocks wait for producer flags of epoch `want` for at most
// `spins` polls, the combiners for block flags of epoch `cwant` for at most
// `cspins` (each equal to epoch and SPIN_LIMIT but where the test build forces
// that wait to give up). grid 512 + 8 * nblk (+ 128), block 256.
template <bool LUT, bool COMBINE>
__global__ void __launch_bounds__(256)
k_qkv_attn(const uint8_t* __restrict__ Wqkv, float3 scales, const float* __restrict__ gamma,
    const float* __restrict__ xin, const lh_step_params* __restrict__ params,
    float* __restrict__ qout, float* __restrict__ kcache, float* __restrict__ vcache,
    uint32_t capacity, uint32_t nblk, float* __restrict__ PM, float* __restrict__ PT,
    float* __restrict__ PA, unsigned long long* __restrict__ arrive,
    unsigned long long* flags, unsigned long long* bflags, unsigned long long epoch,
    unsigned long long want, uint32_t spins, unsigned long long cwant, uint32_t cspins,
    float* __restrict__ out)
{
    __shared__ union {
        QkvShared<LUT> qkv;
        AttnShared attn;
        CombineShared combine;
    } sh;
    const uint32_t kvh = blockIdx.x & 7;
    if (!COMBINE && blockIdx.x >= 8 * (QKV_PRODUCERS + nblk)) {
        const uint32_t r = (blockIdx.x - 8 * (QKV_PRODUCERS + nblk)) >> 3;
        attn_combiner(PM, PT, PA, params, capacity, bflags + kvh * (capacity / LH_ATTN_BLOCK),
            cwant, cspins, kvh * 4 + (r >> 2), r & 3, out, sh.combine);
        return;
    }
    if (blockIdx.x < 8 * QKV_PRODUCERS) {
        qkv_rope_body<LUT, true>(Wqkv, scales, gamma, xin, params, qout, kcache, vcache,
            capacity, blockIdx.x >> 3, kvh, 0, sh.qkv);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the rows are in L2
        __syncthreads();
        if (threadIdx.x == 0) {
            flags[kvh * QKV_PRODUCERS + (blockIdx.x >> 3)] = producer_flag(epoch, xcc_id());
        }
        return;
    }
    attn_block<COMBINE ? TAIL_COMBINE : TAIL_FLAG, true>(qout, kcache, vcache, params, capacity,
        nblk, PM, PT, PA, arrive, flags + kvh * QKV_PRODUCERS, bflags, epoch, want, spins, out,
        (blockIdx.x >> 3) - QKV_PRODUCERS, kvh, 0, sh.attn);
}

// RMSNorm -> gate and up rows -> SiLU(gate)*up (src/metal_encode.m:162-171).
// A workgroup of eight waves owns inner rows 36b .. 36b+35, so the model's
// 9216 rows fill the 256 CUs with one workgroup each and the input row is
// staged and normalized once per CU: waves 0..3 dot nine gate rows each,
// waves 4..7 the matching up rows, each as a RowStream with three rows in
// flight. The scaled dots meet in LDS, where threads 0..35 form
// SiLU(gate)*up. grid (9216/36, count), block 512.
constexpr int GATEUP_ROWS = 9;  // rows per wave
constexpr int GATEUP_DEPTH = 3; // rows of loads in flight per wave

template <bool LUT>
__global__ void __launch_bounds__(512)
k_gateup_silu(const uint8_t* __restrict__ Wgate, const uint8_t* __restrict__ Wup, float2 scales,
    const float* __restrict__ gamma, const float* __restrict__ xin, float* __restrict__ gated)
{
    constexpr int T = 512;
    constexpr int NR = 4 * GATEUP_ROWS;
    __shared__ float lut_s[LUT ? 256 : 1];
    __shared__ float4 xin_s[3 * 4 * 64];
    __shared__ float prod[2][NR];
    __shared__ float r_s;
    if constexpr (LUT) {
        fill_lut(lut_s);  // published by the norm's barriers, before any dot
    }
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const uint32_t t = blockIdx.y;
    const bool up = wave >= 4;
    const uint32_t k0 = GATEUP_ROWS * (wave & 3);
    const uint8_t* W = up ? Wup : Wgate;
    uint32_t rr[GATEUP_ROWS];
#pragma unroll
    for (int r = 0; r < GATEUP_ROWS; r++) {
        rr[r] = blockIdx.x * NR + k0 + r;
    }
    float2 xv[1536 / T], gv[1536 / T];
    norm_load<T>(xin + (size_t)t * LH_HIDDEN, gamma, xv, gv);
    RowStream<K_FP8, 3, GATEUP_ROWS, GATEUP_DEPTH> stream;
    stream.start(W, rr);
    norm_commit<T>(xv, gv, xin_s, &r_s);
    float dots[GATEUP_ROWS];
    stream.template run<LUT>(W, rr, xin_s, lut_s, dots);
    if (lane == 0) {
        const float scale = up ? scales.y : scales.x;
#pragma unroll
        for (int r = 0; r < GATEUP_ROWS; r++) {
            prod[up][k0 + r] = dots[r] * scale;
        }
    }
    __syncthreads();
    if (tid < NR) {
        gated[(size_t)t * LH_INNER + blockIdx.x * NR + tid] = silu(prod[0][tid]) * prod[1][tid];
    }
}

// Final RMSNorm -> tied BF16 head (src/metal_encode.m:204-210); the embedding
// stays BF16 in HBM and widens exactly in registers. Eight waves of four rows
// per workgroup share one staging of the row (the row loads are issued before
// any weight load). grid (VOCAB/32), block 512. With nonfinite set, a wave
// that writes an Inf or NaN logit stores 1 there (the caller clears it
// first), so the host need not scan every logit.
__global__ void __launch_bounds__(512)
k_head(const uint16_t* __restrict__ E, const float* __restrict__ gamma,
    const float* __restrict__ xrow, float* __restrict__ logits, uint32_t* __restrict__ nonfinite)
{
    constexpr int T = 512;
    __shared__ float4 xin_s[3 * 4 * 64];
    __shared__ float r_s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * 8 + wave) * 4;
    const uint32_t rr[4] = {row0, row0 + 1, row0 + 2, row0 + 3};
    float2 xv[1536 / T], gv[1536 / T];
    norm_load<T>(xrow, gamma, xv, gv);
    __syncthreads();
    WVec<K_BF16> wv[4][3];
    issue_rows<K_BF16, 3, 4>(E, rr, wv);
    norm_commit<T>(xv, gv, xin_s, &r_s);
    float dots[4];
    dot_rows<K_BF16, false, 3, 4>(wv, xin_s, nullptr, dots);
    if (lane == 0) {
        uint32_t bad = 0;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            logits[row0 + r] = dots[r];
            bad |= (__float_as_uint(dots[r]) & 0x7f800000u) == 0x7f800000u;
        }
        if (bad && nonfinite) {
            *nonfinite = 1u;
        }
    }
}

// Standalone canonical RMSNorm, one wave per token row (width <= 16384).
__global__ void __launch_bounds__(64)
k_rmsnorm(const float* __restrict__ gamma, const float* __restrict__ x, float* __restrict__ out,
    uint32_t width)
{
    const int lane = threadIdx.x & 63;
    const float* row = x + (size_t)blockIdx.x * width;
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < width; c0 += LH_CHUNK) {
        const uint32_t col = c0 + lane * LH_LANE_COLS;
        for (uint32_t j = 0; j < 16 && col + j < width; j++) {
            acc = __builtin_fmaf(row[col + j], row[col + j], acc);
        }
    }
    const float ss = wave_lane0(wave_tree64(acc));
    const float r = 1.0f / __builtin_sqrtf(ss / (float)width + 1e-5f);
    for (uint32_t c = lane; c < width; c += 64) {
        out[(size_t)blockIdx.x * width + c] = gamma[c] * (row[c] * r);
    }
}

}  // namespace lh

using namespace lh;

// ---------------------------------------------------------------------------
// Launchers (C ABI, internal).

template <int KIND, bool LUT, int NCH, int R>
static int launch_rows(const void* W, float scale, const float* x, float* y, const float* residual,
    uint32_t rows, uint32_t tokens, hipStream_t s)
{
    dim3 grid(rows / (4 * R), tokens);
    if (residual) {
        hipLaunchKernelGGL((k_rows<KIND, LUT, NCH, R, true>), grid, dim3(256), 0, s, W, scale, x,
            y, residual, rows);
    } else {
        hipLaunchKernelGGL((k_rows<KIND, LUT, NCH, R, false>), grid, dim3(256), 0, s, W, scale, x,
            y, residual, rows);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}


// Model shapes (3072, 4096 or 9216 columns) use the unrolled kernel. FP8 and
// BF16 weights take three rows per wave where the row count allows it (the
// model's 3072-row o and down projections then give each SIMD of the 256 CUs
// the same work); resident FP32 rows take fewer to fit the register file.
// Returns 1 when the shape is not a model shape.
template <int KIND, bool LUT>
static int launch_model_rows(const void* W, float scale, const float* x, float* y,
    const float* residual, uint32_t rows, uint32_t cols, uint32_t tokens, hipStream_t s)
{
    if constexpr (KIND != K_F32) {
        if (rows % 12 == 0) {
            if (cols == 3072) {
                return launch_rows<KIND, LUT, 3, 3>(W, scale, x, y, residual, rows, tokens, s);
            }
            if (cols == 4096) {
                return launch_rows<KIND, LUT, 4, 3>(W, scale, x, y, residual, rows, tokens, s);
            }
            if (cols == 9216) {
                return launch_rows<KIND, LUT, 9, 3>(W, scale, x, y, residual, rows, tokens, s);
            }
        }
    }
    if (cols == 3072 && rows % 8 == 0) {
        return launch_rows<KIND, LUT, 3, 2>(W, scale, x, y, residual, rows, tokens, s);
    }
    if (cols == 4096 && rows % 8 == 0) {
        return launch_rows<KIND, LUT, 4, 2>(W, scale, x, y, residual, rows, tokens, s);
    }
    if (cols == 9216 && rows % 4 == 0) {
        return launch_rows<KIND, LUT, 9, 1>(W, scale, x, y, residual, rows, tokens, s);
    }
    return 1;
}

template <int KIND, bool LUT, bool VEC>
static int launch_generic(const void* W, float scale, const float* x, float* y,
    const float* residual, uint32_t rows, uint32_t cols, uint32_t tokens, hipStream_t s)
{
    dim3 grid((rows + 3) / 4, tokens);
    hipLaunchKernelGGL((k_rows_generic<KIND, LUT, VEC>), grid, dim3(256), 0, s, W, scale, x, y,
        residual, rows, cols);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int KIND, bool LUT>
static int dispatch(const void* W, float scale, const float* x, float* y, const float* residual,
    uint32_t rows, uint32_t cols, uint32_t tokens, bool vec, hipStream_t s)
{
    if (vec) {
        const int rc = launch_model_rows<KIND, LUT>(W, scale, x, y, residual, rows, cols, tokens, s);
        if (rc <= 0) {
            return rc;
        }
        return launch_generic<KIND, LUT, true>(W, scale, x, y, residual, rows, cols, tokens, s);
    }
    return launch_generic<KIND, LUT, false>(W, scale, x, y, residual, rows, cols, tokens, s);
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
        ((uintptr_t)x % 16) == 0 && cols % 4 == 0;
    if (kind == K_FP8) {
        return lookup ? dispatch<K_FP8, true>(W, scale, x, y, residual, rows, cols, tokens, vec, s)
                      : dispatch<K_FP8, false>(W, scale, x, y, residual, rows, cols, tokens, vec, s);
    }
    if (kind == K_BF16) {
        return dispatch<K_BF16, false>(W, scale, x, y, residual, rows, cols, tokens, vec, s);
    }
    if (kind == K_F32) {
        return dispatch<K_F32, false>(W, scale, x, y, residual, rows, cols, tokens, vec, s);
    }
    return -1;
}

extern "C" int lh_launch_qkv_rope(int lookup, const uint8_t* Wqkv, float sq, float sk, float sv,
    const float* gamma, const float* x, const lh_step_params* params, uint32_t count,
    float* q, float* kcache_layer, float* vcache_layer, uint32_t capacity, hipStream_t s)
{
    dim3 grid(48 * 64 / 6, count);
    float3 scales = make_float3(sq, sk, sv);
    if (lookup) {
        hipLaunchKernelGGL(k_qkv_rope<true>, grid, dim3(256), 0, s, Wqkv, scales, gamma, x, params,
            q, kcache_layer, vcache_layer, capacity);
    } else {
        hipLaunchKernelGGL(k_qkv_rope<false>, grid, dim3(256), 0, s, Wqkv, scales, gamma, x, params,
            q, kcache_layer, vcache_layer, capacity);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

#ifndef LH_ATTN_FUSED_BLOCKS
#define LH_ATTN_FUSED_BLOCKS LH_ATTN_FUSED_MAX   // largest block grid combined in one launch
#endif

// One decode token (count 1): the q|k|v projection, the attention blocks and
// their combine in one launch. arrive: the blocks' 8 zeroed arrival words
// (left zeroed); flags: the producers' 512 flags; bflags: 8 * capacity/64
// block flags; epoch new for every launch on them (nonzero). fault (test
// build only): LH_HANDOFF_BLOCKS makes the blocks, LH_HANDOFF_COMBINERS the
// combiners (past 16 blocks), wait for an epoch nobody stores,
// LH_GIVE_UP_POLLS polls at most, so they give up and the step's output is
// NaN. Callers check lh_attention_chained(length) first.
extern "C" int lh_launch_qkv_attention(int lookup, const uint8_t* Wqkv, float sq, float sk,
    float sv, const float* gamma, const float* x, const lh_step_params* params, uint32_t length,
    float* q, float* kcache_layer, float* vcache_layer, uint32_t capacity, float* PM, float* PT,
    float* PA, unsigned long long* arrive, unsigned long long* flags, unsigned long long* bflags,
    unsigned long long epoch, int fault, float* out, hipStream_t s)
{
    if (capacity % LH_ATTN_BLOCK || length + 1 > capacity || !arrive || !flags || !bflags ||
        !epoch) {
        return -1;
    }
    const bool blocks = fault == LH_HANDOFF_BLOCKS, combiners = fault == LH_HANDOFF_COMBINERS;
    const unsigned long long want = blocks ? epoch + 1 : epoch;
    const uint32_t spins = blocks ? LH_GIVE_UP_POLLS : SPIN_LIMIT;
    const unsigned long long cwant = combiners ? epoch + 1 : epoch;
    const uint32_t cspins = combiners ? LH_GIVE_UP_POLLS : SPIN_LIMIT;
    const uint32_t nblk = lh_attention_blocks(length, 1);
    const bool combine = nblk <= LH_ATTN_FUSED_BLOCKS;
    const dim3 grid(8 * QKV_PRODUCERS + LH_KV_HEADS * nblk + (combine ? 0 : LH_HEADS * 4));
    const float3 scales = make_float3(sq, sk, sv);
#define LH_QKV_ATTN(L, C) hipLaunchKernelGGL((k_qkv_attn<L, C>), grid, dim3(256), 0, s, Wqkv, \
        scales, gamma, x, params, q, kcache_layer, vcache_layer, capacity, nblk, PM, PT, PA, \
        arrive, flags, bflags, epoch, want, spins, cwant, cspins, out)
    if (lookup) {
        if (combine) {
            LH_QKV_ATTN(true, true);
        } else {
            LH_QKV_ATTN(true, false);
        }
    } else {
        if (combine) {
            LH_QKV_ATTN(false, true);
        } else {
            LH_QKV_ATTN(false, false);
        }
    }
#undef LH_QKV_ATTN
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_gateup_silu(int lookup, const uint8_t* Wgate, const uint8_t* Wup,
    float sg, float su, const float* gamma, const float* x, uint32_t count, float* gated,
    hipStream_t s)
{
    static_assert(LH_INNER % (4 * GATEUP_ROWS) == 0, "gate/up rows per workgroup");
    dim3 grid(LH_INNER / (4 * GATEUP_ROWS), count);
    float2 scales = make_float2(sg, su);
    if (lookup) {
        hipLaunchKernelGGL(k_gateup_silu<true>, grid, dim3(512), 0, s, Wgate, Wup, scales, gamma, x, gated);
    } else {
        hipLaunchKernelGGL(k_gateup_silu<false>, grid, dim3(512), 0, s, Wgate, Wup, scales, gamma, x, gated);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_head(const uint16_t* E, const float* gamma, const float* xrow,
    float* logits, uint32_t* nonfinite, hipStream_t s)
{
    hipLaunchKernelGGL(k_head, dim3(LH_VOCAB / 32), dim3(512), 0, s, E, gamma, xrow, logits,
        nonfinite);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int lh_launch_rmsnorm(const float* gamma, const float* x, float* out, uint32_t width,
    uint32_t tokens, hipStream_t s)
{
    if (!width || width > 16 * LH_CHUNK || !tokens) {
        return -1;
    }
    hipLaunchKernelGGL(k_rmsnorm, dim3(tokens), dim3(64), 0, s, gamma, x, out, width);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
