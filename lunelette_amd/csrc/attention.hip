// Causal GQA attention over the resident FP32 KV cache, split across
// workgroups by 64-position blocks (src/metal_kernels.metal:80-132 computes the
// same softmax(q.k/sqrt(128)).V with one SIMD group walking every position).
//
// k_attn_blocks  (block b, kv head, token t): the four query heads sharing the
//   kv head, over the block's valid positions p:
//     c_i  = chain over d in [32i, 32i+32) of fma(q_d, k_pd)   (i = 0..3)
//     s_p  = fl(((c_0 + c_1) + (c_2 + c_3)) * 1/sqrt(128))
//     m_b  = max_p s_p,  e_p = exp(s_p - m_b),  T_b = 64-lane tree of e,
//     A_b[d] = chain_p fma(e_p, v_pd)  (from 0, position order).
// k_attn_combine (head, token): M = max_b m_b, f_b = exp(m_b - M); groups of
//   8 consecutive blocks chain S_g[d] = fma(f_b, A_b[d], .) and
//   U_g = fma(f_b, T_b, .) from 0; A = S_0 + S_1 + ..., T = U_0 + U_1 + ...
//   left to right; out[d] = A[d] / T.
//
// KV layout [kv_head][capacity][128] per layer: a block's K or V tile is one
// contiguous 32 KiB read (K's words permuted inside the tile, lh_ktile_word).
// q and K go to LDS by direct loads (the scores read them there: lane =
// position, quarter of the head dimension); V comes to registers meanwhile and
// overwrites K's LDS region once the scores are done, for the P.V chains. A
// workgroup holds 35 KiB of LDS and 85 registers, so four fit on a CU. Rows at
// or past length+t+1 never enter arithmetic. Up to 16 blocks, the last
// workgroup of each (token, kv head) group to finish combines in the same
// launch: the group runs on one XCD, so the hand-off needs no L2 write-back
// (only the stores' acknowledgements and one L2 atomic per workgroup). Longer
// grids run the combine as its own kernel, 128 workgroups wide, since one
// workgroup's reads of every partial would outlast the launch it saves.
#include "lh_attention_blocks.h"
#include "lh_device.h"
#include "lh_internal.h"

#include <pthread.h>

namespace lh {

// grid (8 * nblk * count): workgroup id = (t * nblk + b) * 8 + kvh, so every
// block of a (token, kv head) group runs on one XCD (the dispatcher deals a
// launch's workgroups to the 8 XCDs in turn, so ids that agree mod 8 share
// one). TAIL_COMBINE: the last workgroup of a group to arrive combines the
// group's four heads itself (k_attn_combine's schedule), reading the
// partials from that XCD's L2. TAIL_FLAG (one token): 128 combiner
// workgroups follow the blocks, id 8 * nblk + (4 * (h % 4) + qd) * 8 + h / 4
// for head h and dimension quarter qd, so each runs on its kv head's XCD and
// combines from its L2 once the head's blocks have flagged their partials
// (flags of epoch `cwant`, at most `cspins` polls; see attn_combiner).
template <AttnTail TAIL>
__global__ void __launch_bounds__(256)
k_attn_blocks(const float* __restrict__ q, const float* __restrict__ kcache,
    const float* __restrict__ vcache, const lh_step_params* __restrict__ params,
    uint32_t capacity, uint32_t nblk, float* __restrict__ PM, float* __restrict__ PT,
    float* __restrict__ PA, unsigned long long* __restrict__ arrive, unsigned long long* bflags,
    unsigned long long epoch, unsigned long long cwant, uint32_t cspins, float* __restrict__ out)
{
    __shared__ union {
        AttnShared blocks;
        CombineShared combine;
    } sh;
    const uint32_t id = blockIdx.x;
    if (TAIL == TAIL_FLAG && id >= 8 * nblk) {
        const uint32_t j = id - 8 * nblk, kvh = j & 7, r = j >> 3;
        attn_combiner(PM, PT, PA, params, capacity, bflags + kvh * (capacity / LH_ATTN_BLOCK),
            cwant, cspins, kvh * 4 + (r >> 2), r & 3, out, sh.combine);
        return;
    }
    const uint32_t kvh = id & 7, b = (id >> 3) % nblk, t = (id >> 3) / nblk;
    attn_block<TAIL, false>(q, kcache, vcache, params, capacity, nblk, PM, PT, PA, arrive, nullptr,
        bflags, epoch, 0, 0, out, b, kvh, t, sh.blocks);
}

// grid (32 heads x 4 dimension quarters, count), 256 threads (attn_combine).
__global__ void __launch_bounds__(256)
k_attn_combine(const float* __restrict__ PM, const float* __restrict__ PT,
    const float* __restrict__ PA, const lh_step_params* __restrict__ params, uint32_t capacity,
    float* __restrict__ out)
{
    __shared__ CombineShared sh;
    const uint32_t t = blockIdx.y;
    attn_combine(PM, PT, PA, params->length + t + 1, capacity, blockIdx.x >> 2, blockIdx.x & 3,
        t, out, sh);
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

// One decode token without a host upload of the step record: workgroup 0
// writes params (the YaRN row of position length expands to the
// [cos | cos], [sin | sin] halves the RoPE reads), and the three workgroups
// widen the 3072 BF16 values of row id, four per thread. grid 3, block 256.
__global__ void __launch_bounds__(256)
k_step_embed(const uint16_t* __restrict__ E, const float* __restrict__ yarn, int32_t id,
    uint32_t length, float qfactor, lh_step_params* __restrict__ params, float* __restrict__ x)
{
    const uint32_t tid = threadIdx.x, g = blockIdx.x * 256 + tid;
    const uint2 raw = reinterpret_cast<const uint2*>(E + (size_t)id * LH_HIDDEN)[g];
    reinterpret_cast<float4*>(x)[g] = make_float4(bf16_to_f32((uint16_t)raw.x),
        bf16_to_f32((uint16_t)(raw.x >> 16)), bf16_to_f32((uint16_t)raw.y),
        bf16_to_f32((uint16_t)(raw.y >> 16)));
    if (blockIdx.x == 0) {
        lh_token_params* tp = &params->tokens[0];
        const float* row = yarn + (size_t)length * 128;
        if (tid < 64) {
            tp->cosine[tid] = tp->cosine[tid + 64] = row[tid];
        } else if (tid < 128) {
            tp->sine[tid - 64] = tp->sine[tid] = row[tid];
        } else if (tid == 128) {
            params->length = length;
            params->count = 1;
            tp->id = id;
            tp->qfactor = qfactor;
            tp->position = length;
        }
    }
}

}  // namespace lh

using namespace lh;

extern "C" int lh_launch_step_embed(const uint16_t* E, const float* yarn, int32_t id,
    uint32_t length, float qfactor, lh_step_params* params, float* x, hipStream_t s)
{
    static_assert(LH_HIDDEN == 3 * 256 * 4, "three workgroups of four values per thread");
    hipLaunchKernelGGL(k_step_embed, dim3(3), dim3(256), 0, s, E, yarn, id, length, qfactor,
        params, x);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

#ifndef LH_ATTN_FUSED_BLOCKS
#define LH_ATTN_FUSED_BLOCKS LH_ATTN_FUSED_MAX   // largest block grid combined in the blocks kernel
#endif
static_assert(LH_ATTN_FUSED_BLOCKS <= lh::FUSED_MAX_BLOCKS, "fused combine capacity");

// Whether a launch's workgroups whose ids agree mod 8 run on one XCD, per
// device, as measured by lh_attention_xcd_probe (0 unknown, 1 yes, 2 no).
static int xcd_dispatch[64];

namespace lh {
__global__ void k_xcd_probe(uint32_t* out)
{
    if (threadIdx.x == 0) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 3)" : "=s"(xcc));
        out[blockIdx.x] = xcc;
    }
}
}  // namespace lh

// Once per device: runs launches of 1, 7, 64, 509 and 1467 workgroups, each
// recording the XCD it ran on into d_words (at least 2048 words, left
// zeroed), and records whether in every launch the workgroups whose ids agree
// mod 8 ran on one XCD (the dispatcher deals workgroups to the XCDs in turn;
// which XCD a launch starts on varies). *ok receives the verdict.
// Synchronizes the stream when it probes.
extern "C" int lh_attention_xcd_probe(uint32_t* d_words, size_t words, int* ok, hipStream_t s)
{
    static const uint32_t grids[] = {1, 7, 64, 509, 1467};
    int device = -1;
    if (!d_words || words < 2048 || hipGetDevice(&device) != hipSuccess || device < 0 ||
        device >= 64) {
        return -1;
    }
    const int known = __atomic_load_n(&xcd_dispatch[device], __ATOMIC_RELAXED);
    if (known) {
        *ok = known == 1;
        return 0;
    }
    uint32_t host[2048];
    size_t at = 0;
    for (uint32_t g : grids) {
        hipLaunchKernelGGL(lh::k_xcd_probe, dim3(g), dim3(64), 0, s, d_words + at);
        at += g;
    }
    if (hipGetLastError() != hipSuccess ||
        hipMemcpyAsync(host, d_words, at * sizeof(uint32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipMemsetAsync(d_words, 0, words * sizeof(uint32_t), s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        return -1;
    }
    int good = 1;
    at = 0;
    for (uint32_t g : grids) {
        for (uint32_t i = 8; i < g; i++) {
            good &= host[at + i] == host[at + i % 8];
        }
        at += g;
    }
    __atomic_store_n(&xcd_dispatch[device], good ? 1 : 2, __ATOMIC_RELAXED);
    *ok = good;
    return 0;
}

static bool fused_attention_ok()
{
    int device = -1;
    return hipGetDevice(&device) == hipSuccess && device >= 0 && device < 64 &&
        __atomic_load_n(&xcd_dispatch[device], __ATOMIC_RELAXED) == 1;
}

// A decode token whose attention spans at most this many blocks (4608
// positions) runs q|k|v and the attention blocks in one launch. Measured on
// the 26-layer decode step: 34, 29 and 18 us faster at 1000, 3000 and 4300
// positions, 30 to 50 us slower from 5500 on, where the blocks outnumber the
// CU slots the projection leaves free and those waiting hold slots the later
// ones need.
#ifndef LH_CHAIN_MAX_BLOCKS
#define LH_CHAIN_MAX_BLOCKS 72
#endif

extern "C" int lh_attention_chained(uint32_t length)
{
    return lh_attention_blocks(length, 1) <= LH_CHAIN_MAX_BLOCKS && fused_attention_ok();
}

// The kernels read the step length from params (device memory); `length`
// here must equal params->length and only sizes the block grid. On a device
// whose dispatch the probe confirmed, with arrive set (count * 8 zeroed
// arrival words, ARRIVE_STRIDE 64-bit words apart, left zeroed) a block grid
// of at most LH_ATTN_FUSED_BLOCKS combines in its own launch; with bflags
// set (8 * capacity/64 words; epoch nonzero and new for every launch on them)
// one token's longer grid runs its blocks and combiners in one launch;
// otherwise blocks and k_attn_combine run as two launches. fault (test build
// only): LH_HANDOFF_COMBINERS makes the combiners wait for an epoch no block
// stores, LH_GIVE_UP_POLLS polls at most, so they give up and write NaN.
extern "C" int lh_launch_attention(const float* q, const float* kcache_layer,
    const float* vcache_layer, const lh_step_params* params, uint32_t length, uint32_t count,
    uint32_t capacity, float* PM, float* PT, float* PA, unsigned long long* arrive,
    unsigned long long* bflags, unsigned long long epoch, int fault, float* out, hipStream_t s)
{
    if (!count || capacity % LH_ATTN_BLOCK || length + count > capacity) {
        return -1;
    }
    const uint32_t nblk = lh_attention_blocks(length, count);
    const dim3 grid(LH_KV_HEADS * nblk * count);
    const bool ok = fused_attention_ok();
    if (ok && arrive && nblk <= LH_ATTN_FUSED_BLOCKS) {
        hipLaunchKernelGGL(k_attn_blocks<TAIL_COMBINE>, grid, dim3(256), 0, s, q, kcache_layer,
            vcache_layer, params, capacity, nblk, PM, PT, PA, arrive, nullptr, 0ull, 0ull, 0u,
            out);
    } else if (ok && bflags && epoch && count == 1) {
        const bool forced = fault == LH_HANDOFF_COMBINERS;
        hipLaunchKernelGGL(k_attn_blocks<TAIL_FLAG>, dim3(LH_KV_HEADS * nblk + LH_HEADS * 4),
            dim3(256), 0, s, q, kcache_layer, vcache_layer, params, capacity, nblk, PM, PT, PA,
            nullptr, bflags, epoch, forced ? epoch + 1 : epoch,
            forced ? LH_GIVE_UP_POLLS : SPIN_LIMIT, out);
    } else {
        hipLaunchKernelGGL(k_attn_blocks<TAIL_NONE>, grid, dim3(256), 0, s, q, kcache_layer,
            vcache_layer, params, capacity, nblk, PM, PT, PA, nullptr, nullptr, 0ull, 0ull, 0u,
            nullptr);
        hipLaunchKernelGGL(k_attn_combine, dim3(LH_HEADS * 4, count), dim3(256), 0, s, PM, PT, PA,
            params, capacity, out);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// lh_attention_noalloc: the same two kernels for callers that cannot allocate.
// The step header (only `length` is read) and the split-KV partials live in
// one file-scope device array per GPU. Host code never passes the array's
// name to a kernel: its device address comes from hipGetSymbolAddress, taken
// once per device on the first call there. Layout: 256-byte header, then PM
// and PT ([count][32][capacity/64] floats each), then PA (x 128).
namespace lh {
constexpr size_t NOALLOC_POSITIONS = 65536;   // largest count * capacity
constexpr size_t NOALLOC_PARTIALS = NOALLOC_POSITIONS / LH_ATTN_BLOCK * LH_HEADS;
constexpr size_t NOALLOC_BYTES = 256 + 4 * NOALLOC_PARTIALS * (2 + LH_HEAD_DIM);
__device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

__global__ void k_set_step(lh_step_params* params, uint32_t length, uint32_t count)
{
    if (threadIdx.x == 0) {
        params->length = length;
        params->count = count;
    }
}
}  // namespace lh

static pthread_mutex_t noalloc_lock = PTHREAD_MUTEX_INITIALIZER;
static unsigned char* noalloc_base[64];

extern "C" int lh_attention_noalloc(const float* d_q, const float* d_keys, const float* d_values,
    size_t length, size_t count, size_t capacity, float* d_out, void* stream)
{
    if (!d_q || !d_keys || !d_values || !d_out || !count || !capacity ||
        capacity % LH_ATTN_BLOCK || length > capacity || count > capacity - length) {
        lh_set_error("attention_noalloc: need q, K, V and out, capacity a multiple of 64, "
            "length + count <= capacity");
        return -1;
    }
    if (count > lh::NOALLOC_POSITIONS / capacity) {
        lh_set_error("attention_noalloc: count * capacity = %zu exceeds the %zu positions of "
            "the static scratch", count * capacity, lh::NOALLOC_POSITIONS);
        return -1;
    }
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
        lh_set_error("attention_noalloc: no current device");
        return -1;
    }
    pthread_mutex_lock(&noalloc_lock);
    if (!noalloc_base[device]) {
        void* ptr = nullptr;
        const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(lh::scratch));
        if (status != hipSuccess || !ptr) {
            pthread_mutex_unlock(&noalloc_lock);
            lh_set_error("attention_noalloc: scratch address: %s", hipGetErrorString(status));
            return -1;
        }
        noalloc_base[device] = static_cast<unsigned char*>(ptr);
    }
    unsigned char* base = noalloc_base[device];
    pthread_mutex_unlock(&noalloc_lock);
    const size_t partials = count * LH_HEADS * (capacity / LH_ATTN_BLOCK);
    lh_step_params* params = reinterpret_cast<lh_step_params*>(base);
    float* PM = reinterpret_cast<float*>(base + 256);
    float* PT = PM + partials;
    float* PA = PT + partials;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(lh::k_set_step, dim3(1), dim3(64), 0, s, params, (uint32_t)length,
        (uint32_t)count);
    if (hipGetLastError() != hipSuccess ||
        lh_launch_attention(d_q, d_keys, d_values, params, (uint32_t)length, (uint32_t)count,
            (uint32_t)capacity, PM, PT, PA, nullptr, nullptr, 0ull, 0, d_out, s)) {
        lh_set_error("attention_noalloc: launch failed");
        return -1;
    }
    return 0;
}

extern "C" uint32_t lh_attention_blocks(uint32_t length, uint32_t count)
{
    return (length + count + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
}

extern "C" int lh_launch_embed(const uint16_t* E, const lh_step_params* params, uint32_t count,
    float* x, hipStream_t s)
{
    hipLaunchKernelGGL(k_embed, dim3(count), dim3(256), 0, s, E, params, x);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// Multi-token attention on the matrix cores (the PREFILL_MPS path; the
// precise path keeps the block/combine kernels above): a flash attention on
// the FP16 and BF16 matrix cores (v_mfma_f32_16x16x32_{f16,bf16}),
// tolerance-checked, not bit-mirrored.
//
// Workgroup (32-token tile, kv head), eight waves: wave w is query head
// 4*kvh + w % 4 over the tile's 16-token half w / 4, so the four GQA heads and
// both halves share every K/V block staged in LDS (one staging serves 32
// tokens), one workgroup per CU. Per 64-position block:
//   S^T[64 x 16] = K[64 x 128] Q^T, Q in registers; a lane holds one
//     token's column (16 positions, the other three lane groups the rest);
//   online softmax per token in the base-2 domain (v_exp_f32), causal mask
//     p <= length + t; the row statistics reduce over the lane's own values
//     and two permlane swaps;
//   O^T[128 x 16] += V^T[128 x 64] P^T: the lane's column of P^T is
//     exactly its PV B operand (k slots = the positions of its S^T rows),
//     so P never leaves the registers.
// out = O / l. grid tiles * 8 * splits (1-D, fa_coords), block 512. With
// splits > 1 split z takes a contiguous range of the tile's blocks and writes
// its unnormalized (max, sum, O) rows as part z of PM/PT/PA (partial stride
// capacity/64 per (token, head)), merged by k_attn_merge. With xs set, the
// output goes to xs as the o projection's two FP16 planes (plane stride
// xs_tokens * 4096, one power of two per (token, kv head) in xs_scale)
// instead of FP32 rows of out.
// Measured at 256 tokens after a 4096-token prefix: 88 us (94 us with
// S = Q K^T and P through a per-wave LDS tile, whose reuse of the K planes
// cost a third barrier per block: per block about 1.5k cycles of barrier
// skew, 1.5k of staging, 1.0k of the second barrier, 2.1k of QK^T, 1.0k of
// the third barrier, 1.7k of softmax and P tile, 1.6k of PV; 104 us with
// QK^T over three exact BF16 planes of Q and K, six products). Earlier: V's
// transposed planes and the P tiles in 128-byte rows with an XOR swizzle
// (16-way bank conflicts on the staging writes, 5.3k cycles of split) and
// the softmax's row reductions through LDS swizzles, 129 us; 16-token
// workgroups of four waves, two per CU, 169 us; the FP32 matrix cores
// (v_mfma_f32_16x16x4_f32, exact products) with 16-token workgroups 198 us.
// Also measured: waves as (head, 32-position half) over all 32 tokens with
// S^T in registers feeding PV directly and the raw tiles through LDS by
// direct loads: 94 us at the 4096-token prefix but slower on short prefixes
// (16.8 against 12.5 us on a 256-token chunk with no prefix): its per-block
// staging and two barriers per block dominated, as here.
namespace lh {

constexpr uint32_t FA_TQ = 16;                      // tokens per workgroup
// Scores in the base-2 domain: s = q.k * (1/sqrt(128)) * log2(e), so the
// softmax weights are exp2(s - m) on the hardware v_exp_f32; the row maxima
// in PM are in this domain too (k_attn_merge).
constexpr float FA_SCALE_LOG2 = 0.12751743074062763f;

typedef float fa_floatx4 __attribute__((ext_vector_type(4)));

// Maximum (and sum) over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lane
// groups that hold one MFMA operand row or D column), in all four: v_permlane16_swap /
// v_permlane32_swap of a register with itself hands every lane its
// partner's value in one of the two results.
__device__ __forceinline__ float col4_max(float v)
{
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float w = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const uint32_t x = __float_as_uint(w);
    const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float col4_sum(float v)
{
    const uint32_t u = __float_as_uint(v);
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float w = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const uint32_t x = __float_as_uint(w);
    const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Workgroup coordinates of the matrix-core attention: a 1-D grid of
// tiles * 8 * splits workgroups whose ids are dealt round-robin to the 8
// XCDs, arranged so that XCD x runs every (token tile, KV split) of kv head
// x. The 16-token tiles of a kv head then re-read its K/V blocks from their
// XCD's L2 instead of the Infinity Cache.
struct FaCoords {
    uint32_t t0, kvh, z, splits;
};

__device__ __forceinline__ FaCoords fa_coords(uint32_t tiles)
{
    const uint32_t w = blockIdx.x, qq = w >> 3;
    return {(qq % tiles) * FA_TQ, w & 7u, qq / tiles, gridDim.x / (8 * tiles)};
}


// The operands as 16-bit planes:
//   QK^T: Q and K as two FP16 planes of the row scaled by a power of two
//     (its largest magnitude into [2^14, 2^15)): per (token, head) row for
//     Q, per position for K, h = f16(x 2^e), l = f16(x 2^e - h), about 22
//     significant bits each. Products ql kh, qh kl, qh kh (smallest first;
//     ql kl lies near 2^-22 of the leading one), then times 2^-eq 2^-ek
//     (exact), so the scores keep near-FP32 accuracy, which the softmax
//     needs;
//   PV: P and V in two truncated BF16 planes (hi + mid, 16 significant
//     bits); products pm vh, ph vm, ph vh, so the output's relative error
//     stays near 2^-16.
// Every 16-bit product is exact in FP32; accumulation is the hardware's FP32.
// Workgroup and grid as described above.
// LDS (69 KiB): the block's K planes [2][64 pos][128 dims], each 16-byte
// chunk of a row XOR-swizzled by the row index, the 64 per-position factors
// 2^-ek, and V planes transposed [2][128 dims][64 pos] in 144-byte rows, so
// the MFMA operand reads and the staging writes are conflict-free.
typedef __bf16 fa_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 fa_f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t fa_u32x4 __attribute__((ext_vector_type(4)));

// Transposed V rows hold 64 positions (128 bytes) padded to 144 bytes:
// 16 consecutive rows then start 36 banks apart, which spreads the operand
// reads and the staging writes over all 64 banks.
constexpr uint32_t FB_ROW = 144;
constexpr uint32_t FB_KPLANE = LH_ATTN_BLOCK * LH_HEAD_DIM * 2;   // bytes per K plane
constexpr uint32_t FB_VPLANE = LH_HEAD_DIM * FB_ROW;              // bytes per V plane

// Byte offset of (row r, element e) in a K plane: rows of 256 bytes, chunk
// e / 8 XOR (r & 15).
__device__ __forceinline__ uint32_t fb_k_at(uint32_t r, uint32_t e)
{
    return r * 256 + (((e >> 3) ^ (r & 15)) << 4) + (e & 7) * 2;
}

// Byte offset of (dim d, position r) in a transposed V plane.
__device__ __forceinline__ uint32_t fb_v_at(uint32_t d, uint32_t r)
{
    return d * FB_ROW + r * 2;
}

__device__ __forceinline__ uint32_t fb_hi(float x)
{
    return __float_as_uint(x) >> 16;
}

// Two FP16 planes of four values scaled by f (h = f16(v f), l = f16(v f - h)),
// packed as two 32-bit pairs each.
__device__ __forceinline__ void f16_planes4(float4 v, float f, uint2& h, uint2& l)
{
    float r0, r1, r2, r3;
    const uint32_t a = f16_hi(v.x * f, r0), b = f16_hi(v.y * f, r1);
    const uint32_t c = f16_hi(v.z * f, r2), d = f16_hi(v.w * f, r3);
    h = make_uint2(a | (b << 16), c | (d << 16));
    l = make_uint2(f16_bits(r0) | (f16_bits(r1) << 16), f16_bits(r2) | (f16_bits(r3) << 16));
}

// Two truncated BF16 planes of x: hi and mid (x - hi, truncated).
__device__ __forceinline__ void fb_split2(float x, uint32_t& h, uint32_t& m)
{
    const uint32_t hb = __float_as_uint(x) & 0xffff0000u;
    h = hb >> 16;
    m = __float_as_uint(x - __uint_as_float(hb)) >> 16;
}

__global__ void __launch_bounds__(512, 1)
k_attn_mfma(const float* __restrict__ q, const float* __restrict__ kcache,
    const float* __restrict__ vcache, uint32_t length, uint32_t count, uint32_t capacity,
    float* __restrict__ PM, float* __restrict__ PT, float* __restrict__ PA, float* __restrict__ out,
    uint16_t* __restrict__ xs, uint32_t xs_tokens, float* __restrict__ xs_scale)
{
    __shared__ __attribute__((aligned(16))) uint8_t Kp[2 * FB_KPLANE];
    __shared__ __attribute__((aligned(16))) uint8_t Vp[2 * FB_VPLANE];
    __shared__ float sk[LH_ATTN_BLOCK];
    const FaCoords fc = fa_coords((count + 2 * FA_TQ - 1) / (2 * FA_TQ));
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t t0 = 2 * fc.t0 + FA_TQ * (wave >> 2), kvh = fc.kvh;
    const uint32_t g = lane >> 4, l16 = lane & 15;
    const uint32_t head = kvh * 4 + (wave & 3);
    // The second 16-token subtile can lie past count: it then runs on the
    // first subtile's last token (clamped) and stores nothing.
    const uint32_t t0c = t0 < count ? t0 : t0 - FA_TQ;
    const uint32_t last = (t0c + FA_TQ < count ? t0c + FA_TQ : count) - 1;   // last real token
    // Q operand of k-chunk kc (the B operand of S^T = K Q^T): lane (token
    // l16, group g) holds dims 32 kc + 8g .. +7, as two FP16 planes of the
    // row scaled by 2^eq (its largest magnitude into [2^14, 2^15)). fq =
    // 2^-eq * log2(e) / sqrt(128) for the lane's token, whose S^T column the
    // lane also holds.
    const uint32_t tq = t0 + l16 <= last ? t0 + l16 : last;
    fa_f16x8 qh[4], ql[4];
    float fq;
    {
        const float4* src = reinterpret_cast<const float4*>(
            q + (size_t)tq * LH_QUERY + head * LH_HEAD_DIM + 8 * g);
        float4 a[4], b[4];
        float mx = 0.0f;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            a[kc] = src[8 * kc];
            b[kc] = src[8 * kc + 1];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a[kc].x), fabsf(a[kc].y)),
                                 fmaxf(fabsf(a[kc].z), fabsf(a[kc].w))));
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(b[kc].x), fabsf(b[kc].y)),
                                 fmaxf(fabsf(b[kc].z), fabsf(b[kc].w))));
        }
        const int eq = row_exponent(col4_max(mx));
        const float f = exp2i(eq);
        fq = exp2i(-eq) * FA_SCALE_LOG2;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            uint2 h0, l0, h1, l1;
            f16_planes4(a[kc], f, h0, l0);
            f16_planes4(b[kc], f, h1, l1);
            qh[kc] = __builtin_bit_cast(fa_f16x8, fa_u32x4{h0.x, h0.y, h1.x, h1.y});
            ql[kc] = __builtin_bit_cast(fa_f16x8, fa_u32x4{l0.x, l0.y, l1.x, l1.y});
        }
    }
    const uint32_t limit = length + tq;   // the lane's token's last visible position
    // Online-softmax state of the lane's token (replicated over its four
    // lane groups) and O^T tiles i: dims 16 i + 4g + r of the lane's token.
    float m = -__builtin_inff(), l = 0.0f;
    fa_floatx4 o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        o[i] = fa_floatx4{0.f, 0.f, 0.f, 0.f};
    }
    // The block range and the staging's visible rows follow the workgroup's
    // last token (both subtiles share every barrier and every staged block).
    const uint32_t tw = 2 * fc.t0;
    const uint32_t last_wg = (tw + 2 * FA_TQ < count ? tw + 2 * FA_TQ : count) - 1;
    const uint32_t nb = (length + last_wg + 1 + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    const uint32_t splits = fc.splits, z = fc.z;
    const uint32_t per = (nb + splits - 1) / splits;
    const uint32_t b_begin = z * per < nb ? z * per : nb;
    const uint32_t b_end = b_begin + per < nb ? b_begin + per : nb;
    const size_t head_base = lh_kv_index(capacity, 0, kvh, 0);
    // Raw K and V of block b in registers, the next block's issued before
    // this block's MFMAs. K: thread tid holds float4 words tid + 256 i of the
    // tile (lh_ktile_word order); V: rows 2 rp and 2 rp + 1, float4 column
    // tid % 32, rp = tid / 32 + 8 i, so that two consecutive positions of a
    // dimension pack into one 32-bit word of the transposed planes.
    // V staging item j (0..7) of thread tid: lane l of wave w takes dim
    // 16 (j % 8) + l % 16 and positions r0, r0 + 1 with r0 = 2 (4 w + l / 16),
    // so one wave instruction covers 16 dims x 4 position pairs: the loads
    // read 4 x 64 contiguous bytes, and the packed-pair writes of the
    // transposed planes land on 64 distinct banks.
    auto v_item = [&](int j, uint32_t& d, uint32_t& r0) {
        d = 16 * j + (lane & 15);
        r0 = 2 * (4 * wave + (lane >> 4));
    };
    // K: wave w takes positions 8w .. 8w+7 of the block; lane l holds
    // position kp = 8w + (l % 32) / 4, quarter kq = l % 4, dims
    // 32 kq + 4 (2i + l / 32) .. +3 for i = 0..3 (tile word order
    // lh_ktile_word: each load reads two contiguous 512-byte runs), so the
    // eight lanes of a position hold all its 128 dims.
    const uint32_t kp = 8 * wave + ((lane & 31) >> 2), kq = lane & 3, khalf = lane >> 5;
    fa_floatx4 kr[4];
    float vr[16];
    auto load_block = [&](uint32_t b) {
        const fa_floatx4* kb = reinterpret_cast<const fa_floatx4*>(
            kcache + head_base + (size_t)b * LH_ATTN_BLOCK * LH_HEAD_DIM);
        const fa_floatx4* vb = reinterpret_cast<const fa_floatx4*>(
            vcache + head_base + (size_t)b * LH_ATTN_BLOCK * LH_HEAD_DIM);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[i] = kb[lh_ktile_word(kp, kq, 2 * i + khalf)];
        }
        const float* vf = reinterpret_cast<const float*>(vb);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t d, r0;
            v_item(j, d, r0);
            vr[2 * j] = vf[r0 * LH_HEAD_DIM + d];
            vr[2 * j + 1] = vf[(r0 + 1) * LH_HEAD_DIM + d];
        }
    };
    if (b_begin < b_end) {
        load_block(b_begin);
    }
    // Rows past the tile's last visible position hold whatever an earlier
    // sequence (or a failed step) left in the cache; they are staged as zeros
    // (0 * Inf would be NaN in P.V).
    const uint32_t visible = length + last_wg;
    const fa_floatx4 zero = fa_floatx4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t b = b_begin; b < b_end; b++) {
        __syncthreads();   // the previous block's planes are consumed
        {
            // K: the position's largest magnitude over its eight lanes (a
            // DPP quad, then the other 32-lane half), its power of two 2^ek
            // (into [2^14, 2^15)), and the two FP16 planes; sk[p] = 2^-ek.
            const bool kvis = b * LH_ATTN_BLOCK + kp <= visible;
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[i] = kvis ? kr[i] : zero;
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(kr[i].x), fabsf(kr[i].y)),
                                     fmaxf(fabsf(kr[i].z), fabsf(kr[i].w))));
            }
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0xB1, 0xf,
                0xf, false)));   // quad_perm [1,0,3,2]
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x4E, 0xf,
                0xf, false)));   // quad_perm [2,3,0,1]
            const uint32_t mu = __float_as_uint(mx);
            const auto p32 = __builtin_amdgcn_permlane32_swap(mu, mu, false, false);
            const int ek = row_exponent(fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1])));
            if ((lane & 35) == 0) {
                sk[kp] = exp2i(-ek);
            }
            const float f = exp2i(ek);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint2 h, lo;
                f16_planes4(make_float4(kr[i].x, kr[i].y, kr[i].z, kr[i].w), f, h, lo);
                const uint32_t at = fb_k_at(kp, 32 * kq + 4 * (2 * i + khalf));
                *reinterpret_cast<uint2*>(Kp + at) = h;
                *reinterpret_cast<uint2*>(Kp + FB_KPLANE + at) = lo;
            }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t d, r0;
            v_item(j, d, r0);
            const float v0 = b * LH_ATTN_BLOCK + r0 <= visible ? vr[2 * j] : 0.0f;
            const float v1 = b * LH_ATTN_BLOCK + r0 + 1 <= visible ? vr[2 * j + 1] : 0.0f;
            uint32_t h0, m0, h1, m1;
            fb_split2(v0, h0, m0);
            fb_split2(v1, h1, m1);
            const uint32_t at = fb_v_at(d, r0);
            *reinterpret_cast<uint32_t*>(Vp + at) = h0 | (h1 << 16);
            *reinterpret_cast<uint32_t*>(Vp + FB_VPLANE + at) = m0 | (m1 << 16);
        }
        __syncthreads();
        if (b + 1 < b_end) {
            load_block(b + 1);   // in flight during this block's MFMAs
        }
        // S^T tiles j = 0..3: rows positions 16j + 4g + r, columns tokens l16
        // (A operand K: row 16j + l16, dims 32kc + 8g .. +7).
        fa_floatx4 s[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            s[j] = zero;
        }
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t at = fb_k_at(16 * j + l16, 32 * kc + 8 * g);
                const fa_f16x8 kh = *reinterpret_cast<const fa_f16x8*>(Kp + at);
                const fa_f16x8 kl = *reinterpret_cast<const fa_f16x8*>(Kp + FB_KPLANE + at);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[kc], s[j], 0, 0, 0);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[kc], s[j], 0, 0, 0);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[kc], s[j], 0, 0, 0);
            }
        }
        // Scale (2^-ek of the row's position, fq of the token), causal mask,
        // online softmax of the lane's token over its 16 values and its three
        // other lane groups; P^T as the PV B operand of position chunk pc:
        // k slots 0..3 = positions 32 pc + 4g + r (tile j = 2 pc), slots 4..7
        // = 32 pc + 16 + 4g + r (tile j = 2 pc + 1).
        fa_bf16x8 ph[2], pm[2];
        {
            float v[16];
            float mx = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const fa_floatx4 fk = *reinterpret_cast<const fa_floatx4*>(sk + 16 * j + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t p = b * LH_ATTN_BLOCK + 16 * j + 4 * g + r;
                    const float x = p <= limit ? s[j][r] * fk[r] * fq : -__builtin_inff();
                    v[4 * j + r] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = col4_max(mx);
            // A split can start past a token's last visible position: keep
            // its row empty (no exp of -inf - -inf).
            const float m_new = fmaxf(m, mx);
            const bool empty = m_new == -__builtin_inff();
            const float alpha = empty ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
            float sum = 0.0f;
#pragma unroll
            for (int pc = 0; pc < 2; pc++) {
                fa_u32x4 hi, mid;
#pragma unroll
                for (int k = 0; k < 8; k += 2) {
                    const float e0 = empty ? 0.0f : __builtin_amdgcn_exp2f(v[8 * pc + k] - m_new);
                    const float e1 = empty ? 0.0f : __builtin_amdgcn_exp2f(v[8 * pc + k + 1] - m_new);
                    sum = sum + e0;
                    sum = sum + e1;
                    uint32_t h0, m0, h1, m1;
                    fb_split2(e0, h0, m0);
                    fb_split2(e1, h1, m1);
                    hi[k / 2] = h0 | (h1 << 16);
                    mid[k / 2] = m0 | (m1 << 16);
                }
                ph[pc] = __builtin_bit_cast(fa_bf16x8, hi);
                pm[pc] = __builtin_bit_cast(fa_bf16x8, mid);
            }
            l = l * alpha + col4_sum(sum);
            m = m_new;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                o[i] = o[i] * alpha;
            }
        }
        // O^T += V^T P^T: A operand of dim tile i: lane (dim 16 i + l16, group
        // g) holds V at positions 32 pc + 4g .. +3 and 32 pc + 16 + 4g .. +3
        // (two 8-byte reads per plane), the slots of P^T above.
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t d = 16 * i + l16;
#pragma unroll
            for (int pc = 0; pc < 2; pc++) {
                const uint32_t a0 = fb_v_at(d, 32 * pc + 4 * g);
                const uint32_t a1 = fb_v_at(d, 32 * pc + 16 + 4 * g);
                const uint2 h0 = *reinterpret_cast<const uint2*>(Vp + a0);
                const uint2 h1 = *reinterpret_cast<const uint2*>(Vp + a1);
                const uint2 m0 = *reinterpret_cast<const uint2*>(Vp + FB_VPLANE + a0);
                const uint2 m1 = *reinterpret_cast<const uint2*>(Vp + FB_VPLANE + a1);
                const fa_bf16x8 vh = __builtin_bit_cast(fa_bf16x8, fa_u32x4{h0.x, h0.y, h1.x, h1.y});
                const fa_bf16x8 vm = __builtin_bit_cast(fa_bf16x8, fa_u32x4{m0.x, m0.y, m1.x, m1.y});
                o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vm, ph[pc], o[i], 0, 0, 0);
                o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pm[pc], o[i], 0, 0, 0);
                o[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[pc], o[i], 0, 0, 0);
            }
        }
    }
    // Output planes (one split): each token's four query heads of this kv
    // head (512 columns, one K split of the o projection) share one power of
    // two 2^e, their largest magnitude into [2^14, 2^15), before the split
    // into two FP16 planes; xs_scale[t][kv head] = 2^-e. The heads' maxima
    // meet in LDS before any wave leaves.
    __shared__ float gmax[2 * FA_TQ][4];
    if (splits == 1 && xs) {
        float mr = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            mr = fmaxf(mr, fmaxf(fmaxf(fabsf(o[i].x), fabsf(o[i].y)),
                                 fmaxf(fabsf(o[i].z), fabsf(o[i].w))));
        }
        mr = col4_max(mr) / l;
        if (g == 0) {
            gmax[FA_TQ * (wave >> 2) + l16][wave & 3] = mr;
        }
        __syncthreads();
    }
    // The lane's token and its O^T values: dims 16 i + 4g .. +3.
    const uint32_t t = t0 + l16;
    if (t0 >= count || t > last) {
        return;
    }
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    if (splits == 1) {
        const float inv = 1.0f / l;
        if (xs) {
            const float* gm = gmax[FA_TQ * (wave >> 2) + l16];
            const int e = row_exponent(fmaxf(fmaxf(gm[0], gm[1]), fmaxf(gm[2], gm[3])));
            if (g == 0 && (wave & 3) == 0) {
                xs_scale[t * LH_KV_HEADS + kvh] = exp2i(-e);
            }
            const float f = exp2i(e);
            const size_t plane = (size_t)xs_tokens * LH_QUERY;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const fa_floatx4 v = o[i] * (inv * f);
                store_f16x2_4(xs, plane, xs_at(t, head * LH_HEAD_DIM + 16 * i + 4 * g, LH_QUERY),
                    make_float4(v.x, v.y, v.z, v.w));
            }
        } else {
            float* dst = out + (size_t)t * LH_QUERY + head * LH_HEAD_DIM + 4 * g;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const fa_floatx4 v = o[i] * inv;
                *reinterpret_cast<float4*>(dst + 16 * i) = make_float4(v.x, v.y, v.z, v.w);
            }
        }
    } else {
        const size_t part = ((size_t)t * LH_HEADS + head) * nbc + z;
        if (g == 0) {
            PM[part] = m;
            PT[part] = l;
        }
        float* dst = PA + part * LH_HEAD_DIM + 4 * g;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            *reinterpret_cast<float4*>(dst + 16 * i) = make_float4(o[i].x, o[i].y, o[i].z, o[i].w);
        }
    }
}

// The wide variant for long prefixes (k_attn_mfma_wide): 64-token
// workgroups, each wave running two 16-token subtiles over every staged
// block, so each block is split into planes once per 64 tokens. The two
// passes' Q planes and O accumulators double the per-wave state; the raw
// K/V tiles therefore come to LDS by direct loads (136 KiB of LDS) instead of
// through registers, and each K and V fragment read from LDS feeds both
// passes. Measured (attention + merge, 256 tokens): 88.5 against 95.8 us
// after a 4096-token prefix, 148 against 170 us after 8192, 255 against 304
// us after 16128; slower on short prefixes (28.6 against 22.5 us with no
// prefix: half the workgroups) and for 64 tokens, where the launcher keeps
// k_attn_mfma.
constexpr uint32_t WIDE_PASSES = 2;                          // subtiles per wave
constexpr uint32_t WIDE_WG = 2 * WIDE_PASSES * FA_TQ;        // tokens per workgroup
constexpr uint32_t WIDE_MIN_LENGTH = 2048;                   // prefix from which it pays
constexpr uint32_t WIDE_MIN_COUNT = 128;                     // tokens from which it pays

__global__ void __launch_bounds__(512, 1)
k_attn_mfma_wide(const float* __restrict__ q, const float* __restrict__ kcache,
    const float* __restrict__ vcache, uint32_t length, uint32_t count, uint32_t capacity,
    float* __restrict__ PM, float* __restrict__ PT, float* __restrict__ PA, float* __restrict__ out,
    uint16_t* __restrict__ xs, uint32_t xs_tokens, float* __restrict__ xs_scale)
{
    __shared__ __attribute__((aligned(16))) uint8_t Kp[2 * FB_KPLANE];
    __shared__ __attribute__((aligned(16))) uint8_t Vp[2 * FB_VPLANE];
    __shared__ float sk[LH_ATTN_BLOCK];
    const FaCoords fc = fa_coords((count + WIDE_WG - 1) / WIDE_WG);
    const uint32_t tid = threadIdx.x, kvh = fc.kvh;
    uint32_t lane = tid & 63, wave = tid >> 6;
    uint32_t g = lane >> 4, l16 = lane & 15;
    uint32_t head = kvh * 4 + (wave & 3);
    // The workgroup's WIDE_WG tokens start at tw; wave w runs 16-token subtiles
    // 2 pass + w / 4 in passes 0 and 1 over every staged block.
    const uint32_t tw = fc.t0 * (WIDE_WG / FA_TQ);
    const uint32_t last_wg = (tw + WIDE_WG < count ? tw + WIDE_WG : count) - 1;
    // A subtile can lie past count: it then runs on the last real subtile's
    // tokens (clamped) and stores nothing.
    const uint32_t last_sub = (count - 1) / FA_TQ * FA_TQ;
    uint32_t t0[WIDE_PASSES], last[WIDE_PASSES];
    // The lane's token in pass ps (clamped to the subtile's last real token).
    auto tq_of = [&](int ps) { return t0[ps] + l16 <= last[ps] ? t0[ps] + l16 : last[ps]; };
    // Q operand of k-chunk kc (the B operand of S^T = K Q^T): lane (token
    // l16, group g) holds dims 32 kc + 8g .. +7, as two FP16 planes of the
    // row scaled by 2^eq (its largest magnitude into [2^14, 2^15)). fq =
    // 2^-eq * log2(e) / sqrt(128) for the lane's token, whose S^T column the
    // lane also holds.
    fa_f16x8 qh[WIDE_PASSES][4], ql[WIDE_PASSES][4];
    float fq[WIDE_PASSES];
    // Online-softmax state of the lane's token (replicated over its four
    // lane groups) and O^T tiles i: dims 16 i + 4g + r of the lane's token.
    float m[WIDE_PASSES], l[WIDE_PASSES];
    fa_floatx4 o[WIDE_PASSES][8];
#pragma unroll
    for (int ps = 0; ps < WIDE_PASSES; ps++) {
        t0[ps] = tw + FA_TQ * (2 * ps + (wave >> 2));
        const uint32_t t0c = t0[ps] < count ? t0[ps] : last_sub;
        last[ps] = (t0c + FA_TQ < count ? t0c + FA_TQ : count) - 1;   // last real token
        const uint32_t tq = t0[ps] + l16 <= last[ps] ? t0[ps] + l16 : last[ps];
        const float4* src = reinterpret_cast<const float4*>(
            q + (size_t)tq * LH_QUERY + head * LH_HEAD_DIM + 8 * g);
        float4 a[4], b[4];
        float mx = 0.0f;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            a[kc] = src[8 * kc];
            b[kc] = src[8 * kc + 1];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a[kc].x), fabsf(a[kc].y)),
                                 fmaxf(fabsf(a[kc].z), fabsf(a[kc].w))));
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(b[kc].x), fabsf(b[kc].y)),
                                 fmaxf(fabsf(b[kc].z), fabsf(b[kc].w))));
        }
        const int eq = row_exponent(col4_max(mx));
        const float f = exp2i(eq);
        fq[ps] = exp2i(-eq) * FA_SCALE_LOG2;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            uint2 h0, l0, h1, l1;
            f16_planes4(a[kc], f, h0, l0);
            f16_planes4(b[kc], f, h1, l1);
            qh[ps][kc] = __builtin_bit_cast(fa_f16x8, fa_u32x4{h0.x, h0.y, h1.x, h1.y});
            ql[ps][kc] = __builtin_bit_cast(fa_f16x8, fa_u32x4{l0.x, l0.y, l1.x, l1.y});
        }
        m[ps] = -__builtin_inff();
        l[ps] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            o[ps][i] = fa_floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    // The block range and the staging's visible rows follow the workgroup's
    // last token (all subtiles share every barrier and every staged block).
    const uint32_t nb = (length + last_wg + 1 + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    const uint32_t splits = fc.splits, z = fc.z;
    const uint32_t per = (nb + splits - 1) / splits;
    const uint32_t b_begin = z * per < nb ? z * per : nb;
    const uint32_t b_end = b_begin + per < nb ? b_begin + per : nb;
    const size_t head_base = lh_kv_index(capacity, 0, kvh, 0);
    // Raw K and V of block b go to LDS by direct loads (the next block's
    // issued once this block's staging has read them, in flight during its
    // MFMAs): the tiles as they lie in the cache, K in lh_ktile_word order,
    // V row-major. Wave w, load i copies the 1 KiB chunk 8i + w of each.
    // V staging item j (0..7) of thread tid: lane l of wave w takes dim
    // 16 ((j + l / 16) % 8) + l % 16 and positions r0, r0 + 1 with
    // r0 = 2 (4 w + l / 16). The four 16-lane groups of a wave read four
    // different 16-dim blocks of the raw tile, so the reads of the row-major
    // raw V land on 64 distinct banks (rows are 128 words apart, so without
    // the rotation the groups' reads met on the same 16 banks); the
    // packed-pair writes of the transposed planes land on 64 distinct banks
    // either way (row d starts 36 d words in).
    auto v_item = [&](int j, uint32_t& d, uint32_t& r0) {
        d = 16 * ((j + (lane >> 4)) & 7) + (lane & 15);
        r0 = 2 * (4 * wave + (lane >> 4));
    };
    // K: wave w takes positions 8w .. 8w+7 of the block; lane l holds
    // position kp = 8w + (l % 32) / 4, quarter kq = l % 4, dims
    // 32 kq + 4 (2i + l / 32) .. +3 for i = 0..3, so the eight lanes of a
    // position hold all its 128 dims.
    const uint32_t kp = 8 * wave + ((lane & 31) >> 2), kq = lane & 3, khalf = lane >> 5;
    __shared__ __attribute__((aligned(16))) fa_floatx4 Kraw[LH_ATTN_BLOCK * LH_HEAD_DIM / 4];
    __shared__ __attribute__((aligned(16))) fa_floatx4 Vraw[LH_ATTN_BLOCK * LH_HEAD_DIM / 4];
    auto load_block = [&](uint32_t b) {
        const fa_floatx4* kb = reinterpret_cast<const fa_floatx4*>(
            kcache + head_base + (size_t)b * LH_ATTN_BLOCK * LH_HEAD_DIM);
        const fa_floatx4* vb = reinterpret_cast<const fa_floatx4*>(
            vcache + head_base + (size_t)b * LH_ATTN_BLOCK * LH_HEAD_DIM);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t c = 8 * i + wave;
            __builtin_amdgcn_global_load_lds(kb + 64 * c + lane, Kraw + 64 * c, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vb + 64 * c + lane, Vraw + 64 * c, 16, 0, 0);
        }
    };
    if (b_begin < b_end) {
        load_block(b_begin);
    }
    // Rows past the tile's last visible position hold whatever an earlier
    // sequence (or a failed step) left in the cache; they are staged as zeros
    // (0 * Inf would be NaN in P.V).
    const uint32_t visible = length + last_wg;
    const fa_floatx4 zero = fa_floatx4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t b = b_begin; b < b_end; b++) {
        // Block b's raw tiles have landed (each wave waits for its own direct
        // loads) and the previous block's planes are consumed.
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __syncthreads();
        {
            fa_floatx4 kr[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[i] = Kraw[lh_ktile_word(kp, kq, 2 * i + khalf)];
            }
            // K: the position's largest magnitude over its eight lanes (a
            // DPP quad, then the other 32-lane half), its power of two 2^ek
            // (into [2^14, 2^15)), and the two FP16 planes; sk[p] = 2^-ek.
            const bool kvis = b * LH_ATTN_BLOCK + kp <= visible;
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                kr[i] = kvis ? kr[i] : zero;
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(kr[i].x), fabsf(kr[i].y)),
                                     fmaxf(fabsf(kr[i].z), fabsf(kr[i].w))));
            }
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0xB1, 0xf,
                0xf, false)));   // quad_perm [1,0,3,2]
            mx = fmaxf(mx, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(mx), 0x4E, 0xf,
                0xf, false)));   // quad_perm [2,3,0,1]
            const uint32_t mu = __float_as_uint(mx);
            const auto p32 = __builtin_amdgcn_permlane32_swap(mu, mu, false, false);
            const int ek = row_exponent(fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1])));
            if ((lane & 35) == 0) {
                // The position again from the thread id (a register held for
                // it across the loop would spill).
                uint32_t t = threadIdx.x;
                asm volatile("" : "+v"(t));
                sk[8 * (t >> 6) + ((t & 31) >> 2)] = exp2i(-ek);
            }
            const float f = exp2i(ek);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint2 h, lo;
                f16_planes4(make_float4(kr[i].x, kr[i].y, kr[i].z, kr[i].w), f, h, lo);
                const uint32_t at = fb_k_at(kp, 32 * kq + 4 * (2 * i + khalf));
                *reinterpret_cast<uint2*>(Kp + at) = h;
                *reinterpret_cast<uint2*>(Kp + FB_KPLANE + at) = lo;
            }
        }
        const float* vf = reinterpret_cast<const float*>(Vraw);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t d, r0;
            v_item(j, d, r0);
            const float v0 = b * LH_ATTN_BLOCK + r0 <= visible ? vf[r0 * LH_HEAD_DIM + d] : 0.0f;
            const float v1 = b * LH_ATTN_BLOCK + r0 + 1 <= visible ?
                vf[(r0 + 1) * LH_HEAD_DIM + d] : 0.0f;
            uint32_t h0, m0, h1, m1;
            fb_split2(v0, h0, m0);
            fb_split2(v1, h1, m1);
            const uint32_t at = fb_v_at(d, r0);
            *reinterpret_cast<uint32_t*>(Vp + at) = h0 | (h1 << 16);
            *reinterpret_cast<uint32_t*>(Vp + FB_VPLANE + at) = m0 | (m1 << 16);
        }
        __syncthreads();
        if (b + 1 < b_end) {
            load_block(b + 1);   // in flight during this block's MFMAs
        }
        // S^T tiles j = 0..3 of each pass: rows positions 16j + 4g + r,
        // columns tokens l16 (A operand K: row 16j + l16, dims 32kc + 8g ..
        // +7, read once for both passes).
        fa_floatx4 s[WIDE_PASSES][4];
#pragma unroll
        for (int ps = 0; ps < WIDE_PASSES; ps++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                s[ps][j] = zero;
            }
        }
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t at = fb_k_at(16 * j + l16, 32 * kc + 8 * g);
                const fa_f16x8 kh = *reinterpret_cast<const fa_f16x8*>(Kp + at);
                const fa_f16x8 kl = *reinterpret_cast<const fa_f16x8*>(Kp + FB_KPLANE + at);
#pragma unroll
                for (int ps = 0; ps < WIDE_PASSES; ps++) {
                    s[ps][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[ps][kc], s[ps][j], 0, 0, 0);
                    s[ps][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[ps][kc], s[ps][j], 0, 0, 0);
                    s[ps][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[ps][kc], s[ps][j], 0, 0, 0);
                }
            }
        }
        // Scale (2^-ek of the row's position, fq of the token), causal mask,
        // online softmax of the lane's token over its 16 values and its three
        // other lane groups; P^T as the PV B operand of position chunk pc:
        // k slots 0..3 = positions 32 pc + 4g + r (tile j = 2 pc), slots 4..7
        // = 32 pc + 16 + 4g + r (tile j = 2 pc + 1).
        fa_bf16x8 ph[WIDE_PASSES][2], pm[WIDE_PASSES][2];
#pragma unroll
        for (int ps = 0; ps < WIDE_PASSES; ps++) {
            // The scaled, masked scores in place (s[ps] holds them from here).
            float mx = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const fa_floatx4 fk = *reinterpret_cast<const fa_floatx4*>(sk + 16 * j + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t p = b * LH_ATTN_BLOCK + 16 * j + 4 * g + r;
                    const float x = p <= length + tq_of(ps) ? s[ps][j][r] * fk[r] * fq[ps] :
                        -__builtin_inff();
                    s[ps][j][r] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = col4_max(mx);
            // A split can start past a token's last visible position: keep
            // its row empty (no exp of -inf - -inf).
            const float m_new = fmaxf(m[ps], mx);
            const bool empty = m_new == -__builtin_inff();
            const float alpha = empty ? 1.0f : __builtin_amdgcn_exp2f(m[ps] - m_new);
            float sum = 0.0f;
#pragma unroll
            for (int pc = 0; pc < 2; pc++) {
                fa_u32x4 hi, mid;
#pragma unroll
                for (int k = 0; k < 8; k += 2) {
                    const float x0 = s[ps][2 * pc + k / 4][k % 4];
                    const float x1 = s[ps][2 * pc + (k + 1) / 4][(k + 1) % 4];
                    const float e0 = empty ? 0.0f : __builtin_amdgcn_exp2f(x0 - m_new);
                    const float e1 = empty ? 0.0f : __builtin_amdgcn_exp2f(x1 - m_new);
                    sum = sum + e0;
                    sum = sum + e1;
                    uint32_t h0, m0, h1, m1;
                    fb_split2(e0, h0, m0);
                    fb_split2(e1, h1, m1);
                    hi[k / 2] = h0 | (h1 << 16);
                    mid[k / 2] = m0 | (m1 << 16);
                }
                ph[ps][pc] = __builtin_bit_cast(fa_bf16x8, hi);
                pm[ps][pc] = __builtin_bit_cast(fa_bf16x8, mid);
            }
            l[ps] = l[ps] * alpha + col4_sum(sum);
            m[ps] = m_new;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                o[ps][i] = o[ps][i] * alpha;
            }
        }
        // O^T += V^T P^T: A operand of dim tile i: lane (dim 16 i + l16, group
        // g) holds V at positions 32 pc + 4g .. +3 and 32 pc + 16 + 4g .. +3
        // (two 8-byte reads per plane, read once for both passes), the slots
        // of P^T above.
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t d = 16 * i + l16;
#pragma unroll
            for (int pc = 0; pc < 2; pc++) {
                const uint32_t a0 = fb_v_at(d, 32 * pc + 4 * g);
                const uint32_t a1 = fb_v_at(d, 32 * pc + 16 + 4 * g);
                const uint2 h0 = *reinterpret_cast<const uint2*>(Vp + a0);
                const uint2 h1 = *reinterpret_cast<const uint2*>(Vp + a1);
                const uint2 m0 = *reinterpret_cast<const uint2*>(Vp + FB_VPLANE + a0);
                const uint2 m1 = *reinterpret_cast<const uint2*>(Vp + FB_VPLANE + a1);
                const fa_bf16x8 vh = __builtin_bit_cast(fa_bf16x8, fa_u32x4{h0.x, h0.y, h1.x, h1.y});
                const fa_bf16x8 vm = __builtin_bit_cast(fa_bf16x8, fa_u32x4{m0.x, m0.y, m1.x, m1.y});
#pragma unroll
                for (int ps = 0; ps < WIDE_PASSES; ps++) {
                    o[ps][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vm, ph[ps][pc], o[ps][i], 0, 0, 0);
                    o[ps][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pm[ps][pc], o[ps][i], 0, 0, 0);
                    o[ps][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[ps][pc], o[ps][i], 0, 0, 0);
                }
            }
        }
    }
    // Output planes (one split): each token's four query heads of this kv
    // head (512 columns, one K split of the o projection) share one power of
    // two 2^e, their largest magnitude into [2^14, 2^15), before the split
    // into two FP16 planes; xs_scale[t][kv head] = 2^-e. The heads' maxima
    // meet in LDS before any wave leaves.
    // The lane's coordinates again (held across the block loop they would
    // spill: the loop needs every register).
    {
        uint32_t tid_e = threadIdx.x;
        asm volatile("" : "+v"(tid_e));
        lane = tid_e & 63;
        g = lane >> 4;
        l16 = lane & 15;
        const uint32_t wave_e = __builtin_amdgcn_readfirstlane(tid_e >> 6);
#pragma unroll
        for (int ps = 0; ps < WIDE_PASSES; ps++) {
            t0[ps] = tw + FA_TQ * (2 * ps + (wave_e >> 2));
            const uint32_t t0c = t0[ps] < count ? t0[ps] : last_sub;
            last[ps] = (t0c + FA_TQ < count ? t0c + FA_TQ : count) - 1;
        }
        head = kvh * 4 + (wave_e & 3);
        wave = wave_e;
    }
    __shared__ float gmax[WIDE_WG][4];
    if (splits == 1 && xs) {
#pragma unroll
        for (int ps = 0; ps < WIDE_PASSES; ps++) {
            float mr = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                mr = fmaxf(mr, fmaxf(fmaxf(fabsf(o[ps][i].x), fabsf(o[ps][i].y)),
                                     fmaxf(fabsf(o[ps][i].z), fabsf(o[ps][i].w))));
            }
            mr = col4_max(mr) / l[ps];
            if (g == 0) {
                gmax[t0[ps] - tw + l16][wave & 3] = mr;
            }
        }
        __syncthreads();
    }
    // The lane's token and its O^T values: dims 16 i + 4g .. +3.
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
#pragma unroll
    for (int ps = 0; ps < WIDE_PASSES; ps++) {
        const uint32_t t = t0[ps] + l16;
        if (t0[ps] >= count || t > last[ps]) {
            continue;
        }
        if (splits == 1) {
            const float inv = 1.0f / l[ps];
            if (xs) {
                const float* gm = gmax[t0[ps] - tw + l16];
                const int e = row_exponent(fmaxf(fmaxf(gm[0], gm[1]), fmaxf(gm[2], gm[3])));
                if (g == 0 && (wave & 3) == 0) {
                    xs_scale[t * LH_KV_HEADS + kvh] = exp2i(-e);
                }
                const float f = exp2i(e);
                const size_t plane = (size_t)xs_tokens * LH_QUERY;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const fa_floatx4 v = o[ps][i] * (inv * f);
                    store_f16x2_4(xs, plane,
                        xs_at(t, head * LH_HEAD_DIM + 16 * i + 4 * g, LH_QUERY),
                        make_float4(v.x, v.y, v.z, v.w));
                }
            } else {
                float* dst = out + (size_t)t * LH_QUERY + head * LH_HEAD_DIM + 4 * g;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const fa_floatx4 v = o[ps][i] * inv;
                    *reinterpret_cast<float4*>(dst + 16 * i) = make_float4(v.x, v.y, v.z, v.w);
                }
            }
        } else {
            const size_t part = ((size_t)t * LH_HEADS + head) * nbc + z;
            if (g == 0) {
                PM[part] = m[ps];
                PT[part] = l[ps];
            }
            float* dst = PA + part * LH_HEAD_DIM + 4 * g;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                *reinterpret_cast<float4*>(dst + 16 * i) =
                    make_float4(o[ps][i].x, o[ps][i].y, o[ps][i].z, o[ps][i].w);
            }
        }
    }
}

// Merge of k_attn_mfma's KV splits (tolerance path): per (token, head)
// M = max m_z, f_z = exp2(m_z - M) (base-2 maxima), out = (sum f_z O_z) / (sum f_z l_z) with
// the sums in split order. A split whose positions are all masked for the row
// holds m = -inf, l = 0, O = 0 and contributes nothing; split 0 always holds
// position 0, so M is finite. grid (count * 8), block 256: one wave per
// (token, head), lane l owns dims 2l and 2l + 1. Every split's m, l and O
// words are requested before the first is used (index clamped to the last
// split, so MAXP >= parts loads stay in bounds): one memory round trip, where
// a loop over a run-time split count waited for each split's loads in turn.
template <uint32_t MAXP>
__global__ void __launch_bounds__(256)
k_attn_merge(const float* __restrict__ PM, const float* __restrict__ PT,
    const float* __restrict__ PA, uint32_t capacity, uint32_t parts, uint32_t count,
    float* __restrict__ out, uint16_t* __restrict__ xs, uint32_t xs_tokens,
    float* __restrict__ xs_scale)
{
    // Workgroup w merges four heads of one token. When count is a multiple of
    // 128 the workgroups of a 16-token group share an XCD (ids are dealt
    // round-robin to the 8 XCDs), so the plane blocks the group shares
    // (xs_at) are written through one L2.
    uint32_t th = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (count % 128 == 0) {
        const uint32_t w = blockIdx.x, q = w >> 3, hg = q & 7;
        const uint32_t t = (((q >> 7) << 3) + (w & 7)) * 16 + ((q >> 3) & 15);
        th = t * LH_HEADS + hg * 4 + (threadIdx.x >> 6);
    }
    const uint32_t lane = threadIdx.x & 63;
    if (th >= count * LH_HEADS) {
        return;
    }
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    const float* pm = PM + (size_t)th * nbc;
    const float* pt = PT + (size_t)th * nbc;
    const float2* pa = reinterpret_cast<const float2*>(PA + (size_t)th * nbc * LH_HEAD_DIM) + lane;
    float mz[MAXP], tz[MAXP];
    float2 az[MAXP];
#pragma unroll
    for (uint32_t z = 0; z < MAXP; z++) {
        const uint32_t c = z < parts ? z : parts - 1;
        mz[z] = pm[c];
        tz[z] = pt[c];
        az[z] = pa[(size_t)c * (LH_HEAD_DIM / 2)];
    }
    float M = -__builtin_inff();
#pragma unroll
    for (uint32_t z = 0; z < MAXP; z++) {
        if (z < parts) {
            M = fmaxf(M, mz[z]);
        }
    }
    float2 A = make_float2(0.0f, 0.0f);
    float T = 0.0f;
#pragma unroll
    for (uint32_t z = 0; z < MAXP; z++) {
        if (z < parts) {
            const float f = __builtin_amdgcn_exp2f(mz[z] - M);
            A.x = __builtin_fmaf(f, az[z].x, A.x);
            A.y = __builtin_fmaf(f, az[z].y, A.y);
            T = __builtin_fmaf(f, tz[z], T);
        }
    }
    const uint32_t t = th / LH_HEADS, h = th % LH_HEADS;
    const size_t at = (size_t)t * LH_QUERY + h * LH_HEAD_DIM + 2 * lane;
    if (xs) {
        // The workgroup's waves are the four query heads of one kv head for
        // one token: 512 columns, one K split of the o projection. They share
        // one power of two 2^e (their largest magnitude into [2^14, 2^15))
        // before the split into two FP16 planes; xs_scale[t][kv head] = 2^-e,
        // which the o projection's GEMM applies to that split's products. The
        // lane's two columns are adjacent in the plane: one 4-byte store per
        // plane.
        __shared__ float gmax[4];
        const float vx = A.x / T, vy = A.y / T;
        const float mw = wave_max64(fmaxf(fabsf(vx), fabsf(vy)));
        if (lane == 0) {
            gmax[threadIdx.x >> 6] = mw;
        }
        __syncthreads();
        const int e = row_exponent(fmaxf(fmaxf(gmax[0], gmax[1]), fmaxf(gmax[2], gmax[3])));
        if (threadIdx.x == 0) {
            xs_scale[t * LH_KV_HEADS + h / 4] = exp2i(-e);
        }
        const float f = exp2i(e);
        store_f16x2_2(xs, (size_t)xs_tokens * LH_QUERY,
            xs_at(t, h * LH_HEAD_DIM + 2 * lane, LH_QUERY), vx * f, vy * f);
    } else {
        *reinterpret_cast<float2*>(out + at) = make_float2(A.x / T, A.y / T);
    }
}

}  // namespace lh

extern "C" int lh_launch_attention_mfma(const float* q, const float* kcache_layer,
    const float* vcache_layer, const lh_step_params* params, uint32_t length, uint32_t count,
    uint32_t capacity, float* PM, float* PT, float* PA, float* out, uint16_t* xs, uint32_t xs_tokens,
    float* xs_scale, hipStream_t s)
{
    if (!count || capacity % LH_ATTN_BLOCK || length + count > capacity ||
        (xs && (xs_tokens < count || !xs_scale))) {
        return -1;
    }
    // KV splits so that about 256 workgroups run (one per CU), at most one
    // per block of the longest tile (a 256-token chunk with no prefix runs 4
    // splits of one block: measured 2.7 us per layer faster than 2 splits of
    // two blocks, the merge included).
    const bool wide = length >= lh::WIDE_MIN_LENGTH && count >= lh::WIDE_MIN_COUNT;
    const uint32_t per_wg = wide ? lh::WIDE_WG : 2 * lh::FA_TQ;
    const uint32_t tiles = (count + per_wg - 1) / per_wg;
    const uint32_t nb = (length + count + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    uint32_t splits = 256 / (tiles * LH_KV_HEADS);
    const uint32_t by_length = nb;
    splits = splits < by_length ? splits : by_length;
    splits = splits ? splits : 1;
    if (wide) {
        hipLaunchKernelGGL(lh::k_attn_mfma_wide, dim3(tiles * LH_KV_HEADS * splits), dim3(512), 0,
            s, q, kcache_layer, vcache_layer, length, count, capacity, PM, PT, PA, out, xs,
            xs_tokens, xs_scale);
    } else {
        hipLaunchKernelGGL(lh::k_attn_mfma, dim3(tiles * LH_KV_HEADS * splits), dim3(512), 0, s,
            q, kcache_layer, vcache_layer, length, count, capacity, PM, PT, PA, out, xs,
            xs_tokens, xs_scale);
    }
    if (splits > 1) {
        static_assert(256 / LH_KV_HEADS <= 32, "at most 32 splits");
        const dim3 grid(count * LH_HEADS / 4);
        if (splits <= 4) {
            hipLaunchKernelGGL(lh::k_attn_merge<4>, grid, dim3(256), 0, s, PM, PT, PA, capacity,
                splits, count, out, xs, xs_tokens, xs_scale);
        } else if (splits <= 8) {
            hipLaunchKernelGGL(lh::k_attn_merge<8>, grid, dim3(256), 0, s, PM, PT, PA, capacity,
                splits, count, out, xs, xs_tokens, xs_scale);
        } else if (splits <= 16) {
            hipLaunchKernelGGL(lh::k_attn_merge<16>, grid, dim3(256), 0, s, PM, PT, PA, capacity,
                splits, count, out, xs, xs_tokens, xs_scale);
        } else {
            hipLaunchKernelGGL(lh::k_attn_merge<32>, grid, dim3(256), 0, s, PM, PT, PA, capacity,
                splits, count, out, xs, xs_tokens, xs_scale);
        }
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
