// Decode-attention block workgroup (src/metal_kernels.metal:80-132 computes the
// same softmax(q.k/sqrt(128)).V with one SIMD group walking every position),
// shared by the attention kernels (attention.hip) and the chained
// q|k|v + attention kernel (matvec.hip). For block b, kv head kvh, token t,
// the four query heads sharing the kv head, over the block's valid positions p:
//     c_i  = chain over d in [32i, 32i+32) of fma(q_d, k_pd)   (i = 0..3)
//     s_p  = fl(((c_0 + c_1) + (c_2 + c_3)) * 1/sqrt(128))
//     m_b  = max_p s_p,  e_p = exp(s_p - m_b),  T_b = 64-lane tree of e,
//     A_b[d] = chain_p fma(e_p, v_pd)  (from 0, position order).
// The combine (k_attn_combine, or the last-arriving workgroup of the group):
// M = max_b m_b, f_b = exp(m_b - M); groups of 8 consecutive blocks chain
// S_g[d] = fma(f_b, A_b[d], .) and U_g = fma(f_b, T_b, .) from 0;
// A = S_0 + S_1 + ..., T = U_0 + U_1 + ... left to right; out[d] = A[d] / T.
#pragma once

#include "lh_device.h"

namespace lh {

constexpr uint32_t GROUP = 8;     // blocks chained per combine group

// Arrival words: eight 7-bit fields, field x counting arrivals from XCD x.
// Each word has a 256-byte line of its own (ARRIVE_STRIDE words apart):
// atomics on one line serialize.
constexpr uint32_t ARRIVE_FIELD = 7;
constexpr uint32_t ARRIVE_STRIDE = LH_ARRIVE_STRIDE;

// Workgroups of the q|k|v projection per kv head in the chained kernel (384
// RoPE pairs of six each: four query heads, the key head, the value head).
constexpr uint32_t QKV_PRODUCERS = 64;

// Polls of the producers' flags before a chained block gives up (each poll
// reads the 64 flags from L2 after a short sleep, so about a second).
constexpr uint32_t SPIN_LIMIT = 1u << 21;

// A producer's flag: the launch's epoch and the XCD it ran on.
__device__ __forceinline__ unsigned long long producer_flag(unsigned long long epoch,
    uint32_t xcc)
{
    return epoch << 8 | xcc;
}

// Largest block count a fused launch combines: groups of eight blocks, the
// even ones on lanes 0..31 and the odd ones on lanes 32..63 of the combining
// workgroup's waves.
#ifndef LH_ATTN_FUSED_MAX
#define LH_ATTN_FUSED_MAX 16
#endif
constexpr uint32_t FUSED_MAX_BLOCKS = LH_ATTN_FUSED_MAX;

__device__ __forceinline__ uint32_t xcc_id()
{
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 3)" : "=s"(xcc));
    return xcc;
}

__device__ __forceinline__ uint32_t arrivals(unsigned long long word)
{
    uint32_t total = 0;
#pragma unroll
    for (uint32_t x = 0; x < 8; x++) {
        total += (uint32_t)(word >> (ARRIVE_FIELD * x)) & ((1u << ARRIVE_FIELD) - 1);
    }
    return total;
}

constexpr uint32_t ROUND = 256;   // blocks per combine round (32 groups)

struct CombineShared {
    float wmax[4];
    float fs[ROUND], ts[ROUND];
    float4 sg[ROUND / GROUP][8];
    float ug[ROUND / GROUP];
};

// The combine of head h, dimension quarter qd, token t over the n positions
// (0..n-1): thread (c = tid & 7, s = tid >> 3) owns dims 32qd + 4c .. +3 of
// group s of each 256-block round; every quarter recomputes M and the block
// factors, so the four workgroups of a head are independent. Bitwise the
// schedule above (the dims never mix; groups start at multiples of 8 from
// block 0 and add left to right across rounds).
__device__ __forceinline__ void attn_combine(const float* __restrict__ PM,
    const float* __restrict__ PT, const float* __restrict__ PA, uint32_t n, uint32_t capacity,
    uint32_t h, uint32_t qd, uint32_t t, float* __restrict__ out, CombineShared& sh)
{
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    const size_t th = (size_t)t * LH_HEADS + h;
    const float* pm = PM + th * nbc;
    const float* pt = PT + th * nbc;
    const uint32_t tid = threadIdx.x, c = tid & 7, s = tid >> 3;
    const float4* pa = reinterpret_cast<const float4*>(PA + th * nbc * LH_HEAD_DIM) + 8 * qd + c;
    // A round's partial loads are clamped to the capacity, not to the valid
    // block count, so the first round's issue before the step record is
    // read; rows past the valid count never enter arithmetic.
    float4 a[GROUP];
    float m_own, t_own;
    auto load_round = [&](uint32_t r0) {
#pragma unroll
        for (uint32_t k = 0; k < GROUP; k++) {
            const uint32_t bb = r0 + s * GROUP + k;
            a[k] = pa[(size_t)(bb < nbc ? bb : nbc - 1) * (LH_HEAD_DIM / 4)];
        }
        const uint32_t bb = r0 + tid < nbc ? r0 + tid : nbc - 1;
        m_own = pm[bb];
        t_own = pt[bb];
    };
    load_round(0);
    const uint32_t nb = (n + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    float M = tid < nb ? m_own : -__builtin_inff();
    for (uint32_t j = tid + ROUND; j < nb; j += ROUND) {
        M = fmaxf(M, pm[j]);
    }
    M = wave_max64(M);
    if ((tid & 63) == 0) {
        sh.wmax[tid >> 6] = M;
    }
    __syncthreads();
    M = fmaxf(fmaxf(sh.wmax[0], sh.wmax[1]), fmaxf(sh.wmax[2], sh.wmax[3]));
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    float T = 0.0f;
    for (uint32_t r0 = 0; r0 < nb; r0 += ROUND) {
        if (r0) {
            load_round(r0);
        }
        {
            const uint32_t bb = r0 + tid;
            sh.fs[tid] = bb < nb ? expf_cw(m_own - M) : 0.0f;
            sh.ts[tid] = bb < nb ? t_own : 0.0f;
        }
        __syncthreads();
        float4 Sg = make_float4(0.f, 0.f, 0.f, 0.f);
        float Ug = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < GROUP; k++) {
            if (r0 + s * GROUP + k < nb) {
                const float f = sh.fs[s * GROUP + k];
                Sg.x = __builtin_fmaf(f, a[k].x, Sg.x);
                Sg.y = __builtin_fmaf(f, a[k].y, Sg.y);
                Sg.z = __builtin_fmaf(f, a[k].z, Sg.z);
                Sg.w = __builtin_fmaf(f, a[k].w, Sg.w);
                Ug = __builtin_fmaf(f, sh.ts[s * GROUP + k], Ug);
            }
        }
        sh.sg[s][c] = Sg;
        if (c == 0) {
            sh.ug[s] = Ug;
        }
        __syncthreads();
        if (tid < 8) {
            for (uint32_t g = 0; g < ROUND / GROUP && r0 + g * GROUP < nb; g++) {
                const float4 v = sh.sg[g][c];
                if (r0 == 0 && g == 0) {
                    A = v;
                    T = sh.ug[0];
                } else {
                    A.x = A.x + v.x;
                    A.y = A.y + v.y;
                    A.z = A.z + v.z;
                    A.w = A.w + v.w;
                    T = T + sh.ug[g];
                }
            }
        }
        __syncthreads();
    }
    if (tid < 8) {
        reinterpret_cast<float4*>(out + (size_t)t * LH_QUERY + h * LH_HEAD_DIM)[8 * qd + c] =
            make_float4(A.x / T, A.y / T, A.z / T, A.w / T);
    }
}

// Combiner workgroup of a one-token launch whose blocks (kv head h / 4, on
// this workgroup's XCD) each store bflags[b] = epoch once their partials are
// acknowledged: waits, at most `spins` polls (volatile loads, which miss the
// L1), until the first nb flags carry `want`, then combines from the XCD's L2
// (no workgroup loaded the partials before in this launch, so this CU's L1
// holds none of their lines). If it gives up it writes NaN. want equals the
// launch's epoch except where the test build forces the give-up.
__device__ __forceinline__ void attn_combiner(const float* __restrict__ PM,
    const float* __restrict__ PT, const float* __restrict__ PA,
    const lh_step_params* __restrict__ params, uint32_t capacity,
    const unsigned long long* bflags, unsigned long long want, uint32_t spins, uint32_t h,
    uint32_t qd, float* __restrict__ out, CombineShared& sh)
{
    const uint32_t n = params->length + 1;
    const uint32_t nb = (n + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    const volatile unsigned long long* f = bflags;
    bool ready = false;
    for (uint32_t spin = 0; spin < spins; spin++) {
        int mine = 1;
        for (uint32_t b = threadIdx.x; b < nb; b += 256) {
            mine &= f[b] == want;
        }
        if (__syncthreads_and(mine)) {
            ready = true;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (!ready) {
        if (threadIdx.x < 8) {
            const float nan = __builtin_nanf("");
            reinterpret_cast<float4*>(out + h * LH_HEAD_DIM)[8 * qd + threadIdx.x] =
                make_float4(nan, nan, nan, nan);
        }
        return;
    }
    attn_combine(PM, PT, PA, n, capacity, h, qd, 0, out, sh);
}

// LDS of one block workgroup: one 32 KiB tile region holds K for the scores,
// then V for the P.V chains.
struct AttnShared {
    float4 T[LH_ATTN_BLOCK * LH_HEAD_DIM / 4];
    float4 qs[4][LH_HEAD_DIM / 4];
    float S[4][LH_ATTN_BLOCK];
    uint32_t verdict;
};

// What follows a block's partials. NONE: nothing (k_attn_combine follows).
// COMBINE: the last workgroup of the (token, kv head) group to arrive
// combines. FLAG (one token): once its partial stores are acknowledged the
// block stores bflags[b] = epoch for the combiners of its kv head.
enum AttnTail { TAIL_NONE = 0, TAIL_COMBINE = 1, TAIL_FLAG = 2 };

// The hand-off of a one-launch group. Each workgroup waits until its partial
// stores are acknowledged (the vector L1 writes through, so they are in its
// XCD's L2), then adds its arrival to its XCD's field of the group's word;
// the workgroup that brings the fields' total to nblk returns the word to
// zero for the next launch and combines the group's four heads from the
// partials, which its XCD's L2 holds. That holds only when the whole group ran on its XCD:
// otherwise the word shows it, and the combine writes NaN (never a silently
// stale result). The arithmetic is k_attn_combine's, operation for operation.
template <AttnTail TAIL>
__device__ __forceinline__ void attn_block_tail(const float* __restrict__ PM,
    const float* __restrict__ PT, const float* __restrict__ PA,
    unsigned long long* __restrict__ arrive, float* __restrict__ out, uint32_t t, uint32_t kvh,
    uint32_t nblk, uint32_t nbc, uint32_t n, uint32_t& verdict)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    unsigned long long* slot = arrive + ((size_t)t * LH_KV_HEADS + kvh) * ARRIVE_STRIDE;
    if (tid == 0) {
        const uint32_t xcc = xcc_id();
        const unsigned long long inc = 1ull << (ARRIVE_FIELD * xcc);
        const unsigned long long now =
            __hip_atomic_fetch_add(slot, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
        verdict = arrivals(now) != nblk ? 0u
            : now == (unsigned long long)nblk << (ARRIVE_FIELD * xcc) ? 1u : 2u;
    }
    __syncthreads();
    const uint32_t seen = verdict;
    if (!seen) {
        return;
    }
    if (tid == 0) {
        __hip_atomic_exchange(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // The partials come from L2: no workgroup loaded them before in this
    // launch, so this CU's L1 holds none of their lines.
    const uint32_t nb = (n + LH_ATTN_BLOCK - 1) / LH_ATTN_BLOCK;
    const size_t th = (size_t)t * LH_HEADS + kvh * 4 + wave;
    // Wave w combines head kvh * 4 + w alone: lane = (group gp = lane / 32,
    // dims 4c .. 4c + 3 with c = lane % 32). Every load is issued first (the
    // block maxima and sums with lane = block; the lane's four dims of its
    // groups' blocks, rows past nb clamped). A lane takes its blocks' factors
    // and sums from the lanes that hold them (ds_bpermute), chains its
    // groups, and the odd groups' sums reach lanes 0..31 by a 32-lane swap.
    // Blocks past nb are skipped by selects, so no branch follows the loads.
    const uint32_t c = lane & 31, gp = lane >> 5;
    constexpr uint32_t J = FUSED_MAX_BLOCKS / (2 * GROUP);   // groups per half-wave
    const float* pm = PM + th * nbc;
    const float* pt = PT + th * nbc;
    const float mb = lane < nb ? pm[lane] : -__builtin_inff();
    const float tb = lane < nb ? pt[lane] : 0.0f;
    const float4* pa = reinterpret_cast<const float4*>(PA + th * nbc * LH_HEAD_DIM) + c;
    float4 a[J][GROUP];
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
#pragma unroll
        for (uint32_t k = 0; k < GROUP; k++) {
            const uint32_t bb = (gp + 2 * j) * GROUP + k;
            a[j][k] = pa[(size_t)(bb < nb ? bb : nb - 1) * (LH_HEAD_DIM / 4)];
        }
    }
    const float M = wave_max64(mb);
    const int fl = __float_as_int(expf_cw(mb - M));
    auto upper = [](float v) {   // lane l < 32 receives lane l + 32's v
        const uint32_t u = __float_as_uint(v);
        return __uint_as_float(__builtin_amdgcn_permlane32_swap(u, u, false, false)[1]);
    };
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    float T = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        float4 S = make_float4(0.f, 0.f, 0.f, 0.f);
        float U = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < GROUP; k++) {
            const uint32_t bb = (gp + 2 * j) * GROUP + k;
            const float fb = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * bb, fl));
            const float tk = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * bb, __float_as_int(tb)));
            const bool in = bb < nb;
            S.x = in ? __builtin_fmaf(fb, a[j][k].x, S.x) : S.x;
            S.y = in ? __builtin_fmaf(fb, a[j][k].y, S.y) : S.y;
            S.z = in ? __builtin_fmaf(fb, a[j][k].z, S.z) : S.z;
            S.w = in ? __builtin_fmaf(fb, a[j][k].w, S.w) : S.w;
            U = in ? __builtin_fmaf(fb, tk, U) : U;
        }
        // Lanes 0..31 add group 2j, then group 2j + 1 (from lane + 32), left
        // to right after the groups before them.
        const float4 S1 = make_float4(upper(S.x), upper(S.y), upper(S.z), upper(S.w));
        const float U1 = upper(U);
        const bool in0 = 2 * j * GROUP < nb, in1 = (2 * j + 1) * GROUP < nb;
        if (j == 0) {
            A = S;
            T = U;
        } else if (in0) {
            A = make_float4(A.x + S.x, A.y + S.y, A.z + S.z, A.w + S.w);
            T = T + U;
        }
        if (in1) {
            A = make_float4(A.x + S1.x, A.y + S1.y, A.z + S1.z, A.w + S1.w);
            T = T + U1;
        }
    }
    if (lane < 32) {
        float4 o = make_float4(A.x / T, A.y / T, A.z / T, A.w / T);
        if (seen != 1) {
            o = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                __builtin_nanf(""));
        }
        reinterpret_cast<float4*>(out + (size_t)t * LH_QUERY + (kvh * 4 + wave) * LH_HEAD_DIM)[c] = o;
    }
}

// One block workgroup (256 threads: wave w covers positions 16w..16w+15 for
// the scores, then head kvh * 4 + w for the softmax and P.V chains).
// CHAINED (one decode token, t = 0): q and the current position's K and V rows
// are written in the same launch by the q|k|v workgroups of kv head kvh,
// each of which then stores its flag (this launch's epoch and its XCD) in
// flags[0..63]; the block issues its K/V tile loads, then waits (at most
// `spins` polls) until all QKV_PRODUCERS flags carry the epoch `want` and its
// own XCD, before loading q and patching the current row. A block that gives
// up writes NaN partials (want differs from the producers' epoch only when
// the test build forces that path).
template <AttnTail TAIL, bool CHAINED>
__device__ __forceinline__ void attn_block(const float* __restrict__ q,
    const float* __restrict__ kcache, const float* __restrict__ vcache,
    const lh_step_params* __restrict__ params, uint32_t capacity, uint32_t nblk,
    float* __restrict__ PM, float* __restrict__ PT, float* __restrict__ PA,
    unsigned long long* __restrict__ arrive, const unsigned long long* flags,
    unsigned long long* bflags, unsigned long long epoch, unsigned long long want, uint32_t spins,
    float* __restrict__ out, uint32_t b, uint32_t kvh, uint32_t t, AttnShared& sh)
{
    float4* T = sh.T;
    const uint64_t tile = lh_kv_index(capacity, 0, kvh, (uint64_t)b * LH_ATTN_BLOCK);
    const float4* kb = reinterpret_cast<const float4*>(kcache + tile);
    const float4* vb = reinterpret_cast<const float4*>(vcache + tile);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float4* qrow = reinterpret_cast<const float4*>(
        q + (size_t)t * LH_QUERY + kvh * 4 * LH_HEAD_DIM) + tid;
    // The tile loads do not wait for the step record: the launch grid covers
    // ceil((length + count) / 64) blocks of a capacity that is a multiple of
    // 64, so all 64 rows are in bounds; rows past the valid count are never
    // used in arithmetic.
    // Issue order: the four query rows (2 KiB) and the K tile go to LDS by
    // direct loads, then the V tile to registers. Vector loads complete in
    // issue order, so the scores wait for q and K only (an explicit vmcnt(8))
    // and V lands while they run.
    if (!CHAINED && tid < 128) {
        __builtin_amdgcn_global_load_lds(qrow, reinterpret_cast<float4*>(sh.qs) + 64 * wave, 16,
            0, 0);
    }
    // K: wave w covers positions 16w..16w+15; lane = 4 * (position - 16w) +
    // quarter. The tile's word order (lh_ktile_word) makes load i of wave w
    // the contiguous 1 KiB of words (8w + i) * 64 .. +63, written to LDS in
    // the same order, so lane l later reads word (8w + i) * 64 + l.
    const uint32_t p = 16 * wave + (lane >> 2), quarter = lane & 3;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        __builtin_amdgcn_global_load_lds(kb + (wave * 8 + i) * 64 + lane,
            T + (wave * 8 + i) * 64, 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);   // V's loads stay behind K's
    // (A native vector type: a float4 struct copy is a memcpy that, with the
    // intrinsics around it, stays in scratch memory.)
    typedef float v4f __attribute__((ext_vector_type(4)));
    v4f vr[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        vr[i] = reinterpret_cast<const v4f*>(vb)[tid + 256 * i];   // row (tid + 256 i) >> 5
    }
    // No early exit for blocks past token t's last position (multi-token
    // steps): a branch here lets the compiler sink the V loads below it. Such
    // a workgroup runs with valid = 0 and writes nothing.
    const uint32_t length = params->length;
    const uint32_t n = length + t + 1;
    const uint32_t nbc = capacity / LH_ATTN_BLOCK;
    const uint32_t rest = n > b * LH_ATTN_BLOCK ? n - b * LH_ATTN_BLOCK : 0;
    const uint32_t valid = rest < LH_ATTN_BLOCK ? rest : LH_ATTN_BLOCK;
    bool fed = true;
    if constexpr (CHAINED) {
        // The tiles land before the wait (the memory clobber keeps the loads
        // above it), then wave 0 polls the 64 flags. Volatile loads carry the
        // sc0 sc1 policy, which misses the CU's L1 (a plain load would keep
        // hitting the line its first poll brought in) and is served by the
        // XCD's L2, where the producers' stores land.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (wave == 0) {
            const unsigned long long flag = producer_flag(want, xcc_id());
            const volatile unsigned long long* f = flags + lane;
            bool ready = false;
            for (uint32_t spin = 0; spin < spins && !ready; spin++) {
                ready = __builtin_amdgcn_ballot_w64(*f != flag) == 0;
                if (!ready) {
                    __builtin_amdgcn_s_sleep(2);
                }
            }
            if (lane == 0) {
                sh.verdict = ready;
            }
        }
        __syncthreads();
        fed = sh.verdict != 0;
        // The current row's reloads are volatile: their sc0 sc1 loads miss
        // this CU's L1, which may hold the row's line from the tile loads
        // above, and the compiler cannot reuse the values loaded there from
        // the same (read-only, unaliased) addresses. q was never loaded
        // before the wait on this CU in this launch (the L1 starts each
        // launch empty), so its direct loads come from L2.
        const volatile v4f* kfresh = reinterpret_cast<const volatile v4f*>(kb);
        const volatile v4f* vfresh = reinterpret_cast<const volatile v4f*>(vb);
        if (tid < 128) {
            __builtin_amdgcn_global_load_lds(qrow, reinterpret_cast<float4*>(sh.qs) + 64 * wave,
                16, 0, 0);
        }
        const uint32_t pc = length - b * LH_ATTN_BLOCK;   // current row, if in this block
        if (pc < LH_ATTN_BLOCK) {
            if (tid < 32) {   // K: word (pc/16 * 8 + i) * 64 + (pc%16) * 4 + quarter
                const uint32_t word = ((pc >> 4) * 8 + (tid >> 2)) * 64 + (pc & 15) * 4 + (tid & 3);
                reinterpret_cast<v4f*>(T)[word] = kfresh[word];
            }
            if ((tid >> 5) == (pc & 7)) {   // V: row pc is vr[pc / 8] of these 32 threads
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if ((uint32_t)i == pc >> 3) {
                        vr[i] = vfresh[tid + 256 * i];
                    }
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    } else {
        // s_waitcnt vmcnt(8), then a bare barrier: __syncthreads()'s workgroup
        // fence would also wait for the V loads.
        __builtin_amdgcn_s_waitcnt(0x0f78);
        __builtin_amdgcn_s_barrier();
    }
    // The K and q words of step i + 1 are read while step i's products run.
    float c[4] = {0.f, 0.f, 0.f, 0.f};
    float4 k = T[wave * 8 * 64 + lane];
    float4 qq[4];
#pragma unroll
    for (int hh = 0; hh < 4; hh++) {
        qq[hh] = sh.qs[hh][8 * quarter];
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 kn, qn[4];
        if (i < 7) {
            kn = T[(wave * 8 + i + 1) * 64 + lane];
#pragma unroll
            for (int hh = 0; hh < 4; hh++) {
                qn[hh] = sh.qs[hh][8 * quarter + i + 1];
            }
        }
#pragma unroll
        for (int hh = 0; hh < 4; hh++) {
            c[hh] = __builtin_fmaf(qq[hh].x, k.x, c[hh]);
            c[hh] = __builtin_fmaf(qq[hh].y, k.y, c[hh]);
            c[hh] = __builtin_fmaf(qq[hh].z, k.z, c[hh]);
            c[hh] = __builtin_fmaf(qq[hh].w, k.w, c[hh]);
        }
        if (i < 7) {
            k = kn;
#pragma unroll
            for (int hh = 0; hh < 4; hh++) {
                qq[hh] = qn[hh];
            }
        }
        // Each step's four chains complete here (an empty asm that reads and
        // writes them), so the compiler cannot defer three of them past the
        // loop with every step's operands held in registers.
        asm volatile("" : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]));
    }
#pragma unroll
    for (int hh = 0; hh < 4; hh++) {
        const float v = quad_sum(c[hh]);  // (c0 + c1) + (c2 + c3)
        if (quarter == 0 && p < valid) {
            sh.S[hh][p] = v * LH_SCORE_SCALE;
        }
    }
    __syncthreads();   // every read of K is done; S holds the scores
#pragma unroll
    for (int i = 0; i < 8; i++) {
        reinterpret_cast<v4f*>(T)[tid + 256 * i] = vr[i];
    }
    __syncthreads();
    // Wave w = head kvh*4 + w from here on; lane = position. e_j reaches every
    // lane by a scalar read of lane j.
    const float s = lane < valid ? sh.S[wave][lane] : -__builtin_inff();
    const float m = wave_max64(s);
    const float e = lane < valid ? expf_cw(s - m) : 0.0f;
    const float total = wave_tree64(e);
    const uint32_t d0 = 2 * lane;
    float a0 = 0.0f, a1 = 0.0f;
    const float* vt = reinterpret_cast<const float*>(T) + d0;
    if (valid == LH_ATTN_BLOCK) {
#pragma unroll
        for (uint32_t j = 0; j < LH_ATTN_BLOCK; j++) {
            const float ej = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
            const float2 v = *reinterpret_cast<const float2*>(vt + j * LH_HEAD_DIM);
            a0 = __builtin_fmaf(ej, v.x, a0);
            a1 = __builtin_fmaf(ej, v.y, a1);
        }
    } else {
        for (uint32_t j = 0; j < valid; j++) {
            const float ej = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
            const float2 v = *reinterpret_cast<const float2*>(vt + j * LH_HEAD_DIM);
            a0 = __builtin_fmaf(ej, v.x, a0);
            a1 = __builtin_fmaf(ej, v.y, a1);
        }
    }
    const size_t th = (size_t)t * LH_HEADS + kvh * 4 + wave;
    if (valid) {
        const float nan = __builtin_nanf("");
        if (lane == 0) {
            PM[th * nbc + b] = fed ? m : nan;
            PT[th * nbc + b] = fed ? total : nan;
        }
        *reinterpret_cast<float2*>(PA + (th * nbc + b) * LH_HEAD_DIM + d0) =
            fed ? make_float2(a0, a1) : make_float2(nan, nan);
    }
    if constexpr (TAIL == TAIL_COMBINE) {
        attn_block_tail<TAIL>(PM, PT, PA, arrive, out, t, kvh, nblk, nbc, n, sh.verdict);
    }
    if constexpr (TAIL == TAIL_FLAG) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            bflags[kvh * nbc + b] = epoch;
        }
    }
}

}  // namespace lh
