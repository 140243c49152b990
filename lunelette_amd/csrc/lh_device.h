// Device helpers shared by the gfx950 kernels: weight element decode, the
// fixed 64-lane reduction tree, and the Cody-Waite exp that the CPU oracle
// restates bit for bit. Every reduction order used here is part of the
// canonical schedule described in lh_schedule.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lh_schedule.h"

namespace lh {

// E4M3FN -> FP32. gfx950's v_cvt_pk_f32_fp8 decodes the OCP E4M3FN encoding
// (bias 7, subnormals f*2^-9, 0x7f/0xff NaN), matching src/safetensors.c:505-519
// for every finite code; the all-256-code check runs in the GPU tests.
__device__ __forceinline__ void fp8x4_to_f32(uint32_t packed, float out[4])
{
    auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(packed, false);
    auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(packed, true);
    out[0] = lo[0];
    out[1] = lo[1];
    out[2] = hi[0];
    out[3] = hi[1];
}

// Table decode (the COMPACT_FP8_LOOKUP strategy): unscaled E4M3FN values,
// built once per launch into LDS from the arithmetic decode, so both
// strategies are bitwise identical by construction.
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16)
{
    return __uint_as_float(bits16 << 16);
}

// Pairwise halving tree over the 64 lanes of a wave: after the step with
// distance s, lane i < s holds v_i + v_{i+s}; lane 0 returns the total.
// Distances 32 and 16 use gfx950's v_permlane32_swap / v_permlane16_swap,
// 8..1 a DPP row_shl (lane i reads lane i+s inside its 16-lane row), so the
// whole tree stays in VALU; only lane 0's value is meaningful.
__device__ __forceinline__ float dpp_row_shl(float v, int s)
{
    const int iv = __float_as_int(v);
    int r;
    switch (s) {
    case 8: r = __builtin_amdgcn_update_dpp(0, iv, 0x108, 0xf, 0xf, false); break;
    case 4: r = __builtin_amdgcn_update_dpp(0, iv, 0x104, 0xf, 0xf, false); break;
    case 2: r = __builtin_amdgcn_update_dpp(0, iv, 0x102, 0xf, 0xf, false); break;
    default: r = __builtin_amdgcn_update_dpp(0, iv, 0x101, 0xf, 0xf, false); break;
    }
    return __int_as_float(r);
}

__device__ __forceinline__ float wave_tree64(float v)
{
    const uint32_t u = __float_as_uint(v);
    const auto p32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = v + __uint_as_float(p32[1]);
    const uint32_t w = __float_as_uint(v);
    const auto p16 = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    v = v + __uint_as_float(p16[1]);
    v = v + dpp_row_shl(v, 8);
    v = v + dpp_row_shl(v, 4);
    v = v + dpp_row_shl(v, 2);
    v = v + dpp_row_shl(v, 1);
    return v;
}

// Lane 0's value to every lane (scalar read; lane 0 is active in every caller).
__device__ __forceinline__ float wave_lane0(float v)
{
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Maximum over the 64 lanes, returned in every lane: the halving tree above
// with fmaxf, then lane 0's value broadcast. The maximum does not depend on
// the pairing (NaN lanes are ignored unless all are NaN); only the sign of a
// zero maximum may differ from another pairing, and every use subtracts it.
__device__ __forceinline__ float wave_max64(float v)
{
    const uint32_t u = __float_as_uint(v);
    const auto p32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = fmaxf(v, __uint_as_float(p32[1]));
    const uint32_t w = __float_as_uint(v);
    const auto p16 = __builtin_amdgcn_permlane16_swap(w, w, false, false);
    v = fmaxf(v, __uint_as_float(p16[1]));
    v = fmaxf(v, dpp_row_shl(v, 8));
    v = fmaxf(v, dpp_row_shl(v, 4));
    v = fmaxf(v, dpp_row_shl(v, 2));
    v = fmaxf(v, dpp_row_shl(v, 1));
    return wave_lane0(v);
}

// (c0 + c1) + (c2 + c3) over the four lanes of each aligned quad, in every
// lane of the quad (IEEE addition is commutative, so lane q's c_q + c_(q^1)
// has the bits of lane 0's c0 + c1): two DPP quad permutations.
__device__ __forceinline__ float quad_sum(float c)
{
    const float v = c + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(c), 0xB1, 0xf, 0xf,
        false));  // quad_perm [1,0,3,2]
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf,
        false));  // quad_perm [2,3,0,1]
}

// exp(x): Cody & Waite additive range reduction (Cody, Waite, "Software
// Manual for the Elementary Functions", 1980) with ln2 split so k*ln2_hi is
// exact, then the degree-7 Taylor polynomial of e^r by Horner's rule with
// fused multiply-adds, then ldexp. Below the normal range flushes to +0,
// above ln(FLT_MAX) gives +inf.
__device__ __forceinline__ float expf_cw(float x)
{
    if (x != x) {
        return x;
    }
    if (x > 88.72283935546875f) {
        return __builtin_inff();
    }
    if (x < -87.33654022216796875f) {
        return 0.0f;
    }
    float k = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(k, -0.693145751953125f, x);
    r = __builtin_fmaf(k, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412698412698412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

// SiLU v/(1+exp(-v)) (src/metal_kernels.metal:55-56) with the division
// correctly rounded (hipcc's default fp32 division).
__device__ __forceinline__ float silu(float v)
{
    return v / (1.0f + expf_cw(-v));
}

// Element (token t, column c) of one activation plane of the matrix-core
// GEMMs, for a K-column plane (K a multiple of 64). The plane is tiled so
// that each MFMA A fragment is one contiguous 1 KiB block: 16 tokens x one
// 64-column stage x one 8-column half h of each 16-column group g. Block
// ((t / 16) * (K / 64) + c / 64) * 2 + h holds, at 16-byte word
// g * 16 + t % 16, the eight columns 16g + 8h .. +7 of token t, so lane
// l = 16g + t % 16 of a wave reads its fragment with one 16-byte load at
// l * 16 bytes. Four columns c .. c+3 with c % 4 == 0 stay contiguous.
__device__ __forceinline__ size_t xs_at(uint32_t t, uint32_t c, uint32_t K)
{
    return ((((size_t)(t >> 4) * (K >> 6) + (c >> 6)) * 2 + ((c >> 3) & 1)) << 9) +
        ((((c >> 4) & 3) * 16 + (t & 15)) << 3) + (c & 7);
}

// Token of workgroup w in a launch of one workgroup per token row (count
// rows) that writes activation planes: when count is a multiple of 128,
// every 16-token group goes to one XCD (workgroup ids are dealt round-robin
// to the 8 XCDs), so the plane blocks it shares (xs_at) are written through
// one L2; otherwise token w.
__device__ __forceinline__ uint32_t xs_token(uint32_t w, uint32_t count)
{
    if (count % 128) {
        return w;
    }
    const uint32_t q = w >> 3;
    return (((q >> 4) << 3) + (w & 7)) * 16 + (q & 15);
}

// Exact split x = hi + mid + lo into three BF16 values (truncations; each
// residual is exact in FP32 because each step removes the leading 8
// significant bits), returned as 16-bit patterns.
struct bf16x3 {
    uint32_t hi, mid, lo;
};

__device__ __forceinline__ bf16x3 split3(float x)
{
    const uint32_t xb = __float_as_uint(x);
    const uint32_t hb = xb & 0xffff0000u;
    const float r1 = x - __uint_as_float(hb);
    const uint32_t mb = __float_as_uint(r1) & 0xffff0000u;
    const float r2 = r1 - __uint_as_float(mb);
    return {hb >> 16, mb >> 16, __float_as_uint(r2) >> 16};
}

// Four consecutive values split into the hi/mid/lo planes of xs (plane
// stride `plane` elements), one 8-byte store per plane; `at` is a multiple of 4.
__device__ __forceinline__ void store_split4(uint16_t* xs, size_t plane, size_t at, float4 v)
{
    const bf16x3 a = split3(v.x), b = split3(v.y), c = split3(v.z), d = split3(v.w);
    *reinterpret_cast<uint2*>(xs + at) = make_uint2(a.hi | (b.hi << 16), c.hi | (d.hi << 16));
    *reinterpret_cast<uint2*>(xs + plane + at) =
        make_uint2(a.mid | (b.mid << 16), c.mid | (d.mid << 16));
    *reinterpret_cast<uint2*>(xs + 2 * plane + at) =
        make_uint2(a.lo | (b.lo << 16), c.lo | (d.lo << 16));
}

__device__ __forceinline__ void store_split1(uint16_t* xs, size_t plane, size_t at, float v)
{
    const bf16x3 a = split3(v);
    xs[at] = (uint16_t)a.hi;
    xs[plane + at] = (uint16_t)a.mid;
    xs[2 * plane + at] = (uint16_t)a.lo;
}

// 2^e as a float, e in [-126, 127].
__device__ __forceinline__ float exp2i(int e)
{
    return __uint_as_float((uint32_t)(e + 127) << 23);
}

// Scale exponent of a row whose largest magnitude is m: m * 2^e lies in
// [2^14, 2^15), inside FP16's normal range, so neither FP16 plane overflows.
// 0 for m = 0 or nonfinite m; clamped to [-126, 126] (subnormal m gives 126).
__device__ __forceinline__ int row_exponent(float m)
{
    const uint32_t field = (__float_as_uint(m) >> 23) & 0xffu;
    if (!(m > 0.0f) || field == 0xffu) {
        return 0;
    }
    if (field == 0) {
        return 126;
    }
    const int e = 141 - (int)field;   // m = f * 2^(field - 126), f in [0.5, 1)
    return e < -126 ? -126 : (e > 126 ? 126 : e);
}

// Two-plane FP16 form of an (already scaled) value: h = f16(v), l = f16(v - h);
// v - h is exact in FP32, so h + l carries about 22 significant bits.
__device__ __forceinline__ uint32_t f16_hi(float v, float& rest)
{
    const _Float16 h = (_Float16)v;
    rest = v - (float)h;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t f16_bits(float v)
{
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// Four consecutive scaled values into the two FP16 planes of xs (plane stride
// `plane` elements), one 8-byte store per plane; `at` is a multiple of 4.
__device__ __forceinline__ void store_f16x2_4(uint16_t* xs, size_t plane, size_t at, float4 v)
{
    float ra, rb, rc, rd;
    const uint32_t a = f16_hi(v.x, ra), b = f16_hi(v.y, rb), c = f16_hi(v.z, rc),
                   d = f16_hi(v.w, rd);
    *reinterpret_cast<uint2*>(xs + at) = make_uint2(a | (b << 16), c | (d << 16));
    *reinterpret_cast<uint2*>(xs + plane + at) = make_uint2(
        f16_bits(ra) | (f16_bits(rb) << 16), f16_bits(rc) | (f16_bits(rd) << 16));
}

// Two adjacent scaled values into the two FP16 planes of xs, one 4-byte
// store per plane; `at` is even.
__device__ __forceinline__ void store_f16x2_2(uint16_t* xs, size_t plane, size_t at, float a,
    float b)
{
    float ra, rb;
    const uint32_t ha = f16_hi(a, ra), hb = f16_hi(b, rb);
    *reinterpret_cast<uint32_t*>(xs + at) = ha | (hb << 16);
    *reinterpret_cast<uint32_t*>(xs + plane + at) = f16_bits(ra) | (f16_bits(rb) << 16);
}

}  // namespace lh
