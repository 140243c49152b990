/* Scalar pieces of the oracle: FP8/BF16 decode, YaRN, query factor, greedy
 * selection, the Cody-Waite exp shared with the device kernels, SiLU.
 * TEST INFRASTRUCTURE ONLY (see oracle.h). */
#include "oracle.h"

#include <math.h>
#include <string.h>

/* E4M3FN decode, src/safetensors.c:505-519: e=(b>>3)&15, f=b&7;
 * f*2^-9 when e==0, else (1+f/8)*2^(e-7); bit 7 is the sign; 0x7f/0xff NaN.
 * Pinned by tests/fp8_golden.h (all 256 codes) and the oracle/_ref build. */
float orc_fp8_decode(uint8_t code)
{
    unsigned e = (code >> 3) & 15u;
    unsigned f = code & 7u;
    if (e == 15 && f == 7) {
        return NAN;
    }
    float magnitude = e == 0 ? ldexpf((float)f, -9) : ldexpf((float)(8 + f), (int)e - 10);
    return (code & 128u) ? -magnitude : magnitude;
}

/* BF16 widening is a 16-bit shift (src/safetensors.c:450-456). */
float orc_bf16_widen(uint16_t bits)
{
    uint32_t word = (uint32_t)bits << 16;
    float value;
    memcpy(&value, &word, sizeof value);
    return value;
}

/* Round-to-nearest-even to BF16 (finite inputs). Used to build synthetic
 * BF16 tensors the same way on every side. */
uint16_t orc_bf16_round(float value)
{
    uint32_t word;
    memcpy(&word, &value, sizeof word);
    uint32_t lsb = (word >> 16) & 1u;
    word += 0x7fffu + lsb;
    return (uint16_t)(word >> 16);
}

/* Host YaRN cos/sin for one position, following src/metal_yarn.c:8-33:
 * correction bounds in double, then per half-dim j in FP32 with the literal
 * interpolation (1-ext) and ext terms kept as written. Pinned bitwise against
 * the reference C (oracle/_ref) and to 2e-6 against tests/rope_golden.h. */
int orc_yarn(uint32_t position, float cosine[128], float sine[128])
{
    if (position >= 262144u) {
        return -1;
    }
    const double pi = 3.14159265358979323846;
    const double theta_log2 = 2.0 * log(1e6);
    float low = (float)floor(128.0 * log(16384.0 / (32 * 2.0 * pi)) / theta_log2);
    float high = (float)ceil(128.0 * log(16384.0 / (2.0 * pi)) / theta_log2);
    for (int j = 0; j < 64; j++) {
        float base = powf(1000000.0f, (float)(2 * j) / 128.0f);
        float ramp = fminf(1.0f, fmaxf(0.0f, ((float)j - low) / (high - low)));
        float ext = 1.0f - ramp;
        float interpolated = 1.0f / (16.0f * base);
        float extrapolated = 1.0f / base;
        float inv = interpolated * (1.0f - ext) + extrapolated * ext;
        float angle = inv * (float)position;
        float c = cosf(angle), s = sinf(angle);
        cosine[j] = c;
        cosine[j + 64] = c;
        sine[j] = s;
        sine[j + 64] = s;
    }
    return 0;
}

/* Integer-block query scaling, src/metal_kernels.metal:72-76:
 * 1 + 0.1*ln(1 + floor(pos/16384)); exactly 1.0f below 16384. */
float orc_query_factor(uint32_t position)
{
    return 1.0f + 0.1f * logf(1.0f + (float)(position / 16384u));
}

/* Greedy selection, src/generation.c:8-34: reject any NaN/Inf; strict '>'
 * keeps the lowest id on ties (-0 == +0). Pinned by the oracle/_ref build and
 * the tests/test_generation.c cases. */
int orc_select_greedy(const float *logits, size_t count, int64_t *token)
{
    if (!logits || !token || !count) {
        return -1;
    }
    size_t best = 0;
    for (size_t i = 0; i < count; i++) {
        if (!isfinite(logits[i])) {
            return -1;
        }
        if (logits[i] > logits[best]) {
            best = i;
        }
    }
    *token = (int64_t)best;
    return 0;
}

/* exp(x) by Cody & Waite additive range reduction (W. J. Cody, W. Waite,
 * "Software Manual for the Elementary Functions", 1980): k = rint(x*log2(e)),
 * r = x - k*ln2_hi - k*ln2_lo with ln2_hi holding 15 significant bits so
 * k*ln2_hi is exact, then the degree-7 Taylor polynomial of e^r by Horner's
 * rule with fused multiply-adds, then ldexp. Results below the normal range
 * flush to +0; above ln(FLT_MAX) give +inf. Only +, *, fma, rint and ldexp
 * are used, so the gfx950 kernels reproduce it bit for bit. Accuracy is
 * checked against libm in tests (<= 2 ulp). */
float orc_expf(float x)
{
    if (x != x) {
        return x;
    }
    if (x > 88.72283935546875f) {
        return INFINITY;
    }
    if (x < -87.33654022216796875f) {
        return 0.0f;
    }
    float k = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(k, -0.693145751953125f, x);
    r = fmaf(k, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412698412698412698e-04f;       /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888888889e-03f); /* 1/720 */
    p = fmaf(p, r, 8.33333333333333333333e-03f); /* 1/120 */
    p = fmaf(p, r, 4.16666666666666666667e-02f); /* 1/24 */
    p = fmaf(p, r, 1.66666666666666666667e-01f); /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* SiLU v/(1+exp(-v)), src/metal_kernels.metal:55-56. */
float orc_silu_ref(float v)
{
    return v / (1.0f + expf(-v));
}

float orc_silu_mirror(float v)
{
    return v / (1.0f + orc_expf(-v));
}
