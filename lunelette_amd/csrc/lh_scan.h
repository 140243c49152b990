/* Host scans over the 131072 logits of a step, written so that gcc -O2
 * vectorizes them (16 independent lanes, no early exit in the hot loop). */
#ifndef LH_SCAN_H
#define LH_SCAN_H

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define LH_SCAN_LANES 16

/* Index of the first nonfinite value (exponent bits all ones), or n when
 * every value is finite; n a multiple of LH_SCAN_LANES. */
__attribute__((optimize("tree-vectorize"))) static inline size_t lh_first_nonfinite(
    const float *v, size_t n)
{
    uint32_t lane_bad[LH_SCAN_LANES] = {0};
    for (size_t i = 0; i < n; i += LH_SCAN_LANES) {
        for (size_t k = 0; k < LH_SCAN_LANES; k++) {
            uint32_t bits;
            memcpy(&bits, &v[i + k], sizeof bits);
            lane_bad[k] |= (bits & 0x7f800000u) == 0x7f800000u;
        }
    }
    uint32_t bad = 0;
    for (size_t k = 0; k < LH_SCAN_LANES; k++) {
        bad |= lane_bad[k];
    }
    if (!bad) {
        return n;
    }
    size_t i = 0;
    while (isfinite(v[i])) {
        i++;
    }
    return i;
}

/* One pass: the maximum of v into *best and whether every value is finite
 * (n a positive multiple of LH_SCAN_LANES); *best is meaningful only when
 * every value is finite. */
__attribute__((optimize("tree-vectorize"))) static inline int lh_max_all_finite(const float *v,
    size_t n, float *best)
{
    float lane_max[LH_SCAN_LANES];
    uint32_t lane_bad[LH_SCAN_LANES] = {0};
    for (size_t k = 0; k < LH_SCAN_LANES; k++) {
        lane_max[k] = v[k];
    }
    for (size_t i = 0; i < n; i += LH_SCAN_LANES) {
        for (size_t k = 0; k < LH_SCAN_LANES; k++) {
            uint32_t bits;
            memcpy(&bits, &v[i + k], sizeof bits);
            lane_bad[k] |= (bits & 0x7f800000u) == 0x7f800000u;
            lane_max[k] = v[i + k] > lane_max[k] ? v[i + k] : lane_max[k];
        }
    }
    uint32_t bad = 0;
    float m = lane_max[0];
    for (size_t k = 0; k < LH_SCAN_LANES; k++) {
        bad |= lane_bad[k];
        m = lane_max[k] > m ? lane_max[k] : m;
    }
    *best = m;
    return !bad;
}

/* First index whose value equals x (x occurs in v[0, n)). */
__attribute__((optimize("tree-vectorize"))) static inline size_t lh_first_equal(const float *v,
    size_t n, float x)
{
    size_t block = 0;
    for (; block < n; block += LH_SCAN_LANES) {
        uint32_t hit = 0;
        for (size_t k = 0; k < LH_SCAN_LANES; k++) {
            hit |= v[block + k] == x;
        }
        if (hit) {
            break;
        }
    }
    size_t i = block;
    while (i < n && v[i] != x) {
        i++;
    }
    return i;
}

#endif
