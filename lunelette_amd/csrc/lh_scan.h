/* Host scans over the 131072 logits of a step: GCC vector types with four
 * independent accumulators, branch-free over whole vectors. Two instances
 * are built from lh_scan_body.h, 16-byte vectors for the x86-64 baseline and
 * 32-byte vectors for AVX2, and each call takes the AVX2 one when the CPU
 * has it (about 3x faster). n is a multiple of 32 in every function. */
#ifndef LH_SCAN_H
#define LH_SCAN_H

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define LH_SCAN_ISA sse2
#define LH_SCAN_TARGET
#define LH_SCAN_BYTES 16
#include "lh_scan_body.h"
#undef LH_SCAN_BYTES
#undef LH_SCAN_TARGET
#undef LH_SCAN_ISA

#define LH_SCAN_ISA avx2
#define LH_SCAN_TARGET __attribute__((target("avx2")))
#define LH_SCAN_BYTES 32
#include "lh_scan_body.h"
#undef LH_SCAN_BYTES
#undef LH_SCAN_TARGET
#undef LH_SCAN_ISA

static inline int lh_scan_avx2(void)
{
    return __builtin_cpu_supports("avx2");
}

/* Index of the first nonfinite value (exponent bits all ones), or n when
 * every value is finite. */
static inline size_t lh_first_nonfinite(const float *v, size_t n)
{
    return lh_scan_avx2() ? lh_first_nonfinite_avx2(v, n) : lh_first_nonfinite_sse2(v, n);
}

/* One pass over v: whether every value is finite and, if so, the first
 * index of the maximum in *index. Each lane of the four accumulators keeps
 * the maximum of its residue class of indices under a strict '>' and the
 * pass in which it first occurred; the first index of the overall maximum
 * is the smallest such index among the lanes that hold it (-0.0 and +0.0
 * compare equal), which is what a forward scan with a strict '>' selects. */
static inline int lh_argmax_all_finite(const float *v, size_t n, size_t *index)
{
    return lh_scan_avx2() ? lh_argmax_all_finite_avx2(v, n, index) :
        lh_argmax_all_finite_sse2(v, n, index);
}

#endif
