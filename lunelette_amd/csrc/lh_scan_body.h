/* One instance of the logit scans for one vector width; included by
 * lh_scan.h with LH_SCAN_ISA (name suffix), LH_SCAN_TARGET (function
 * attribute) and LH_SCAN_BYTES (vector width) defined. */
#define LH_SCAN_CAT_(a, b) a##_##b
#define LH_SCAN_CAT(a, b) LH_SCAN_CAT_(a, b)
#define LH_VF LH_SCAN_CAT(lh_vf, LH_SCAN_ISA)
#define LH_VI LH_SCAN_CAT(lh_vi, LH_SCAN_ISA)
#define LH_LANES (LH_SCAN_BYTES / 4)

typedef float LH_VF __attribute__((vector_size(LH_SCAN_BYTES)));
typedef int32_t LH_VI __attribute__((vector_size(LH_SCAN_BYTES)));

/* Lanes of the floats at `at` whose exponent bits are all ones (Inf or NaN)
 * become -1, others 0. */
#define LH_SCAN_NONFINITE(out, at)                                            \
    do {                                                                      \
        LH_VI bits_;                                                          \
        memcpy(&bits_, (at), sizeof bits_);                                   \
        const LH_VI exponent_ = (LH_VI){0} + 0x7f800000;                      \
        (out) = (bits_ & exponent_) == exponent_;                             \
    } while (0)

LH_SCAN_TARGET static size_t LH_SCAN_CAT(lh_first_nonfinite, LH_SCAN_ISA)(const float *v,
    size_t n)
{
    LH_VI bad = {0};
    for (size_t i = 0; i < n; i += LH_LANES) {
        LH_VI lanes;
        LH_SCAN_NONFINITE(lanes, v + i);
        bad |= lanes;
    }
    int32_t any = 0;
    for (int k = 0; k < LH_LANES; k++) {
        any |= bad[k];
    }
    if (!any) {
        return n;
    }
    size_t i = 0;
    while (isfinite(v[i])) {
        i++;
    }
    return i;
}

/* Four named accumulators (not arrays, so they stay in vector registers). */
LH_SCAN_TARGET static int LH_SCAN_CAT(lh_argmax_all_finite, LH_SCAN_ISA)(const float *v,
    size_t n, size_t *index)
{
    enum { STRIDE = 4 * LH_LANES };
    LH_VF b0, b1, b2, b3;
    memcpy(&b0, v, sizeof b0);
    memcpy(&b1, v + LH_LANES, sizeof b1);
    memcpy(&b2, v + 2 * LH_LANES, sizeof b2);
    memcpy(&b3, v + 3 * LH_LANES, sizeof b3);
    LH_VI p0 = {0}, p1 = {0}, p2 = {0}, p3 = {0}, bad = {0}, now = {0};
    const LH_VI one = now + 1;
#define LH_ARGMAX_WAY(b, p, w)                                                \
    do {                                                                      \
        const float *chunk_ = v + i + (w) * LH_LANES;                         \
        LH_VF x_;                                                             \
        memcpy(&x_, chunk_, sizeof x_);                                       \
        LH_VI lanes_;                                                         \
        LH_SCAN_NONFINITE(lanes_, chunk_);                                    \
        bad |= lanes_;                                                        \
        const LH_VI greater_ = x_ > (b);                                      \
        (b) = (LH_VF)(((LH_VI)x_ & greater_) | ((LH_VI)(b) & ~greater_));      \
        (p) = ((p) & ~greater_) | (now & greater_);                           \
    } while (0)
    for (size_t i = 0; i < n; i += STRIDE) {
        LH_ARGMAX_WAY(b0, p0, 0);
        LH_ARGMAX_WAY(b1, p1, 1);
        LH_ARGMAX_WAY(b2, p2, 2);
        LH_ARGMAX_WAY(b3, p3, 3);
        now += one;
    }
#undef LH_ARGMAX_WAY
    const LH_VF best[4] = {b0, b1, b2, b3};
    const LH_VI pass[4] = {p0, p1, p2, p3};
    int32_t any = 0;
    float top = best[0][0];
    for (int w = 0; w < 4; w++) {
        for (int k = 0; k < LH_LANES; k++) {
            any |= bad[k];
            top = best[w][k] > top ? best[w][k] : top;
        }
    }
    if (any) {
        return 0;
    }
    size_t first = n;
    for (int w = 0; w < 4; w++) {
        for (int k = 0; k < LH_LANES; k++) {
            const size_t at = (size_t)pass[w][k] * STRIDE + (size_t)(w * LH_LANES + k);
            if (best[w][k] == top && at < first) {
                first = at;
            }
        }
    }
    *index = first;
    return 1;
}

#undef LH_SCAN_NONFINITE
#undef LH_LANES
#undef LH_VI
#undef LH_VF
#undef LH_SCAN_CAT
#undef LH_SCAN_CAT_
