// Multi-token (chunked prefill) projections on the MFMA matrix cores.
// Placeholder until the split-BF16 GEMM lands: the runtime does not select
// this path (LH_HAVE_MFMA is 0), and calling it reports an error.
#include "lh_internal.h"
#include "lh_layer.h"

extern "C" int lh_layer_forward_mfma(const lh_layer_weights* w, float* d_x, float* d_keys,
    float* d_values, lh_workspace* ws, hipStream_t s)
{
    (void)w; (void)d_x; (void)d_keys; (void)d_values; (void)ws; (void)s;
    lh_set_error("MFMA layer path is not built");
    return -1;
}

extern "C" int lh_mfma_prepare(lh_workspace* ws)
{
    (void)ws;
    return 0;
}
