/* Test-only seams (lh_test_seams.h). Linked into liblunelette_hip_test.so only;
 * the shipped liblunelette_hip.so neither contains nor exports them. */
#include "lh_test_seams.h"
#include "lh_internal.h"
#include "lh_host_alloc.h"

int lunelette_metal_test_inject(struct lunelette_metal *context, int what)
{
    if ((what < LH_FAULT_BEFORE_DEVICE || what > LH_FAULT_CHECKPOINT_ALLOC) &&
        what != LH_FAULT_HANDOFF && what != LH_FAULT_COMBINERS) {
        return -1;
    }
    return lh_runtime_fault(context, what, 0);
}

int lunelette_metal_test_fail_after_layer(struct lunelette_metal *context, uint32_t layer)
{
    return lh_runtime_fault(context, LH_FAULT_AFTER_LAYER, layer);
}

int lunelette_metal_test_set_epoch(struct lunelette_metal *context, uint64_t epoch)
{
    return lh_runtime_fault(context, LH_FAULT_EPOCH, epoch);
}

int lunelette_metal_test_set_logit(struct lunelette_metal *context, size_t index, float value)
{
    return lh_runtime_set_logit(context, index, value);
}

void lunelette_metal_test_fail_allocation(unsigned nth)
{
    lh_allocations_arm(nth);
}

unsigned lunelette_metal_test_allocations(void)
{
    return lh_allocations_count();
}

long lunelette_metal_test_live_allocations(void)
{
    return lh_allocations_live();
}

void lunelette_metal_test_fail_host_allocation(unsigned nth)
{
    lh_host_allocations_arm(nth);
}

unsigned lunelette_metal_test_host_allocations(void)
{
    return lh_host_allocations_count();
}

long lunelette_metal_test_live_host_allocations(void)
{
    return lh_host_allocations_live();
}

int lunelette_metal_test_chained(uint32_t length)
{
    return lh_attention_chained(length);
}
