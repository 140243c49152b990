/* Test-only entry points: host-forced failures for the runtime's state-machine
 * tests. They have no counterpart in the reference ABI and are not part of the
 * shipped library: they are linked only into liblunelette_hip_test.so (the
 * same objects plus test_seams.c), as the reference confines its checkpoint
 * allocation fault to a test build of its runtime object (Makefile:126-129).
 * The faults stand in for the reference's mocked devices and command buffers
 * (tests/test_metal.m:629-954); every one is forced from the host, and every
 * kernel of a failed step still runs to completion. */
#ifndef LH_TEST_SEAMS_H
#define LH_TEST_SEAMS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct lunelette_metal;
/* what = 1: the next execution fails before any device work; 2: the next
 * execution publishes an Inf logit; 3: the next checkpoint allocation fails;
 * 6: in the next execution every attention block that shares a launch with
 * the q|k|v projection waits for producer flags that never come, gives up
 * after 64 polls and writes NaN (each kernel still runs to its end); 7: in
 * the next execution the attention's flag combiners (one token past 16 blocks,
 * in the q|k|v launch or in the attention's own) wait for block flags that
 * never come, give up after 64 polls and write NaN. */
int lunelette_metal_test_inject(struct lunelette_metal *context, int what);
/* The next execution fails after layer `layer`'s kernels ran, so layers
 * 0..layer have written their KV rows for it. */
int lunelette_metal_test_fail_after_layer(struct lunelette_metal *context, uint32_t layer);
/* Sets the context's checkpoint epoch counter (UINT64_MAX: exhausted). */
int lunelette_metal_test_set_epoch(struct lunelette_metal *context, uint64_t epoch);
/* Whether a decode token at this length runs q|k|v and its attention blocks
 * in one launch on the current device. */
int lunelette_metal_test_chained(uint32_t length);
/* Overwrites one published host logit. */
int lunelette_metal_test_set_logit(struct lunelette_metal *context, size_t index, float value);
/* Arms the allocation counter: the nth device or pinned-host allocation from
 * now on fails (0: none fails; the counter still counts). */
void lunelette_metal_test_fail_allocation(unsigned nth);
/* Allocations since the counter was armed, and allocations not yet freed. */
unsigned lunelette_metal_test_allocations(void);
long lunelette_metal_test_live_allocations(void);
/* The same for the host heap allocations of the generation loop, tokenizer
 * and chat framing (lh_host_alloc.h): the nth from now on fails (0: none). A
 * block handed to a caller (token ids, text) stays counted as live. */
void lunelette_metal_test_fail_host_allocation(unsigned nth);
unsigned lunelette_metal_test_host_allocations(void);
long lunelette_metal_test_live_host_allocations(void);

#ifdef __cplusplus
}
#endif

#endif
