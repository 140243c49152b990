/* Heap allocations of the host-side C that parses or generates on behalf of a
 * caller (generation loop, tokenizer, chat framing). They are malloc, calloc,
 * realloc and free (a pointer handed to a caller may be released with free),
 * counted with relaxed atomics, and the nth one after the counter was armed
 * fails: the allocation-failure regressions of the reference
 * (tests/test_generation_alloc.c, tests/test_tokenizer_alloc.c) wrap the
 * sources' malloc the same way. Only the test-seam library (test_seams.c, not
 * part of the shipped library) arms the counter. */
#ifndef LH_HOST_ALLOC_H
#define LH_HOST_ALLOC_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

void *lh_malloc(size_t bytes);
void *lh_calloc(size_t count, size_t size);
/* A failed or refused realloc leaves the block as it was. */
void *lh_realloc(void *block, size_t bytes);
void lh_free(void *block);

/* Arms the counter: the nth allocation from now fails (1-based; 0 never). */
void lh_host_allocations_arm(unsigned nth);
/* Allocations since the counter was armed; blocks allocated and not yet
 * released through lh_free (a block returned to a caller stays counted). */
unsigned lh_host_allocations_count(void);
long lh_host_allocations_live(void);

#ifdef __cplusplus
}
#endif

#endif
