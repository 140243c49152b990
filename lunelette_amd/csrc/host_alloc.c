/* Counted host heap allocations with an armed failure (lh_host_alloc.h). */
#include "lh_host_alloc.h"

#include <stdatomic.h>
#include <stdlib.h>

static atomic_uint fail_at;   /* 1-based allocation to fail; 0 never */
static atomic_uint count;     /* allocations since the counter was armed */
static atomic_long live;      /* blocks not yet released through lh_free */

void lh_host_allocations_arm(unsigned nth)
{
    atomic_store_explicit(&count, 0, memory_order_relaxed);
    atomic_store_explicit(&fail_at, nth, memory_order_relaxed);
}

unsigned lh_host_allocations_count(void)
{
    return atomic_load_explicit(&count, memory_order_relaxed);
}

long lh_host_allocations_live(void)
{
    return atomic_load_explicit(&live, memory_order_relaxed);
}

static int refused(void)
{
    unsigned n = atomic_fetch_add_explicit(&count, 1, memory_order_relaxed) + 1;
    unsigned at = atomic_load_explicit(&fail_at, memory_order_relaxed);
    return at && n == at;
}

static void *counted(void *block)
{
    if (block) {
        atomic_fetch_add_explicit(&live, 1, memory_order_relaxed);
    }
    return block;
}

void *lh_malloc(size_t bytes)
{
    return refused() ? NULL : counted(malloc(bytes));
}

void *lh_calloc(size_t n, size_t size)
{
    return refused() ? NULL : counted(calloc(n, size));
}

void *lh_realloc(void *block, size_t bytes)
{
    if (refused()) {
        return NULL;
    }
    void *grown = realloc(block, bytes);
    return block ? grown : counted(grown);
}

void lh_free(void *block)
{
    if (block) {
        atomic_fetch_sub_explicit(&live, 1, memory_order_relaxed);
        free(block);
    }
}
