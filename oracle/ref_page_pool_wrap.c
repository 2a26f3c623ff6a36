/*
 * Flat entry points over the reference's page pool (src/core/memory_manager.c
 * with src/core/lru_k.c, declared in src/include/page_pool.h), for ctypes.
 * TEST INFRASTRUCTURE ONLY: oracle/Makefile compiles the reference sources
 * where they lie together with this file into oracle/_ref/.  The pool is
 * given HBM pages only, num_pages of each page type with tiny 64-byte pages
 * (the reference allocates a host buffer per page, memory_manager.c:216-223);
 * the entry points act on type PAGE_TYPE_DATA, tier TIER_GPU, whose page ids
 * are 0..num_pages-1 (memory_manager.c:166-184).
 */
#include <stdlib.h>

#include "page_pool.h"

#define REFPOOL_PAGE_BYTES 64

void *refpool_new(int num_pages) {
    NxtGlobalBufferPool *p = (NxtGlobalBufferPool *)calloc(1, sizeof(NxtGlobalBufferPool));
    if (!p) return NULL;
    const size_t total = (size_t)num_pages * PAGE_TYPE_COUNT;
    nxt_pool_init(p, total * REFPOOL_PAGE_BYTES, 0, 0, REFPOOL_PAGE_BYTES, total);
    return p;
}

void refpool_free(void *p) {
    if (!p) return;
    nxt_pool_destroy((NxtGlobalBufferPool *)p);
    free(p);
}

int refpool_alloc(void *p) {
    NxtPage *page = nxt_page_alloc((NxtGlobalBufferPool *)p, PAGE_TYPE_DATA, TIER_GPU);
    return page ? (int)page->page_id : -1;
}

void refpool_ref_inc(void *p, int id) {
    nxt_page_ref_inc(&((NxtGlobalBufferPool *)p)->pages_array[id]);
}

void refpool_ref_dec(void *p, int id) {
    NxtGlobalBufferPool *pool = (NxtGlobalBufferPool *)p;
    nxt_page_ref_dec(pool, &pool->pages_array[id]);
}

int refpool_refs(void *p, int id) { return ((NxtGlobalBufferPool *)p)->pages_array[id].ref_count; }

int refpool_free_count(void *p) {
    return (int)((NxtGlobalBufferPool *)p)->free_counts[TIER_GPU][PAGE_TYPE_DATA];
}
