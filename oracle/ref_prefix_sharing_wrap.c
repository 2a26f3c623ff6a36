/*
 * Flat entry points over the reference's radix tree (src/core/prefix_sharing.c,
 * declared in include/prefix_sharing.h), for ctypes.  TEST INFRASTRUCTURE
 * ONLY: oracle/Makefile compiles the reference source where it lies under the
 * reference tree together with this file into oracle/_ref/; nothing of the
 * reference is copied into this repository.  The tree is created without a
 * page pool (the reference's own tests do the same,
 * tests/test_prefix_sharing.c:28-29).
 */
#include <stdint.h>
#include <stdlib.h>
#include <time.h>

#include "prefix_sharing.h"

/* The tree stamps nodes with clock_gettime(CLOCK_MONOTONIC) in microseconds
 * (prefix_sharing.c:18-23) and evicts the leaf with the oldest stamp.  In
 * this test build that clock is a counter: this hidden definition binds the
 * source's calls at link time, and every reading is one microsecond later
 * than the one before.  The stamps then follow the order in which the tree
 * reads its clock (a match or insert first, then each node it creates),
 * which is the restatement's logical clock, whatever the host's scheduling
 * does to real time between and inside calls. */
static uint64_t g_now_us = 0;

__attribute__((visibility("hidden"))) int clock_gettime(clockid_t id, struct timespec *ts) {
    (void)id;
    g_now_us++;
    ts->tv_sec = (time_t)(g_now_us / 1000000u);
    ts->tv_nsec = (long)(g_now_us % 1000000u) * 1000L;
    return 0;
}

void *refps_new(void) {
    NxtPrefixTree *t = (NxtPrefixTree *)calloc(1, sizeof(NxtPrefixTree));
    if (t) nxt_prefix_tree_init(t, NULL);
    return t;
}

void refps_free(void *t) {
    if (!t) return;
    nxt_prefix_tree_destroy((NxtPrefixTree *)t);
    free(t);
}

/* Returns matched_tokens; page ids go to pages[] (capacity
 * NXT_PREFIX_MAX_MATCH_PAGES), their count to *page_count, the terminal node
 * to *last (NULL when it is the root). */
int refps_match(void *t, const int32_t *tokens, int32_t len, uint32_t *pages, int32_t *page_count,
                void **last) {
    NxtPrefixTree *tree = (NxtPrefixTree *)t;
    NxtMatchResult *r = (NxtMatchResult *)malloc(sizeof(NxtMatchResult));
    if (!r) return -1;
    *r = nxt_prefix_match(tree, tokens, len);
    for (int32_t i = 0; i < r->page_count; i++) pages[i] = r->page_ids[i];
    *page_count = r->page_count;
    *last = r->last_node == tree->root ? NULL : r->last_node;
    const int m = r->matched_tokens;
    free(r);
    return m;
}

int refps_insert(void *t, const int32_t *tokens, int32_t len, const uint32_t *pages,
                 int32_t page_count, int32_t priority) {
    return nxt_prefix_insert((NxtPrefixTree *)t, tokens, len, pages, page_count, priority);
}

int refps_evict(void *t, int32_t num_tokens) {
    return nxt_prefix_evict((NxtPrefixTree *)t, num_tokens);
}

void refps_lock(void *t, void *node) { nxt_prefix_lock((NxtPrefixTree *)t, (NxtPrefixNode *)node); }

void refps_unlock(void *t, void *node) {
    nxt_prefix_unlock((NxtPrefixTree *)t, (NxtPrefixNode *)node);
}

/* total tokens, node count, evictable size, protected size */
void refps_stats(void *t, int32_t *out) {
    NxtPrefixTree *tree = (NxtPrefixTree *)t;
    out[0] = nxt_prefix_total_tokens(tree);
    out[1] = nxt_prefix_node_count(tree);
    out[2] = nxt_prefix_evictable_size(tree);
    out[3] = tree->protected_size;
}
