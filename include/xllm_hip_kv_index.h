/*
 * xLLM HIP backend -- paged KV-cache index (host C-ABI, in libxllm_hip_backend.so).
 *
 * The host side that produces what the paged decode consumes: block_tables,
 * seq_lens, the slots of new tokens (nxt_paged_kv_write_slots) and the
 * shared-prefix groups of a batch (nxt_paged_attention_cascade).  It joins
 * the reference's three host structures to the operator-API page layout:
 *
 *   - block pool: allocation and reference counting of the physical pages
 *     (the [num_blocks] dimension of the K/V caches), with the semantics of
 *     nxt_page_alloc / nxt_page_ref_inc / nxt_page_ref_dec
 *     (src/core/memory_manager.c:207-272) restricted to one tier (HBM) and
 *     one page type: the free list is FIFO (allocation takes the head,
 *     release appends at the tail) and ids run 0..num_blocks-1, so the ids
 *     the reference pool hands out for TIER_GPU / PAGE_TYPE_DATA can be used
 *     as block ids unchanged.
 *   - radix tree: prefix_sharing.h:86-155 (match / insert / evict / lock /
 *     unlock / statistics) over token ids.  The reference stores one page id
 *     per token (prefix_sharing.c:306); here that id is the token's flat
 *     slot, block * block_size + offset, so a matched prefix yields both the
 *     pages to share and the offsets inside them.
 *   - sequences: admission of a prompt against the tree (full pages of the
 *     matched prefix are shared, a partly matched page is copied into a
 *     private page), decode append (scheduler.c:318-321 schedules one new
 *     token per running sequence), and the batch's block tables (every
 *     block_size-th slot of a sequence names its page).
 *
 * Differences from the reference structures, all deliberate:
 *   - The tree holds its own reference on every page its slots touch and
 *     gives it back when a node is evicted or destroyed (the reference's
 *     nxt_prefix_evict only adjusts a byte counter, prefix_sharing.c:375-384).
 *   - Recency is a logical clock (one tick per match / insert call and per
 *     node created), not CLOCK_MONOTONIC microseconds: the eviction order is
 *     the reference's whenever its timestamps differ, and deterministic when
 *     they would tie.
 *   - A match covers at most NXT_PREFIX_MAX_MATCH_PAGES slots and ends at the
 *     first node that would exceed it; the reference keeps counting matched
 *     tokens past a node whose pages it could not append
 *     (prefix_sharing.c:241-257), so its page list and token count disagree.
 *   - Eviction considers every leaf (the reference's walk uses fixed
 *     1024-entry stacks, prefix_sharing.c:338-357).
 *   - insert requires one slot per token; ref_inc / ref_dec of a free block
 *     and unlock of an unlocked node are refused instead of driving counts
 *     negative.
 *   - Tree nodes are named by 64-bit ids, not pointers; an id whose node was
 *     evicted is refused.
 *
 * Not thread-safe (the reference structures have no locks either): one
 * index per model instance; calls on one index must not overlap.
 */
#ifndef XLLM_HIP_KV_INDEX_H_
#define XLLM_HIP_KV_INDEX_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef NXT_PREFIX_MAX_MATCH_PAGES
#define NXT_PREFIX_MAX_MATCH_PAGES 2048 /* prefix_sharing.h:61 */
#endif

enum {
    NXT_KV_OK = 0,
    NXT_KV_E_INVALID = -1,   /* bad handle, argument or id */
    NXT_KV_E_NO_BLOCKS = -2, /* the pool is exhausted even after evicting the tree */
    NXT_KV_E_CAPACITY = -3,  /* a sequence would exceed max_blocks_per_seq pages */
};

typedef struct NxtKvIndex NxtKvIndex;

/* An index over a cache of num_blocks pages of block_size tokens (a power of
 * two); sequences may grow to max_blocks_per_seq pages.  NULL on bad sizes. */
NxtKvIndex *nxt_kv_index_create(int num_blocks, int block_size, int max_blocks_per_seq);
void nxt_kv_index_destroy(NxtKvIndex *ix);

/* ---- block pool (memory_manager.c:207-272) ---- */
/* A free block with one reference, or NXT_KV_E_NO_BLOCKS. */
int nxt_kv_block_alloc(NxtKvIndex *ix);
/* The new count, or NXT_KV_E_INVALID for a bad id or a free block.  A count
 * reaching zero returns the block to the tail of the free list. */
int nxt_kv_block_ref_inc(NxtKvIndex *ix, int block);
int nxt_kv_block_ref_dec(NxtKvIndex *ix, int block);
int nxt_kv_block_refs(const NxtKvIndex *ix, int block);
int nxt_kv_blocks_free(const NxtKvIndex *ix);

/* ---- radix tree (prefix_sharing.h:86-155) ---- */
typedef struct {
    int32_t matched_tokens; /* slots written to `slots` */
    int32_t reserved;
    uint64_t last_node;     /* terminal node (0 = the root: nothing matched) */
} NxtKvMatch;

/* Longest cached prefix of tokens[0..len); writes its slots (capacity
 * min(len, NXT_PREFIX_MAX_MATCH_PAGES)).  Splits the node where the match
 * ends inside it, refreshes recency and hit counts (prefix_sharing.c:211-265). */
int nxt_kv_prefix_match(NxtKvIndex *ix, const int32_t *tokens, int32_t len, int32_t *slots,
                        NxtKvMatch *out);
/* Caches tokens[0..len) at slots[0..len) (each slot's block must be held,
 * refs >= 1); the tree takes its own references.  Returns the length that
 * was already cached (prefix_sharing.c:267-325), or a negative status. */
int32_t nxt_kv_prefix_insert(NxtKvIndex *ix, const int32_t *tokens, int32_t len,
                             const int32_t *slots, int32_t priority);
/* Evicts least-recently-used unlocked leaves until at least num_tokens
 * tokens are gone or none is left; returns the tokens evicted
 * (prefix_sharing.c:327-399). */
int32_t nxt_kv_prefix_evict(NxtKvIndex *ix, int32_t num_tokens);
/* Lock / unlock a node and its ancestors (prefix_sharing.c:401-425). */
int nxt_kv_prefix_lock(NxtKvIndex *ix, uint64_t node);
int nxt_kv_prefix_unlock(NxtKvIndex *ix, uint64_t node);

typedef struct {
    int32_t total_tokens;   /* nxt_prefix_total_tokens */
    int32_t node_count;     /* nxt_prefix_node_count (root included) */
    int32_t evictable_size; /* nxt_prefix_evictable_size */
    int32_t protected_size; /* NxtPrefixTree.protected_size */
} NxtKvTreeStats;
int nxt_kv_prefix_stats(const NxtKvIndex *ix, NxtKvTreeStats *out);

/* ---- sequences ---- */
typedef struct {
    int32_t seq;            /* handle for the calls below */
    int32_t cached_tokens;  /* leading prompt tokens whose K/V is already in the cache
                             * (shared pages, or copied by the copy list) */
    int32_t shared_blocks;  /* leading pages shared with the tree */
    int32_t copy_count;     /* pairs in copy_src / copy_dst */
    int32_t write_count;    /* prompt tokens the caller must write (len - cached_tokens) */
} NxtKvAdmit;

/* Admits a prompt tokens[0..len), 1 <= len <= max_blocks_per_seq *
 * block_size.  Writes slot_mapping[len] (the slot of each prompt token whose
 * K/V the caller must write, -1 for cached ones: the argument of
 * nxt_paged_kv_write_slots over the whole prompt) and copy_src / copy_dst
 * (capacity len): page slots the caller must copy before the first decode
 * (nxt_paged_kv_copy_slots), the partly matched page's tokens.  Locks the
 * matched node until release.  Evicts from the tree when the pool runs out;
 * on failure nothing changes. */
int nxt_kv_seq_admit(NxtKvIndex *ix, const int32_t *tokens, int32_t len, int32_t *slot_mapping,
                     int32_t *copy_src, int32_t *copy_dst, NxtKvAdmit *out);
/* Appends n tokens (a decode step: n = 1) and writes their slots.  All or
 * nothing. */
int nxt_kv_seq_append(NxtKvIndex *ix, int32_t seq, const int32_t *tokens, int32_t n,
                      int32_t *slots);
/* One decode step of a batch: appends tokens[i] to sequence seqs[i] (each at
 * most once) and writes its slot to slots[i].  All or nothing. */
int nxt_kv_batch_append(NxtKvIndex *ix, const int32_t *seqs, int32_t n, const int32_t *tokens,
                        int32_t *slots);
/* Inserts the sequence's tokens so far into the tree (a running sequence's
 * prompt becomes shareable).  Returns what nxt_kv_prefix_insert returns. */
int32_t nxt_kv_seq_cache(NxtKvIndex *ix, int32_t seq);
/* Ends a sequence: with cache != 0 inserts its tokens first; then unlocks its
 * matched node and gives back its page references. */
int nxt_kv_seq_release(NxtKvIndex *ix, int32_t seq, int cache);
int32_t nxt_kv_seq_len(const NxtKvIndex *ix, int32_t seq);

/* The batch of sequences seqs[0..n): block_tables[n][max_blocks] (-1 past
 * each sequence's pages) and seq_lens[n], the nxt_paged_attention inputs. */
int nxt_kv_batch_tables(const NxtKvIndex *ix, const int32_t *seqs, int32_t n,
                        int32_t max_blocks, int32_t *block_tables, int32_t *seq_lens);
/* The batch's shared-prefix groups for nxt_paged_attention_cascade, by the
 * rule of nxt_paged_prefix_groups: sequences whose first page is the same
 * form a group (two or more members), whose prefix is the longest run of
 * leading pages all members share with the lowest-numbered member, counting
 * pages full in both.  prefix_group[n] (-1: none), prefix_blocks (capacity
 * n / 2 + 1), *num_groups; groups are numbered by lowest member. */
int nxt_kv_batch_prefix_groups(const NxtKvIndex *ix, const int32_t *seqs, int32_t n,
                               int32_t *prefix_group, int32_t *prefix_blocks,
                               int32_t *num_groups);

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_KV_INDEX_H_ */
