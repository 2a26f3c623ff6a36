/*
 * Library-internal decode entry points with per-sequence query and output
 * rows, for the model instance (model_instance.cpp), whose requests keep
 * their own buffers: q_rows[s] / o_rows[s] (device arrays of num_seqs
 * pointers) are the [num_heads][head_size] query and output rows of
 * sequence s, 16-byte aligned.  Otherwise the arguments, checks and results
 * of nxt_paged_attention_ex (automatic plan) and nxt_paged_attention_cascade.
 * Hidden symbols: not part of the exported C-ABI.
 */
#ifndef XLLM_HIP_PAGED_DECODE_ROWS_H
#define XLLM_HIP_PAGED_DECODE_ROWS_H

#include "xllm_hip_operator_api.h"

#ifdef __cplusplus
extern "C" {
#endif

__attribute__((visibility("hidden"))) int xhip_paged_attention_rows(
    const char *const *q_rows, char *const *o_rows, const void *key_cache,
    const void *value_cache, const int *block_tables, const int *seq_lens, int num_seqs,
    int num_heads, int head_size, int num_kv_heads, float scale, int max_num_blocks_per_seq,
    int block_size, int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream);

__attribute__((visibility("hidden"))) int xhip_paged_attention_cascade_rows(
    const char *const *q_rows, char *const *o_rows, const void *key_cache,
    const void *value_cache, const int *block_tables, const int *seq_lens,
    const int *prefix_group, const int *prefix_blocks, int max_groups, int num_seqs,
    int num_heads, int head_size, int num_kv_heads, float scale, int max_num_blocks_per_seq,
    int block_size, int kv_block_stride, int kv_head_stride, int kv_dtype, nxt_stream_t stream);

/* One sequence's decode step whose new token is not in the cache yet (the
 * model instance's one-request exec): attends over the seq_len[0] cached
 * tokens (block_table: the sequence's row) into the fp32 states state_rows
 * [num_heads][head_size] / state_lse [num_heads], folds in the new token's
 * rows new_k / new_v ([num_kv_heads][head_size]) and writes `out`
 * ([num_heads][head_size]); the same launches then store the token's rows
 * to cache slot new_slot, new_page to *new_table_entry (if not NULL) and
 * new_len (= seq_len[0] + 1) to *new_len_entry, which may be seq_len itself.
 * head_size 32, 64 or 128. */
__attribute__((visibility("hidden"))) int xhip_paged_attention_fold_new(
    void *out, const void *query, const void *key_cache, const void *value_cache,
    const int *block_table, const int *seq_len, float *state_rows, float *state_lse,
    const void *new_k, const void *new_v, int *new_table_entry, int *new_len_entry, int new_slot,
    int new_page, int new_len, int num_heads, int head_size, int num_kv_heads, float scale,
    int max_num_blocks_per_seq, int block_size, int kv_block_stride, int kv_head_stride,
    int kv_dtype, nxt_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_PAGED_DECODE_ROWS_H */
