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

#ifdef __cplusplus
}
#endif

#endif /* XLLM_HIP_PAGED_DECODE_ROWS_H */
