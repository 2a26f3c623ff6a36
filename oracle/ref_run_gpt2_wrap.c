/*
 * Build wrapper that exposes the reference's own CPU paged attention
 * (static paged_attention of examples/run_gpt2.c:46-83) from a shared object
 * in oracle/_ref/.  TEST INFRASTRUCTURE ONLY: the reference source is compiled
 * where it lies under the reference tree (REF_EXAMPLES include path set by
 * oracle/Makefile); nothing of it is copied into this repository.  The
 * reference's main() is renamed so the object links as a library.
 */
#define main xllm_reference_run_gpt2_main
#include "run_gpt2.c"
#undef main

void ref_gpt2_paged_attention(const float *query, const float *key_cache,
                              const float *value_cache, const int *page_table,
                              int seq_len, int num_heads, int head_dim, int page_size,
                              float *output) {
    paged_attention(query, key_cache, value_cache, page_table, seq_len, num_heads,
                    head_dim, page_size, output);
}
