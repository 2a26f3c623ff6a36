// Launch parameters of the paged KV-append kernel (paged_kv_append.hip).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "fast_div.h"

namespace xhip {

struct KvAppendParams {
    void *key_cache;
    void *value_cache;
    const void *key;           // [num_tokens][num_kv_heads][row_bytes], or the caches
    const void *value;         // themselves when src_slots is set
    const int *src_slots;      // [num_tokens] copy mode: token i's rows are read from
                               // this cache slot (null: from key / value)
    const char *const *key_rows;    // [num_tokens] gather mode: token i's [num_kv_heads]
    const char *const *value_rows;  // rows start at key_rows[i] / value_rows[i]
    const int *slots;          // [num_tokens] flat slots, or null: use block_tables + positions
    const int *block_tables;   // [num_tokens][max_blocks] (decode: token s = sequence s)
    const int *positions;      // [num_tokens]
    long long kv_block_stride_bytes;
    long long kv_head_stride_bytes;
    int num_tokens;
    int num_kv_heads;
    int row_bytes;             // head_size * element bytes, a multiple of 16
    int row_chunks;            // row_bytes / 16
    int block_size;            // power of two
    int bs_shift;
    int max_blocks;
    int max_ctx;               // max_blocks * block_size
    // set by launch_kv_append for each of its launches:
    int tok0;                  // first token of the launch
    uint32_t chunks;           // 16-byte chunks of K (and of V) in the launch
    DivMagic row_div;          // division by row_chunks
    DivMagic head_div;         // division by num_kv_heads
};

hipError_t launch_kv_append(const KvAppendParams &p, hipStream_t stream);

// Block-table work of a staging launch (the model instance's tables kept on
// the device between execs): the first head_bytes of the staged bytes go to
// `head` (a whole upload of the tables) instead of the destination, whose
// first byte then receives staged byte head_bytes; and `count` (index,
// value) int pairs, host-pinned, are stored as table[index] = value (the
// entries of pages opened since the last upload).
struct StageTables {
    void *head;
    long long head_bytes;  // a multiple of 16
    const int *pairs;
    int count;
    int *table;
};

// Copies `bytes` (a multiple of 16; both addresses 16-byte aligned) from
// host-pinned memory to device memory with a kernel on `stream`, with the
// table work of `t` when set.
hipError_t launch_stage_copy(void *dst, const void *host_src, size_t bytes, hipStream_t stream,
                             const StageTables *t = nullptr);

// launch_stage_copy and launch_kv_append(p) in one launch; p's per-token
// arrays (slots, key_rows, value_rows; src_slots unused) must be readable
// by the device where they are, e.g. in the host-pinned source being copied.
hipError_t launch_stage_copy_append(void *dst, const void *host_src, size_t bytes,
                                    const KvAppendParams &p, hipStream_t stream,
                                    const StageTables *t = nullptr);

// Queues a one-thread kernel that stores `value` to `word` (host-coherent
// pinned memory) with system scope, after everything queued on `stream`.
hipError_t launch_exec_signal(unsigned *word, unsigned value, hipStream_t stream);

}  // namespace xhip
