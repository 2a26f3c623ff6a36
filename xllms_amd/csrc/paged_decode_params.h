// Launch parameters shared by the host launcher and the gfx950 kernels of the
// paged-decode attention.  Plain data, passed by value as the kernel argument.
#pragma once

#include <stdint.h>

namespace xhip {

enum KvType : int { KV_F16 = 1, KV_BF16 = 2, KV_F32 = 3 };

// Work decomposition.  One wavefront is one work item
// (sequence, kv head, head tile, partition): it streams the partition's
// tokens of that kv head once and serves every query head of its head tile
// (the whole GQA group when group <= 8).  A workgroup holds kWavesPerGroup
// items; the head tiles of one (sequence, kv head, partition) are adjacent
// items, so they share a workgroup and hence the CU's L1 for the same pages.
constexpr int kWavesPerGroup = 4;
constexpr int kMaxHeadTile = 8;   // query heads per wavefront
constexpr int kLoadsPerTile = 4;  // 16-byte K (and V) loads per lane per tile

struct DecodeParams {
    void *out;                 // [num_seqs][num_heads][head_size], element type
    const void *q;             // [num_seqs][num_heads][head_size]
    const void *k;             // paged K cache (element type)
    const void *v;             // paged V cache
    const int *block_tables;   // [num_seqs][max_blocks]
    const int *seq_lens;       // [num_seqs]
    float *ws_o;               // [num_seqs*num_heads*max_parts][head_size] fp32
    float *ws_ml;              // [num_seqs*num_heads*max_parts][2] (max, sum)
    long long kv_block_stride; // elements
    long long kv_head_stride;  // elements
    int num_seqs;
    int num_heads;
    int num_kv_heads;
    int group;                 // num_heads / num_kv_heads
    int head_tiles;            // ceil(group / head tile), 1, 2 or 4
    int max_blocks;            // block-table row length
    int block_size;
    int bs_shift;              // log2(block_size)
    int part_tokens;           // split-K partition length (tokens)
    int max_parts;             // ceil(max_ctx / part_tokens)
    int max_ctx;               // max_blocks * block_size
    float scale_log2;          // scale * log2(e)
};

}  // namespace xhip
