// Launch parameters shared by the host launcher and the gfx950 kernels of the
// paged-decode attention.  Plain data, passed by value as the kernel argument.
#pragma once

#include <stdint.h>

namespace xhip {

enum KvType : int { KV_F16 = 1, KV_BF16 = 2, KV_F32 = 3 };

// Work decomposition (stream-K over the whole batch).
//
// The batch is the sequence of segments (sequence s, kv head, head tile) in
// that order; segment (s, .) holds T_s = ceil(L_s / tile_tokens) tiles.  All
// segments laid end to end form `total` split units, where a segment of T
// tiles costs T + seg_cost units: its tiles, after seg_cost units of
// start-up (the dependent loads before its first tile computes; measured on
// MI355X at ~1.5 tiles' time).  Wavefront w of the launch owns the
// contiguous unit range [w*tpw, min((w+1)*tpw, total)) with
// tpw = max(min_tiles_per_wave, ceil(total / num_waves)) and computes the
// tiles that fall in it, so every wavefront spends the same time whatever
// the ragged lengths -- a run of one-tile segments no longer lands on one
// wavefront as tiles of equal weight.
// A segment that lies inside one wavefront's range is finished there and
// written straight to the output; a segment cut by range boundaries leaves
// one fp32 partial (m, l, o) per wavefront that touched it, in that
// wavefront's slot 0 (the segment holds the wavefront's first tile) or
// slot 1 (it holds the wavefront's last tile but not its first), and
// paged_decode_merge_kernel combines them.
constexpr int kWavesPerGroup = 4;    // VALU tile path: wavefronts per workgroup
constexpr int kMfmaWavesPerGroup = 4;  // MFMA tile path
constexpr int kMaxHeadTile = 8;      // query heads per wavefront, VALU tile path
constexpr int kMfmaHeads = 16;       // query heads per MFMA row block (R blocks per wavefront)
constexpr int kMfmaWideMaxHeadSize = 128;  // largest head_size with R = 2
constexpr int kMfmaMaxGroup = 64;    // largest GQA group on the MFMA path (head tiles of 16 or 32)
constexpr int kMergeCols = 32;       // float4 columns per workgroup of the chunked merge
constexpr int kLoadsPerTile = 4;     // 16-byte K (and V) loads per lane per tile
constexpr int kMaxSeqsPerLaunch = 8192;  // the per-workgroup prefix scan lives in LDS

// Small batches on the VALU tile path (DecodeParams::segment_launch): one
// workgroup of kSegWaves wavefronts per segment (or per share of a segment,
// DecodeParams::segment_split), each wavefront with kSegTiles tiles in
// flight, at most kSegRounds rounds of them (so segments of at most
// kSegWaves * kSegTiles * kSegRounds tiles per workgroup), head tiles of at
// most kSegMaxHeadTile heads.
constexpr int kSegWaves = 16;
constexpr int kSegTiles = 2;
constexpr int kSegRounds = 4;
constexpr int kSegMaxHeadTile = 2;

// Workgroup-level combine of cut segments (MFMA tile path, head_size <=
// 128): the kMfmaWavesPerGroup wavefronts of a workgroup own consecutive
// stream-K ranges, so the pieces of one segment that fall in one workgroup
// are merged through LDS at the end of the kernel.  Only one fp32 partial
// per (segment, workgroup it spans) is left for the merge kernel, in the
// slot of the leftmost wavefront holding a piece of it, and a segment lying
// inside one workgroup is written finished.  Mode 1 (one row block): every
// wavefront has an LDS slot.  Mode 2 (two row blocks, whose slots would
// not leave room for two workgroups per CU): one relay slot per workgroup.
// 0: no combine (head_size > 128).
constexpr int mfma_wg_fixup(int rows_per_tile, int head_size) {
    return head_size > 128 ? 0 : rows_per_tile == kMfmaHeads ? 1 : 2;
}

struct DecodeParams {
    void *out;                 // [num_seqs][num_heads][head_size], element type
    const void *q;             // [num_seqs][num_heads][head_size]
    // Per-sequence rows (the serving path, whose requests keep their own
    // query and output buffers): when set, sequence s's [num_heads][head_size]
    // query rows start at q_rows[s] and its output rows at o_rows[s], and
    // q / out are unused.
    const char *const *q_rows;
    char *const *o_rows;
    const void *k;             // paged K cache (element type)
    const void *v;             // paged V cache
    const int *block_tables;   // [num_seqs][max_blocks]
    const int *seq_lens;       // [num_seqs]
    float *ws_o;               // [num_waves*2][head_tile][head_size] fp32 partial outputs
    float *ws_ml;              // [num_waves*2][head_tile][2] (running max, running sum)
    int *ws_prefix;            // [num_seqs + 1] split units before each sequence (written by wg 0)
    long long kv_block_stride; // elements
    long long kv_head_stride;  // elements
    int num_seqs;
    int num_heads;
    int num_kv_heads;
    int group;                 // num_heads / num_kv_heads
    int head_tiles;            // ceil(group / head tile), 1 to 4
    int max_blocks;            // block-table row length
    int block_size;
    int bs_shift;              // log2(block_size)
    int max_ctx;               // max_blocks * block_size
    int num_waves;             // wavefronts of the partition kernel launch
    int min_tiles_per_wave;    // lower bound of tpw (>= 1), in split units
    int seg_cost;              // split units a segment costs on top of its tiles
    float scale_log2;          // scale * log2(e)
    int merge_per_segment;     // 1: merge with one workgroup per segment
    int segment_launch;        // 1 (VALU tile path, automatic plan, whole outputs): one
                               // round of workgroups over the segments
                               // (paged_decode_segment_kernel); num_waves is unused
    int segment_split;         // workgroups per segment under segment_launch (1, 2 or 4):
                               // with 1 the workgroup writes the rows and nothing else
                               // runs; above 1 workgroup j of a segment takes its tiles
                               // j, j + S, ... and leaves an fp32 partial in ws_o / ws_ml
                               // slot (segment * S + j), which
                               // paged_decode_segment_merge_kernel combines
    int pair_tiles;            // 1 (MFMA path, head_tiles == 2, wg_fix == 0): paired head
                               // tiles.  A segment is (sequence, kv head); the two
                               // wavefronts 2k, 2k + 1 of the launch walk the same stream-K
                               // range (range k of num_waves / 2), wavefront 2k + t
                               // computing head tile t, so both read each page at the same
                               // time on one CU.  Partial j of a cut segment whose first
                               // range is k0, head tile t: slot 2 (2 (k0 + j) + t) + (j == 0 ?
                               // the first range's slot : 0)
    int wg_fix;                // 1: the partition kernel combined each segment's pieces
                               // inside a workgroup (mfma_wg_fixup): partial j >= 1 of a
                               // segment is in slot 2 * kMfmaWavesPerGroup * (its
                               // workgroup), and a segment inside one workgroup is finished
    // Partial-output mode (cascade passes): when out_f32 is set, every
    // (sequence, head) row is written in fp32 to out_f32 (indexed like out)
    // together with its log-sum-exp in log2 units, m + log2(l), to
    // out_lse[seq * num_heads + head] (-inf for an empty row); out is unused.
    float *out_f32;
    float *out_lse;
    // fp16 states (the fused cascade launch over fp16 K/V): the rows of
    // partial-output mode go to out_h instead of out_f32, and the partials
    // of cut pieces to ws_h instead of ws_o, both normalized (o / l) in fp16
    // and indexed like the fp32 buffers; a partial's ws_ml pair is then
    // (m + log2 l, 1), or (-inf, 0) when empty.  This is the state format of
    // the reference's partition merge (element-type partial outputs with an
    // fp32 log-sum-exp, operators/flashinfer_adapter.cu:255-260), at half
    // the bytes of fp32 states.
    void *out_h;
    void *ws_h;
    int cached_seqs;           // sequences [0, cached_seqs) load K/V cacheable (pages read
                               // by several wavefronts close in time); the rest nontemporal
    int skip_empty;            // 1: the rows of empty sequences are left unwritten (their
                               // reader never reads them)
    // Prefix fold (cascade suffix pass): when fold_row is set, sequence s
    // with fold_row[s] >= 0 continues the attention of an earlier pass over
    // its shared prefix.  That pass left, for (kv head h, query head g of
    // the group), the normalized row fold_out[r * head_size ..] and its
    // log-sum-exp fold_lse[r] (log2 units) at r = v * fold_kr + h * fold_rows
    // + j with v, j = divmod(fold_row[s] + g, fold_rows).  Such a state is
    // the online softmax's (m = lse, l = 1, o = row): the piece that starts a
    // segment (token 0) begins from it instead of the empty state, and an
    // empty sequence outputs the prefix row.
    const int *fold_row;
    const float *fold_out;
    const float *fold_lse;
    int fold_rows;
    int fold_kr;
    // New-token fold (the serving path's one-request decode step, one
    // sequence): the partition kernel attends over the sequence's cached
    // tokens in partial-output mode, and the merge kernel (chunk grid) takes
    // every segment's state -- the finished row and its log-sum-exp, or its
    // partials -- folds in the step's new token, whose rows ([num_kv_heads]
    // [head_size], element type) are at nt_k / nt_v instead of in the cache
    // (score q . k_new, the online log-sum-exp update with v_new), and writes
    // the output rows to `out`.  The merge also writes the token's K/V rows
    // to its cache slot nt_slot, nt_page to *nt_table when the token opens a
    // page (nt_table not null), and nt_len to *nt_lens.
    int nt_fold;
    const void *nt_k;
    const void *nt_v;
    int *nt_table;
    int *nt_lens;
    int nt_slot;
    int nt_page;
    int nt_len;
    // Per-workgroup timestamps (wg_trace.h): written only by the kernels of
    // the instrumented measurement build (XHIP_WG_TRACE); null otherwise.
    unsigned long long *wg_trace;
};


}  // namespace xhip
