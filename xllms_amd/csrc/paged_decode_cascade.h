// Prefix-aware (cascade) decode: launch parameters and launchers of the plan
// and detection kernels (paged_decode_cascade.hip) and of the attention over
// the plan's two batches on the MFMA tile path (paged_decode_cascade_attn.h).
// Other tile paths run the attention through the ordinary partition + merge
// kernels twice: once on the prefix batch, and once on the suffix batch,
// which starts every member's segments from its prefix result
// (DecodeParams::fold_row) and writes the output.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "paged_decode_params.h"

namespace xhip {

// Query rows per kv head of a prefix-batch sequence are a multiple of the
// MFMA head tile: one wavefront serves 16 (member, head) rows of a group per
// page.
constexpr int kCascadeRows = 16;
// Sequences one detection workgroup handles (LDS hash table).
constexpr int kCascadeMaxSeqs = 4096;

struct CascadeParams {
    // caller's batch
    const int *block_tables;   // [num_seqs][max_blocks]
    const int *seq_lens;       // [num_seqs]
    const void *q;             // [num_seqs][num_heads][head_size]
    const char *const *q_rows; // non-null: sequence s's query rows start at q_rows[s] (q unused)
    void *out;                 // [num_seqs][num_heads][head_size], element type
    const int *prefix_group;   // [num_seqs] group id < max_groups, or -1
    const int *prefix_blocks;  // [max_groups] shared full pages of each group
    int num_seqs, num_heads, num_kv_heads, group, head_size, elem_bytes, kv_dtype;
    int max_blocks, block_size, max_ctx;
    int max_groups;
    int rows;                  // R: query rows per kv head of a prefix-batch sequence
                               // (16 * ceil(G / 16))
    int v_max;                 // prefix-batch sequences reserved (an upper bound)
    // plan (workspace)
    int *g_count;              // [max_groups] members
    int *g_first;              // [max_groups] lowest member
    int *g_vbase;              // [max_groups] first prefix-batch sequence
    int *g_moff;               // [max_groups] offset of the group in member_seq
    int *member_seq;           // [num_seqs] members of every group, by group
    int *rank;                 // [num_seqs] member rank inside its group (-1: none)
    int *v_group;              // [v_max] group of a prefix-batch sequence (-1: unused)
    int *v_lens;               // [v_max]
    int *v_bt;                 // [v_max][max_blocks]
    void *v_q;                 // [v_max][num_kv_heads * rows][head_size]
    int *s_lens;               // [num_seqs] suffix lengths
    int *s_bt;                 // [num_seqs][max_blocks] suffix block tables
    int *p_row;                // [num_seqs] fold base of each member: the row index, in
                               // the group's prefix-batch rows laid end to end, of its
                               // first query head (g_vbase * rows + rank * group); -1
    // Descriptors the first plan kernel writes for the gather, so that each
    // gather item waits on one load of them instead of a chain of lookups:
    int *v_desc;               // [v_max][8] group (-1: unused), its g_vbase, g_count,
                               // g_moff, g_first, prefix_blocks, 0, 0
    int *s_pblk;               // [num_seqs] shared prefix pages of a member (0: none)
};

// Plan: group membership and the prefix / suffix batches.
hipError_t launch_cascade_plan(const CascadeParams &c, hipStream_t stream);

// The caller's arrays for the cascade's in-kernel plan (at most
// kInPlanGroupsMax groups, and LDS for two workgroups per CU): the partition
// launch builds both batches from them in LDS, with no plan launches
// (paged_decode_cascade_attn.h).
// Wavefront 0 of every workgroup lays the groups out 64 at a time; beyond
// 256 groups the plan kernels, which do it with 1024 threads once, are the
// shorter path.
constexpr int kInPlanGroupsMax = 256;
struct CascadeInPlan {
    const int *lens;           // [num_seqs] caller's sequence lengths
    const int *tables;         // [num_seqs][max_blocks] caller's block tables
    const int *prefix_group;   // [num_seqs]
    const int *prefix_blocks;  // [num_groups]
    int num_groups;            // max_groups, <= kInPlanGroupsMax
};

// Attention of the cascade on the MFMA tile path (paged_decode_cascade_attn.h):
// the prefix batch pp (32-row head tiles) and the suffix batch ps (head
// tiles of 16 * rs rows) in one partition launch of ps.num_waves
// wavefronts (>= 8), then the merge that writes ps's output rows (ps.out or
// ps.o_rows) from both.  ip null: the plan kernels built both batches
// (launch_cascade_plan); else the partition launch plans them itself from
// ip, and pp.seq_lens, ps.seq_lens and p_row are workspace it fills for the
// merge.  lds_bytes: the launch's dynamic LDS (inplan_lds_bytes with ip).
// head_size 32, 64, 96 or 128; hipErrorInvalidValue otherwise.
size_t inplan_lds_bytes(int num_seqs, int v_max, int num_groups);
int cascade_attn_occupancy_f16(int head_size, int rs, bool inplan, size_t lds_bytes);
int cascade_attn_occupancy_bf16(int head_size, int rs, bool inplan, size_t lds_bytes);
hipError_t launch_cascade_attn_f16(const DecodeParams &pp, const DecodeParams &ps,
                                   const int *p_row, int rows, int head_size, int rs,
                                   const CascadeInPlan *ip, hipStream_t stream,
                                   hipEvent_t ev_start, hipEvent_t ev_stop);
hipError_t launch_cascade_attn_bf16(const DecodeParams &pp, const DecodeParams &ps,
                                    const int *p_row, int rows, int head_size, int rs,
                                    const CascadeInPlan *ip, hipStream_t stream,
                                    hipEvent_t ev_start, hipEvent_t ev_stop);

// Detection of shared prefixes from the block tables (one workgroup,
// num_seqs <= kCascadeMaxSeqs): sequences whose first page is the same
// physical page form a group (at least two members); the group's prefix is
// the longest run of leading pages every member shares with the group's
// lowest-numbered member, counting only pages full in both.  Writes
// prefix_group[num_seqs] (-1: none), prefix_blocks[num_groups] and
// *num_groups (all device memory).
hipError_t launch_prefix_detect(const int *block_tables, const int *seq_lens, int num_seqs,
                                int max_blocks, int block_size, int *prefix_group,
                                int *prefix_blocks, int *num_groups, hipStream_t stream);

}  // namespace xhip
