// Prefix-aware (cascade) decode on gfx950: plan and detection kernels.  No
// counterpart in the reference (its decode reads every sequence's pages,
// shared or not); see paged_decode_cascade.h.
//
// A group is a set of sequences whose first P pages are the same physical
// pages.  Attention over a group's shared prefix is computed once per page
// for all of its members: the plan gathers the members' query rows, R per kv
// head, into the sequences of a prefix batch whose block table is the shared
// prefix, and shifts every member's own block table past the prefix into a
// suffix batch.  On the MFMA tile path both batches run in one partition
// launch and one merge combines each member's prefix and suffix states
// (paged_decode_cascade_attn.h).  Elsewhere the ordinary partition + merge
// kernels run the prefix batch in partial-output mode (fp32 rows plus their
// log-sum-exp lse_p; prefix pages loaded cacheable, since the rows of a
// group read them close in time), then the suffix batch with a prefix fold:
// (lse_p, O_p) is the online softmax state (m = lse_p, l = 1, o = O_p), so a
// member's suffix segments start from it and the suffix pass writes
//   O = (2^(lse_p-m) O_p + sum_t 2^(s_t-m) v_t) / (2^(lse_p-m) + sum_t 2^(s_t-m)),
// the attention over prefix and suffix together.  A row of the prefix batch
// depends only on its own query (the MFMA tile
// computes every (token, row) score and every (dim, row) output from that
// row alone), so where a member lands among the rows does not change its
// result, and rows no member uses are never read.
#include <hip/hip_runtime.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>

#include "paged_decode_cascade.h"
#include "paged_decode_kernels.h"

namespace xhip {

namespace {

constexpr int kPlanThreads = 1024;

typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int clamp_len(int L, int max_ctx) {
    return L < 0 ? 0 : (L > max_ctx ? max_ctx : L);
}

// Shared prefix pages of sequence s under the caller's grouping, or 0 when
// the entry is out of range (then the sequence is decoded without cascade).
__device__ __forceinline__ int member_prefix(const CascadeParams &c, int s, int *group) {
    const int g = c.prefix_group[s];
    *group = -1;
    if (g < 0 || g >= c.max_groups) return 0;
    const int P = c.prefix_blocks[g];
    if (P < 1 || P > c.max_blocks) return 0;
    if ((long long)P * c.block_size > clamp_len(c.seq_lens[s], c.max_ctx)) return 0;
    *group = g;
    return P;
}

// Exclusive scan, in place, of n ints of global memory by one workgroup of
// kPlanThreads threads; returns the total to every thread.
__device__ int block_exclusive_scan(int *a, int n, int *part) {
    const int tid = threadIdx.x;
    const int per = (n + kPlanThreads - 1) / kPlanThreads;
    const int i0 = tid * per;
    int local = 0;
    for (int i = i0; i < i0 + per && i < n; i++) local += a[i];
    part[tid] = local;
    __syncthreads();
    for (int off = 1; off < kPlanThreads; off <<= 1) {
        const int v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int run = part[tid] - local;
    for (int i = i0; i < i0 + per && i < n; i++) {
        const int v = a[i];
        a[i] = run;
        run += v;
    }
    const int total = part[kPlanThreads - 1];
    __syncthreads();
    return total;
}

// The gather's descriptors (CascadeParams::v_desc, s_pblk) and the suffix
// batch's per-member lengths and fold bases, written by part 1.
__device__ __forceinline__ void write_v_desc(const CascadeParams &c, int v, int g, int vbase,
                                             int count, int moff, int first) {
    i32x4_t *d = (i32x4_t *)(c.v_desc + (size_t)v * 8);
    d[0] = i32x4_t{g, vbase, count, moff};
    d[1] = i32x4_t{first, g >= 0 ? c.prefix_blocks[g] : 0, 0, 0};
}

// Member s with P shared pages (0: none; then vbase and rank are unused).
__device__ __forceinline__ void write_s_desc(const CascadeParams &c, int s, int P, int vbase,
                                             int rank) {
    c.s_pblk[s] = P;
    c.s_lens[s] = P > 0 ? clamp_len(c.seq_lens[s], c.max_ctx) - P * c.block_size : c.seq_lens[s];
    c.p_row[s] = P > 0 ? vbase * c.rows + rank * c.group : -1;
}

// Plan, part 1 (one workgroup): members, ranks, and where every group's rows
// go in the prefix batch.
__global__ __launch_bounds__(kPlanThreads) void cascade_plan_meta_kernel(const CascadeParams c) {
    __shared__ int part[kPlanThreads];
    const int tid = threadIdx.x;
    const int B = c.num_seqs, NG = c.max_groups;
    for (int g = tid; g < NG; g += kPlanThreads) {
        c.g_count[g] = 0;
        c.g_first[g] = INT_MAX;
    }
    __syncthreads();
    for (int s = tid; s < B; s += kPlanThreads) {
        int g;
        member_prefix(c, s, &g);
        int r = -1;
        if (g >= 0) {
            r = atomicAdd(&c.g_count[g], 1);
            atomicMin(&c.g_first[g], s);
        }
        c.rank[s] = r;
    }
    __syncthreads();
    // prefix sequences of every group: ceil(members * group / rows)
    for (int g = tid; g < NG; g += kPlanThreads) {
        c.g_vbase[g] = (c.g_count[g] * c.group + c.rows - 1) / c.rows;
        c.g_moff[g] = c.g_count[g];
    }
    __syncthreads();
    const int vt = block_exclusive_scan(c.g_vbase, NG, part);
    block_exclusive_scan(c.g_moff, NG, part);
    for (int s = tid; s < B; s += kPlanThreads) {
        const int r = c.rank[s];
        if (r >= 0) c.member_seq[c.g_moff[c.prefix_group[s]] + r] = s;
    }
    for (int g = tid; g < NG; g += kPlanThreads) {
        const int n = (c.g_count[g] * c.group + c.rows - 1) / c.rows;
        for (int k = 0; k < n; k++) {
            c.v_group[c.g_vbase[g] + k] = g;
            write_v_desc(c, c.g_vbase[g] + k, g, c.g_vbase[g], c.g_count[g], c.g_moff[g],
                         c.g_first[g]);
        }
    }
    for (int v = vt + tid; v < c.v_max; v += kPlanThreads) {
        c.v_group[v] = -1;
        write_v_desc(c, v, -1, 0, 0, 0, 0);
    }
    for (int s = tid; s < B; s += kPlanThreads) {
        int g;
        const int P = c.rank[s] >= 0 ? member_prefix(c, s, &g) : 0;
        write_s_desc(c, s, P, P > 0 ? c.g_vbase[g] : 0, c.rank[s]);
    }
}

// Plan, part 1 with the work arrays in LDS (batches of up to kPlanLdsSeqs
// sequences and kPlanLdsGroups groups): the same results as
// cascade_plan_meta_kernel, which keeps them in global memory and so waits
// for a global round trip at each of its ~10 steps.  Here the inputs are read
// once and the results stored at the end.
constexpr int kPlanLdsGroups = 1024;
constexpr int kPlanLdsSeqs = 4096;

__global__ __launch_bounds__(kPlanThreads) void cascade_plan_meta_lds_kernel(const CascadeParams c) {
    __shared__ int part[kPlanThreads];
    __shared__ int l_count[kPlanLdsGroups], l_first[kPlanLdsGroups];
    __shared__ int l_vbase[kPlanLdsGroups], l_moff[kPlanLdsGroups];
    __shared__ int l_group[kPlanLdsSeqs], l_rank[kPlanLdsSeqs];
    const int tid = threadIdx.x;
    const int B = c.num_seqs, NG = c.max_groups;
    for (int g = tid; g < NG; g += kPlanThreads) {
        l_count[g] = 0;
        l_first[g] = INT_MAX;
    }
    __syncthreads();
    for (int s = tid; s < B; s += kPlanThreads) {
        int g;
        member_prefix(c, s, &g);
        int r = -1;
        if (g >= 0) {
            r = atomicAdd(&l_count[g], 1);
            atomicMin(&l_first[g], s);
        }
        l_group[s] = g;
        l_rank[s] = r;
        c.rank[s] = r;
    }
    __syncthreads();
    // prefix sequences of every group: ceil(members * group / rows)
    for (int g = tid; g < NG; g += kPlanThreads) {
        l_vbase[g] = (l_count[g] * c.group + c.rows - 1) / c.rows;
        l_moff[g] = l_count[g];
    }
    __syncthreads();
    int vt;
    if (NG <= 64) {
        // one wavefront scans both arrays with shuffles (no workgroup barriers)
        if (tid < 64) {
            const int a = tid < NG ? l_vbase[tid] : 0, b = tid < NG ? l_moff[tid] : 0;
            int sa = a, sb = b;
            for (int off = 1; off < 64; off <<= 1) {
                const int ua = __shfl_up(sa, off), ub = __shfl_up(sb, off);
                if (tid >= off) {
                    sa += ua;
                    sb += ub;
                }
            }
            if (tid < NG) {
                l_vbase[tid] = sa - a;
                l_moff[tid] = sb - b;
            }
            if (tid == 63) part[0] = sa;
        }
        __syncthreads();
        vt = part[0];
    } else {
        vt = block_exclusive_scan(l_vbase, NG, part);
        block_exclusive_scan(l_moff, NG, part);
    }
    for (int g = tid; g < NG; g += kPlanThreads) {
        c.g_count[g] = l_count[g];
        c.g_first[g] = l_first[g];
        c.g_vbase[g] = l_vbase[g];
        c.g_moff[g] = l_moff[g];
        const int n = (l_count[g] * c.group + c.rows - 1) / c.rows;
        for (int k = 0; k < n; k++) {
            c.v_group[l_vbase[g] + k] = g;
            write_v_desc(c, l_vbase[g] + k, g, l_vbase[g], l_count[g], l_moff[g], l_first[g]);
        }
    }
    for (int s = tid; s < B; s += kPlanThreads) {
        const int r = l_rank[s];
        const int g = l_group[s];
        if (r >= 0) c.member_seq[l_moff[g] + r] = s;
        write_s_desc(c, s, g >= 0 ? c.prefix_blocks[g] : 0, g >= 0 ? l_vbase[g] : 0, r);
    }
    for (int v = vt + tid; v < c.v_max; v += kPlanThreads) {
        c.v_group[v] = -1;
        write_v_desc(c, v, -1, 0, 0, 0, 0);
    }
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Plan, part 2 (grid-stride): the prefix batch (gathered query rows, block
// tables = the shared prefix, lengths) and the suffix batch (block tables
// shifted past the prefix, lengths).
__global__ __launch_bounds__(256) void cascade_plan_gather_kernel(const CascadeParams c) {
    const int R = c.rows;
    const int KR = c.num_kv_heads * R;
    const int CH = c.head_size * c.elem_bytes / 16;
    const size_t row_bytes = (size_t)c.head_size * c.elem_bytes;
    const long long n1 = (long long)c.v_max * KR * CH;
    const long long n2 = (long long)c.v_max * c.max_blocks;
    const long long n3 = (long long)c.num_seqs * c.max_blocks;
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n1 + n2 + n3;
         i += stride) {
        if (i < n1) {
            const int ch = (int)(i % CH);
            const long long row = i / CH;
            const int v = (int)(row / KR);
            const int hj = (int)(row - (long long)v * KR);
            // {group, its g_vbase, g_count, g_moff}
            const i32x4_t d = *(const i32x4_t *)(c.v_desc + (size_t)v * 8);
            if (d.x < 0) continue;  // unused: its length is 0, its rows are never read
            const int h = hj / R, j = hj - h * R;
            const int rig = (v - d.y) * R + j;
            const int r = rig / c.group, gq = rig - r * c.group;
            if (r >= d.z) continue;  // no member: never read
            const int s = c.member_seq[d.w + r];
            const size_t hrow = (size_t)h * c.group + gq;
            const char *src = c.q_rows ? c.q_rows[s] + hrow * row_bytes
                                       : (const char *)c.q + ((size_t)s * c.num_heads + hrow) * row_bytes;
            const size_t dst = ((size_t)v * KR + hj) * row_bytes + (size_t)ch * 16;
            *(u32x4_t *)((char *)c.v_q + dst) = *(const u32x4_t *)(src + (size_t)ch * 16);
        } else if (i < n1 + n2) {
            const long long k = i - n1;
            const int v = (int)(k / c.max_blocks), b = (int)(k - (long long)v * c.max_blocks);
            // {g_first, prefix pages} (0 pages when the sequence is unused)
            const i32x4_t d = *(const i32x4_t *)(c.v_desc + (size_t)v * 8 + 4);
            const int P = d.y;
            if (b == 0) c.v_lens[v] = P * c.block_size;
            if (b < P) c.v_bt[k] = c.block_tables[(size_t)d.x * c.max_blocks + b];
        } else {
            // (the suffix lengths and fold bases were written with s_pblk)
            const long long k = i - n1 - n2;
            const int s = (int)(k / c.max_blocks), b = (int)(k - (long long)s * c.max_blocks);
            const int P = c.s_pblk[s];
            c.s_bt[k] = b + P < c.max_blocks ? c.block_tables[(size_t)s * c.max_blocks + b + P]
                                              : -1;
        }
    }
}

// Detection (one workgroup): open-addressing hash table in LDS from a first
// page id to its group, then the shared run of every member against the
// group's lowest member.
constexpr int kDetectTable = 2 * kCascadeMaxSeqs;

__global__ __launch_bounds__(kPlanThreads) void prefix_detect_kernel(
    const int *block_tables, const int *seq_lens, int num_seqs, int max_blocks, int block_size,
    int *prefix_group, int *prefix_blocks, int *num_groups) {
    __shared__ int tkey[kDetectTable];   // first page id; later the group id of the slot
    __shared__ int tmin[kDetectTable];   // lowest member
    __shared__ int tcnt[kDetectTable];   // members
    __shared__ int tpre[kDetectTable];   // shared leading pages
    __shared__ int part[kPlanThreads];
    const int tid = threadIdx.x;
    const long long max_ctx = (long long)max_blocks * block_size;
    for (int h = tid; h < kDetectTable; h += kPlanThreads) {
        tkey[h] = -1;
        tmin[h] = INT_MAX;
        tcnt[h] = 0;
        tpre[h] = INT_MAX;
    }
    __syncthreads();
    auto len_of = [&](int s) {
        const int L = seq_lens[s];
        return L < 0 ? 0 : (L > max_ctx ? (int)max_ctx : L);
    };
    for (int s = tid; s < num_seqs; s += kPlanThreads) {
        const int key = len_of(s) >= block_size ? block_tables[(size_t)s * max_blocks] : -1;
        int slot = -1;
        if (key >= 0) {
            int h = (int)(((uint32_t)key * 2654435761u) >> 19) & (kDetectTable - 1);
            for (;;) {  // the table holds at most num_seqs <= kDetectTable / 2 keys
                const int old = atomicCAS(&tkey[h], -1, key);
                if (old == -1 || old == key) break;
                h = (h + 1) & (kDetectTable - 1);
            }
            atomicMin(&tmin[h], s);
            atomicAdd(&tcnt[h], 1);
            slot = h;
        }
        prefix_group[s] = slot;  // scratch until the last phase
    }
    __syncthreads();
    for (int s = tid; s < num_seqs; s += kPlanThreads) {
        const int slot = prefix_group[s];
        if (slot < 0 || tcnt[slot] < 2) continue;
        const int lead = tmin[slot];
        const int n = min(len_of(s), len_of(lead)) / block_size;
        const int *a = block_tables + (size_t)s * max_blocks;
        const int *b = block_tables + (size_t)lead * max_blocks;
        int P = 0;
        while (P < n && a[P] == b[P]) P++;
        atomicMin(&tpre[slot], P);
    }
    __syncthreads();
    // group ids: leaders of groups with >= 2 members and >= 1 shared page,
    // numbered in sequence order
    const int per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
    const int s0 = tid * per;
    int local = 0;
    for (int s = s0; s < s0 + per && s < num_seqs; s++) {
        const int slot = prefix_group[s];
        local += slot >= 0 && tmin[slot] == s && tcnt[slot] >= 2 && tpre[slot] >= 1;
    }
    part[tid] = local;
    __syncthreads();
    for (int off = 1; off < kPlanThreads; off <<= 1) {
        const int v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int id = part[tid] - local;
    for (int s = s0; s < s0 + per && s < num_seqs; s++) {
        const int slot = prefix_group[s];
        if (slot >= 0 && tmin[slot] == s && tcnt[slot] >= 2 && tpre[slot] >= 1) {
            tkey[slot] = id;
            prefix_blocks[id] = tpre[slot];
            id++;
        }
    }
    if (tid == kPlanThreads - 1) *num_groups = part[kPlanThreads - 1];
    __syncthreads();
    for (int s = tid; s < num_seqs; s += kPlanThreads) {
        const int slot = prefix_group[s];
        prefix_group[s] = (slot >= 0 && tcnt[slot] >= 2 && tpre[slot] >= 1) ? tkey[slot] : -1;
    }
}

unsigned grid_for(long long n) {
    long long b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    return (unsigned)(b > 0 ? b : 1);
}

}  // namespace

hipError_t launch_cascade_plan(const CascadeParams &c, hipStream_t stream) {
    if (c.max_groups <= kPlanLdsGroups && c.num_seqs <= kPlanLdsSeqs)
        cascade_plan_meta_lds_kernel<<<1, kPlanThreads, 0, stream>>>(c);
    else
        cascade_plan_meta_kernel<<<1, kPlanThreads, 0, stream>>>(c);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const long long n = (long long)c.v_max * c.num_kv_heads * c.rows *
                            (c.head_size * c.elem_bytes / 16) +
                        (long long)(c.v_max + c.num_seqs) * c.max_blocks;
    cascade_plan_gather_kernel<<<grid_for(n), 256, 0, stream>>>(c);
    return hipGetLastError();
}

hipError_t launch_prefix_detect(const int *block_tables, const int *seq_lens, int num_seqs,
                                int max_blocks, int block_size, int *prefix_group,
                                int *prefix_blocks, int *num_groups, hipStream_t stream) {
    prefix_detect_kernel<<<1, kPlanThreads, 0, stream>>>(block_tables, seq_lens, num_seqs,
                                                          max_blocks, block_size, prefix_group,
                                                          prefix_blocks, num_groups);
    return hipGetLastError();
}

}  // namespace xhip
