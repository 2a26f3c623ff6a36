// Attention of the cascade (prefix-aware) decode on the MFMA tile path, in
// two launches: both batches of the plan (paged_decode_cascade.h) in one
// partition launch, then one merge that combines every output row's suffix
// state with its prefix state.  With at most kInPlanGroupsMax groups (and
// LDS for two workgroups per CU) the partition launch also builds the plan
// itself (below); otherwise the plan kernels run first.
//
// Partition.  The workgroups of one launch are split between the prefix
// batch (two 32-row head tiles per (sequence, kv head), R = 2, paired: the
// two wavefronts of a pair walk the same stream-K range, one head tile each,
// so a shared page is loaded for its 64 (member, head) rows by one CU at one
// time) and the suffix batch (the members' own pages, head tiles of the
// caller's group), each running the ordinary MFMA partition body over its
// own stream-K plan.  Every workgroup scans the split units of
// both batches (LDS) and takes the same split: the prefix batch gets a share
// of the workgroups proportional to its wavefront-units (a prefix unit
// occupies a pair of wavefronts) weighted by kCascadeUnitCost, plus the
// workgroups the suffix plan would leave empty.  Measured on MI355X at
// config 5 (cascade step, in-kernel plan, one box): weights 0.65 / 0.75 /
// 0.85 gave 121.3-121.5 / 111.6-111.7 / 114.4-114.5 us (86 / 97 / 108 prefix
// workgroups of 512); without the empty suffix workgroups moved over, 0.85
// (99) gave 113.2-113.3 us.  The step is sensitive to the split: both
// batches' ranges grow by a unit at some workgroup counts.
// Run as two launches, the prefix batch (a few thousand short ranges) spent
// ~30 us mostly in latency while the device's bandwidth went unused; here
// its ranges stream beside the suffix batch's.  Both bodies run in
// partial-output mode: finished segments leave rows and their log-sum-exp,
// cut segments their partials, and the suffix batch no longer starts from
// the prefix result (that would make it wait for the prefix batch).  Over
// fp16 K/V these states are fp16 (DecodeParams::out_h, ws_h): at config 5
// the fp32 states were 15.4 MB written and 14.8 MB read back, and the step
// took 7 us longer (MI355X).  Over bf16 they stay fp32: a bf16 state keeps 8
// significant bits, too few where a prefix row and a suffix row of opposite
// sign nearly cancel.
//
// Merge.  One workgroup per suffix segment (sequence, kv head, head tile);
// for every float4 column of its rows the suffix state (finished row, or the
// partials of its cut segment) and the prefix state of the same query row
// (the prefix batch's row, or its partials) are combined by the online
// log-sum-exp rule and written as the output:
//   O = (2^(lse_p-M) O_p + 2^(lse_s-M) O_s) / (2^(lse_p-M) + 2^(lse_s-M)).
#pragma once

#include <hip/hip_ext.h>

#include <climits>
#include <cstdint>

#include "paged_decode_cascade.h"
#include "paged_decode_mfma.h"

namespace xhip {

// Weight of a prefix-batch split unit against a suffix-batch unit in the
// workgroup split, in percent.
#ifndef XHIP_CASCADE_UNIT_COST
#define XHIP_CASCADE_UNIT_COST 75
#endif
constexpr int kCascadeUnitCost = XHIP_CASCADE_UNIT_COST;

// Workgroups of the prefix body in a launch of G >= 2 workgroups, from the
// split units of the prefix (tp) and suffix (ts) batches: each batch with
// units gets at least one.  The suffix plan gives every wavefront
// ceil(ts / its wavefronts) units (at least min_tpw), which can leave its
// last workgroups nothing: those go to the prefix body, whose ranges get
// shorter while the suffix's stay the same.  Integer arithmetic only: every
// workgroup computes the same split.
__device__ __forceinline__ int cascade_prefix_groups(int tp, int ts, int G, int min_tpw) {
    if (tp <= 0) return 0;
    if (ts <= 0) return G;
    // a prefix unit occupies both wavefronts of a pair
    const long long a = 2LL * tp * kCascadeUnitCost, b = (long long)ts * 100;
    int gp = (int)((a * G + (a + b) / 2) / (a + b));
    gp = gp < 1 ? 1 : (gp > G - 1 ? G - 1 : gp);
    const int ws = (G - gp) * kMfmaWavesPerGroup;
    const int tpw = tiles_per_wave(ts, ws, min_tpw);
    const int used = (ts + tpw - 1) / tpw;  // suffix wavefronts with units
    gp += (ws - used) / kMfmaWavesPerGroup;
    return gp > G - 1 ? G - 1 : gp;
}

// LDS of the two bodies (one runs per workgroup): the prefix body's (paired
// 32-row tiles, no workgroup combine) and the suffix body's.
constexpr int kCascadeMergeLdsSeqs = 1024;

template <int D, int RS> union MfmaLdsPair {
    MfmaLds<D, 2, 0> a;
    MfmaLds<D, RS> b;
};

// Partition launch over both batches.  pp / ps are the prefix and suffix
// batches' plans; their num_waves is the whole launch's (gridDim.x *
// kMfmaWavesPerGroup).  Workgroup 0 also stores both unit prefixes and the
// prefix body's workgroup count (pp.ws_prefix[pp.num_seqs + 1]) for the
// merge.
template <int KV, int D, int RS>
__global__ __launch_bounds__(64 * kMfmaWavesPerGroup, 2) void paged_decode_cascade_mfma_kernel(
    const DecodeParams pp, const DecodeParams ps, const int *__restrict__ plens,
    const int *__restrict__ ptables, const int *__restrict__ slens,
    const int *__restrict__ stables) {
    constexpr int NW = kMfmaWavesPerGroup;
    extern __shared__ int pre[];  // prefix batch (pp.num_seqs + 1), then suffix batch
    __shared__ MfmaLdsPair<D, RS> sm;
    int *pre_p = pre, *pre_s = pre + pp.num_seqs + 1;
    batch_prefix<16, NW>(pp, pre_p);
    batch_prefix<16, NW>(ps, pre_s);
    const int G = gridDim.x;
    const int gp = cascade_prefix_groups(pre_p[pp.num_seqs], pre_s[ps.num_seqs], G,
                                         ps.min_tiles_per_wave);
    if (blockIdx.x == 0 && threadIdx.x == 0) pp.ws_prefix[pp.num_seqs + 1] = gp;
    // neighbouring logical workgroups share an XCD (and its L2).  (Giving
    // every XCD its share of prefix workgroups instead measured 0.5-1 us
    // slower.)
    const int l = xcd_local_block(blockIdx.x, G);
    if (l < gp)
        mfma_partition_body<KV, D, 2, true, kSrcBatch, KV == KV_F16>(pp, plens, ptables, pre_p, l,
                                                                      gp * NW, sm.a);
    else
        mfma_partition_body<KV, D, RS, false, kSrcBatch, KV == KV_F16>(
            ps, slens, stables, pre_s, l - gp, (G - gp) * NW, sm.b);
}

// In-kernel plan.  With at most kInPlanGroupsMax groups, every workgroup of
// the partition launch builds the plan from the caller's arrays in its own
// LDS, instead of two plan launches writing the batches to memory first:
//   1. the caller's lengths, group ids and prefix pages (one round trip);
//   2. members, as in the plan kernels: a group id in range whose prefix of
//      P pages (1 <= P <= max_blocks, P pages within the sequence) is
//      shared; each sequence's suffix length, first private page and split
//      units, scanned within each wavefront;
//   3. by wavefront 0, 64 groups at a time, each group's
//      ceil(members * G / rows) prefix-batch sequences (length, table row =
//      the group's lowest member, split units); by all, the suffix batch's
//      unit prefix;
//   4. the workgroup split.
// Every workgroup computes the same plan.  A prefix-batch piece finds the
// members its query rows belong to when it starts (mfma_load_q, kSrcPrefix):
// the members of a group are ranked in sequence order, so the rows a piece
// computes are the same members' in every workgroup.  Workgroup 0 also
// stores what the merge reads: both unit prefixes, the split and the
// batches' lengths; p_row, every member's first row in the prefix batch, is
// stored by the piece that starts its prefix-batch sequence (kv head 0), and
// -1 for every other sequence by workgroup 0.
// LDS ints of the in-kernel plan: B caller sequences, V prefix-batch
// sequences, NG groups.
__host__ __device__ constexpr long long inplan_lds_ints(long long B, long long V, long long NG) {
    return (V + 1) + (B + 1) + 3 * B + 6 * V + 3 * NG;
}

// Partition launch over both batches with the in-kernel plan.  pp / ps are
// the batches as the merge reads them (their seq_lens: workspace arrays this
// kernel's workgroup 0 fills); lens / tables / pgroup / pblocks are the
// caller's arrays, ps.q / ps.q_rows its query rows.
template <int KV, int D, int RS>
__global__ __launch_bounds__(64 * kMfmaWavesPerGroup, 2) void paged_decode_cascade_inplan_kernel(
    const DecodeParams pp, const DecodeParams ps, const int *__restrict__ lens,
    const int *__restrict__ tables, const int *__restrict__ pgroup,
    const int *__restrict__ pblocks, int num_groups, int *__restrict__ p_row) {
    constexpr int NW = kMfmaWavesPerGroup, NT = 64 * NW;
    extern __shared__ int lds[];
    __shared__ MfmaLdsPair<D, RS> sm;
    __shared__ int s_part[NW];
    __shared__ int s_win[NW][2 * kMfmaHeads];  // prefix pieces' members (mfma_load_q)
    const int B = ps.num_seqs, V = pp.num_seqs, NG = num_groups;
    const int G = ps.group, rows = pp.group, bsz = ps.block_size;
    int *pre_p = lds;
    int *pre_s = pre_p + V + 1;
    int *slen = pre_s + B + 1, *soff = slen + B, *grp = soff + B;
    int *vlen = grp + B, *vrow = vlen + V, *vdesc = vrow + V;
    int *gP = vdesc + 4 * V, *gcnt = gP + NG, *gfirst = gcnt + NG;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    XHIP_WG_BEGIN(pp);

    // 1. (every prefix-batch sequence unused until step 3)
    for (int s = tid; s < B; s += NT) {
        slen[s] = min(max(lens[s], 0), ps.max_ctx);
        grp[s] = pgroup[s];
    }
    for (int g = tid; g < NG; g += NT) {
        gP[g] = pblocks[g];
        gcnt[g] = 0;
        gfirst[g] = INT_MAX;
    }
    for (int v = tid; v < V; v += NT) {
        vlen[v] = 0;
        vrow[v] = 0;
        vdesc[4 * v] = v;
        vdesc[4 * v + 1] = 0;
        vdesc[4 * v + 2] = 0;
        vdesc[4 * v + 3] = -1;
    }
    __syncthreads();
    XHIP_WG_STAMP(pp, 16);
    // 2. (thread t takes sequences [t * per, (t + 1) * per), as batch_prefix)
    const int per = (B + NT - 1) / NT;
    const int segs_s = seq_segments(ps);
    int ls = 0;
    for (int i = 0; i < per; i++) {
        const int s = tid * per + i;
        if (s < B) {
            const int g = grp[s], L = slen[s];
            int P = 0;
            if (g >= 0 && g < NG) {
                P = gP[g];
                if (P < 1 || P > ps.max_blocks || (long long)P * bsz > L) P = 0;
            }
            grp[s] = P > 0 ? g : -1;
            soff[s] = P;
            slen[s] = L - P * bsz;
            if (P > 0) {
                atomicAdd(&gcnt[g], 1);
                atomicMin(&gfirst[g], s);
            }
            const int t = segment_units(ps, (L - P * bsz + 15) >> 4) * segs_s;
            pre_s[s] = t;
            ls += t;
        }
    }
    int is = ls;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(is, off);
        if (lane >= off) is += u;
    }
    if (lane == 63) s_part[wave] = is;
    __syncthreads();
    XHIP_WG_STAMP(pp, 17);
    // 3. (groups 64 at a time, lane g taking group g0 + g)
    if (wave == 0) {
        int vt = 0, tp = 0;  // prefix-batch sequences and units of the groups so far
        for (int g0 = 0; g0 < NG; g0 += 64) {
            const int g = g0 + lane;
            const int n = g < NG ? gcnt[g] : 0;
            const int nv = (n * G + rows - 1) / rows;
            const int u = n > 0 ? segment_units(pp, (gP[g] * bsz + 15) >> 4) * seq_segments(pp) : 0;
            int sv = nv, su = nv * u;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int a = __shfl_up(sv, off), b = __shfl_up(su, off);
                if (lane >= off) {
                    sv += a;
                    su += b;
                }
            }
            const int vb = vt + sv - nv, pb = tp + su - nv * u;
            for (int k = 0; k < nv; k++) {
                const int v = vb + k;
                vlen[v] = gP[g] * bsz;
                vrow[v] = gfirst[g];
                vdesc[4 * v] = vb;
                vdesc[4 * v + 1] = n;
                vdesc[4 * v + 3] = g;
                pre_p[v] = pb + k * u;
            }
            vt += __builtin_amdgcn_readlane(sv, 63);
            tp += __builtin_amdgcn_readlane(su, 63);
        }
        for (int v = vt + lane; v <= V; v += 64) pre_p[v] = tp;  // unused, and the total
    }
    {
        int base = 0;
#pragma unroll
        for (int k = 0; k < NW - 1; k++) base += k < wave ? s_part[k] : 0;
        int run = base + is - ls;
        for (int i = 0; i < per; i++) {
            const int s = tid * per + i;
            if (s < B) {
                const int t = pre_s[s];
                pre_s[s] = run;
                run += t;
            }
        }
        if (tid == NT - 1) pre_s[B] = base + is;
    }
    __syncthreads();
    XHIP_WG_STAMP(pp, 18);
    // 4.
    const int Gw = gridDim.x;
    const int gp = cascade_prefix_groups(pre_p[V], pre_s[B], Gw, ps.min_tiles_per_wave);
    const int l = xcd_local_block(blockIdx.x, Gw);
    if (blockIdx.x == 0) {
        for (int v = tid; v <= V; v += NT) pp.ws_prefix[v] = pre_p[v];
        for (int q = tid; q <= B; q += NT) ps.ws_prefix[q] = pre_s[q];
        if (tid == 0) pp.ws_prefix[V + 1] = gp;
        for (int v = tid; v < V; v += NT) const_cast<int *>(pp.seq_lens)[v] = vlen[v];
        for (int q = tid; q < B; q += NT) {
            const_cast<int *>(ps.seq_lens)[q] = slen[q];
            if (grp[q] < 0) p_row[q] = -1;
        }
    }
    const CascadeLdsPlan cp{slen,  soff,       vlen, vrow, vdesc,         grp,  &s_win[0][0],
                            p_row, (const char *)ps.q, ps.q_rows, ps.num_heads, G, rows, B};
    XHIP_WG_STAMP(pp, 1);
    XHIP_WG_PUT(pp, 3, (unsigned long long)l | ((unsigned long long)(l < gp ? 1 : 2) << 32));
    if (l < gp)
        mfma_partition_body<KV, D, 2, true, kSrcPrefix, KV == KV_F16>(
            pp, nullptr, tables, pre_p, l, gp * NW, sm.a, &cp);
    else
        mfma_partition_body<KV, D, RS, false, kSrcSuffix, KV == KV_F16>(
            ps, nullptr, tables, pre_s, l - gp, (Gw - gp) * NW, sm.b, &cp);
    XHIP_WG_FLUSH(pp);
}

// (m, l, acc) <- (m, l, acc) (+) a finished row: the state (lse, 1, row).
__device__ __forceinline__ void absorb_row(float lse, const f32x4 &row, float &m, float &l,
                                           f32x4 &acc) {
    const float M = fmaxf(m, lse);
    const float Ms = (M == -INFINITY) ? 0.0f : M;
    const float a = fast_exp2(m - Ms), w = fast_exp2(lse - Ms);
    l = l * a + w;
    acc = acc * a + row * w;
    m = M;
}

// The state of one float4 column of a segment of batch p: its partials when
// the partition left the segment cut, else its finished row.  seg is the
// segment's index within its sequence, hrow the column's head in the
// segment's tile (GT heads), c the float4 column in the head; pair_ht >= 0:
// p's head tiles are paired (DecodeParams::pair_tiles) and the column is in
// head tile pair_ht.  HS: the states are fp16 (DecodeParams::out_h, ws_h).
template <int GT, int D, bool HS>
__device__ __forceinline__ void segment_state(const DecodeParams &p, int s, int L, int seg,
                                              int pre_s, int total, int waves, size_t row, int hrow,
                                              int c, float &m, float &l, f32x4 &acc,
                                              int pair_ht = -1) {
    const int Ts = (L + 15) / 16;
    const int seg_start = pre_s + seg * segment_units(p, Ts);
    PartialSlots ps;
    const bool cut =
        pair_ht >= 0
            ? segment_partials_paired(seg_start, seg_start + p.seg_cost, Ts,
                                      tiles_per_wave(total, waves >> 1, p.min_tiles_per_wave),
                                      pair_ht, ps)
            : segment_partials<kMfmaWavesPerGroup>(
                  p, seg_start, seg_start + p.seg_cost, Ts,
                  tiles_per_wave(total, waves, p.min_tiles_per_wave), ps);
    if (cut) {
        merge_partials<GT, D, 8, HS>(p, ps, 0, 1, hrow * 2, hrow * D + c * 4, m, l, acc);
    } else {
        const float lse = p.out_lse[row];
        const f32x4 o = HS ? unpack_h4(*(const u32x2 *)((const char *)p.out_h + (row * D + c * 4) * 2))
                           : *(const f32x4 *)(p.out_f32 + row * D + c * 4);
        absorb_row(lse, o, m, l, acc);
    }
}

// Merge over every suffix segment (sequence s, kv head, head tile of GTS
// heads), NT threads striding over its float4 columns, writing the output
// rows of ps (ps.out or ps.o_rows; its partial-output buffers hold the
// suffix states).  p_row[s] is the row,
// in the prefix batch's rows of a kv head laid end to end (`rows` per
// prefix-batch sequence), of s's first query head; -1: s has no prefix.
template <int KV, int D, int GTS, int NT>
__global__ __launch_bounds__(NT) void paged_decode_cascade_merge_kernel(
    const DecodeParams pp, const DecodeParams ps, const int *__restrict__ p_row, int rows) {
    XHIP_MERGE_SCOPE(pp);
    constexpr int C4 = D / 4;
    constexpr int NW = kMfmaWavesPerGroup;
    constexpr int GTP = 2 * kMfmaHeads;
    constexpr bool HS = KV == KV_F16;  // fp16 states (set by the host for fp16 K/V)
    // The prefix batch's lengths and unit prefixes, loaded with the first
    // round trip (a prefix batch of up to kCascadeMergeLdsSeqs sequences), so
    // finding a column's prefix segment takes no round trip of its own.
    __shared__ int l_vlen[kCascadeMergeLdsSeqs], l_vpre[kCascadeMergeLdsSeqs];
    const bool v_lds = pp.num_seqs <= kCascadeMergeLdsSeqs;
    if (v_lds) {
        for (int v = threadIdx.x; v < pp.num_seqs; v += NT) {
            l_vlen[v] = seq_len_of(pp, v);
            l_vpre[v] = pp.ws_prefix[v];
        }
    }
    const int segs = ps.num_kv_heads * ps.head_tiles;
    const int s = blockIdx.x / segs;
    const int seg = blockIdx.x - s * segs;
    const int kvh = seg / ps.head_tiles;
    const int g0 = (seg - kvh * ps.head_tiles) * GTS;
    const int nh = min(GTS, ps.group - g0);
    const int ncols = nh * C4;
    // the scalars, requested together
    const int Ls = seq_len_of(ps, s);
    const int fb = p_row[s];
    const int tot_s = ps.ws_prefix[ps.num_seqs];
    const int pre_s = ps.ws_prefix[s];
    const int tot_p = pp.ws_prefix[pp.num_seqs];
    const int gp = pp.ws_prefix[pp.num_seqs + 1];
    asm volatile("" ::"s"(Ls), "s"(fb), "s"(tot_s), "s"(pre_s), "s"(tot_p), "s"(gp));
    __syncthreads();
    const int G = ps.num_waves / NW;
    const size_t srow0 = (size_t)s * ps.num_heads + (size_t)kvh * ps.group + g0;
    for (int col = threadIdx.x; col < ncols; col += NT) {
        const int h = col / C4, c = col - h * C4;
        float m = -INFINITY, l = 0.0f;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        if (Ls > 0)
            segment_state<GTS, D, HS>(ps, s, Ls, seg, pre_s, tot_s, (G - gp) * NW, srow0 + h, h,
                                      c, m, l, acc);
        if (fb >= 0) {
            const int q = fb + g0 + h;
            const int v = q / rows, j = q - v * rows;
            const int Lv = v_lds ? l_vlen[v] : seq_len_of(pp, v);
            if (Lv > 0) {
                const int htp = j / GTP;
                const size_t prow = (size_t)v * pp.num_heads + (size_t)kvh * rows + j;
                segment_state<GTP, D, HS>(pp, v, Lv, kvh, v_lds ? l_vpre[v] : pp.ws_prefix[v],
                                          tot_p, gp * NW, prow, j - htp * GTP, c, m, l, acc, htp);
            }
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        char *orow = o_row(ps, s, kvh * ps.group + g0 + h, D, 2);
#pragma unroll
        for (int e = 0; e < 4; e++) store_elem<KV>(orow, c * 4 + e, acc[e] * inv);
    }
}

template <int KV, int D, int RS>
static hipError_t launch_cascade_attn_rs(const DecodeParams &pp, const DecodeParams &ps,
                                         const int *p_row, int rows, const CascadeInPlan *ip,
                                         hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
    const unsigned grid = (unsigned)(ps.num_waves / kMfmaWavesPerGroup);
    const dim3 block(64 * kMfmaWavesPerGroup);
    // the merge reads fp16 states exactly when the K/V are fp16
    const bool hs = KV == KV_F16;
    if ((pp.out_h != nullptr) != hs || (ps.out_h != nullptr) != hs || (pp.ws_h != nullptr) != hs ||
        (ps.ws_h != nullptr) != hs)
        return hipErrorInvalidValue;
    if (ip) {
        const size_t lds =
            (size_t)inplan_lds_ints(ps.num_seqs, pp.num_seqs, ip->num_groups) * sizeof(int);
        auto kernel = paged_decode_cascade_inplan_kernel<KV, D, RS>;
        int *prow = const_cast<int *>(p_row);
        if (ev_start || ev_stop)
            hipExtLaunchKernelGGL(kernel, dim3(grid), block, (std::uint32_t)lds, st, ev_start,
                                  ev_stop, 0u, pp, ps, ip->lens, ip->tables, ip->prefix_group,
                                  ip->prefix_blocks, ip->num_groups, prow);
        else
            hipLaunchKernelGGL(kernel, dim3(grid), block, lds, st, pp, ps, ip->lens, ip->tables,
                               ip->prefix_group, ip->prefix_blocks, ip->num_groups, prow);
    } else {
        const size_t lds = (size_t)(pp.num_seqs + ps.num_seqs + 2) * sizeof(int);
        auto kernel = paged_decode_cascade_mfma_kernel<KV, D, RS>;
        if (ev_start || ev_stop)
            hipExtLaunchKernelGGL(kernel, dim3(grid), block, (std::uint32_t)lds, st, ev_start,
                                  ev_stop, 0u, pp, ps, pp.seq_lens, pp.block_tables, ps.seq_lens,
                                  ps.block_tables);
        else
            hipLaunchKernelGGL(kernel, dim3(grid), block, lds, st, pp, ps, pp.seq_lens,
                               pp.block_tables, ps.seq_lens, ps.block_tables);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned segs = (unsigned)(ps.num_seqs * ps.num_kv_heads * ps.head_tiles);
    paged_decode_cascade_merge_kernel<KV, D, kMfmaHeads * RS, 128>
        <<<segs, 128, 0, st>>>(pp, ps, p_row, rows);
    return hipGetLastError();
}

template <int KV, int D>
static const void *cascade_fn(int rs, bool inplan) {
    if (inplan) {
        if (rs == 1)
            return reinterpret_cast<const void *>(&paged_decode_cascade_inplan_kernel<KV, D, 1>);
        if (rs == 2)
            return reinterpret_cast<const void *>(&paged_decode_cascade_inplan_kernel<KV, D, 2>);
        return nullptr;
    }
    if (rs == 1) return reinterpret_cast<const void *>(&paged_decode_cascade_mfma_kernel<KV, D, 1>);
    if (rs == 2) return reinterpret_cast<const void *>(&paged_decode_cascade_mfma_kernel<KV, D, 2>);
    return nullptr;
}

#define XHIP_FOR_CASCADE_HEAD_SIZES(X) X(32) X(64) X(96) X(128)

template <int KV>
static int cascade_occupancy_dtype(int head_size, int rs, bool inplan, size_t lds_bytes) {
    const void *fn = nullptr;
    switch (head_size) {
#define XHIP_CASE(d) case d: fn = cascade_fn<KV, d>(rs, inplan); break;
        XHIP_FOR_CASCADE_HEAD_SIZES(XHIP_CASE)
#undef XHIP_CASE
    default: break;
    }
    if (!fn) return 0;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 64 * kMfmaWavesPerGroup,
                                                     lds_bytes) != hipSuccess)
        return 0;
    return blocks;
}

template <int KV>
static hipError_t launch_cascade_attn_dtype(const DecodeParams &pp, const DecodeParams &ps,
                                            const int *p_row, int rows, int head_size,
                                            int rs, const CascadeInPlan *ip, hipStream_t st,
                                            hipEvent_t ev_start, hipEvent_t ev_stop) {
    switch (head_size) {
#define XHIP_CASE(d)                                                                          \
    case d:                                                                                   \
        if (rs == 1)                                                                          \
            return launch_cascade_attn_rs<KV, d, 1>(pp, ps, p_row, rows, ip, st, ev_start,    \
                                                    ev_stop);                                 \
        if (rs == 2)                                                                          \
            return launch_cascade_attn_rs<KV, d, 2>(pp, ps, p_row, rows, ip, st, ev_start,    \
                                                    ev_stop);                                 \
        return hipErrorInvalidValue;
        XHIP_FOR_CASCADE_HEAD_SIZES(XHIP_CASE)
#undef XHIP_CASE
    default: return hipErrorInvalidValue;
    }
}

}  // namespace xhip
