// gfx950 (CDNA4) kernels of the paged-decode attention.
//
// Memory-bound by design: every K/V byte of a (sequence, kv head) is read
// once, with 16-byte per-lane global loads that cover whole rows of a page,
// and the whole GQA group of query heads is served from that one read.
//
// Wavefront layout (wave64).  A K or V row of one token is head_size elements,
// i.e. NCH = head_size*elem_bytes/16 sixteen-byte chunks.  RL = next pow2 of
// NCH lanes share a row (lane `col` owns chunk col), and the wavefront holds
// TPL = 64/RL rows per load instruction, so one instruction reads TPL whole
// contiguous rows.  A tile is kLoadsPerTile such loads (TT = 4*TPL tokens; 16
// tokens = one 16-token page for fp16/bf16 d=128).  Each row group of lanes
// (the RL lanes of one `row`) keeps its own online-softmax state (running max
// m, running sum l, unnormalised output o) for every query head of the head
// tile, so the main loop needs no cross-row traffic at all: QK^T is a per-lane
// dot product (v_dot2_f32_f16 / v_dot2_f32_bf16 for 16-bit data, FMA for fp32)
// finished by a DPP butterfly inside the row (quad_perm, row_half_mirror,
// row_mirror), the softmax update is per lane, and PV is per-lane FMAs into the
// lane's own output columns.  The row states are merged once, at the end of
// the partition, with xor shuffles.
//
// Split-K.  The work is distributed stream-K style (paged_decode_params.h):
// each wavefront of one resident round owns an equal, contiguous range of
// the batch's tiles, so ragged lengths cannot leave a tail of idle CUs.  A
// segment finished inside one range is written directly; a segment cut by
// range boundaries leaves fp32 partials (m, l, o) that
// paged_decode_merge_kernel combines with the usual log-sum-exp rescale:
//   M = max_p m_p,  O = sum_p 2^(m_p-M) o_p / sum_p 2^(m_p-M) l_p.
// Scores are kept in log2 units (scale*log2(e) folded into the score) so the
// exponentials are single v_exp_f32 instructions.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "paged_decode_params.h"
#include "wg_trace.h"

namespace xhip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int KV> struct KvTraits;
template <> struct KvTraits<KV_F16> { static constexpr int kBytes = 2; };
template <> struct KvTraits<KV_BF16> { static constexpr int kBytes = 2; };
template <> struct KvTraits<KV_F32> { static constexpr int kBytes = 4; };

constexpr int pow2_ceil(int x) {
    int r = 1;
    while (r < x) r <<= 1;
    return r;
}

// Compile-time geometry of one (dtype, head_size) instantiation.
template <int KV, int D> struct Geometry {
    static constexpr int kElemBytes = KvTraits<KV>::kBytes;
    static constexpr int kVec = 16 / kElemBytes;           // elements per lane chunk
    static constexpr int kChunks = D / kVec;               // chunks per row
    static constexpr int kRowLanes = pow2_ceil(kChunks);   // lanes per row
    static constexpr int kRows = 64 / kRowLanes;           // rows per load
    static constexpr int kTileTokens = kRows * kLoadsPerTile;
    static_assert(D % kVec == 0, "head_size must fill whole 16-byte chunks");
    static_assert(kRowLanes <= 64, "row wider than a wavefront");
};

template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the RL lanes of a row (RL a power of two), result in every lane,
// for N independent values at once: each butterfly step is applied to all N
// before the next, so consecutive DPP instructions never read a register the
// previous instruction wrote (no DPP read-after-write stall).
template <int RL, int N> __device__ __forceinline__ void row_sum_n(float (&v)[N]) {
    if constexpr (RL >= 2) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += dpp_mov<0xB1>(v[i]);  // quad_perm [1,0,3,2]: lane ^ 1
    }
    if constexpr (RL >= 4) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += dpp_mov<0x4E>(v[i]);  // quad_perm [2,3,0,1]: lane ^ 2
    }
    if constexpr (RL >= 8) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += dpp_mov<0x141>(v[i]); // row_half_mirror: other quad
    }
    if constexpr (RL >= 16) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += dpp_mov<0x140>(v[i]); // row_mirror: other half row
    }
    if constexpr (RL >= 32) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += __shfl_xor(v[i], 16);
    }
    if constexpr (RL >= 64) {
#pragma unroll
        for (int i = 0; i < N; i++) v[i] += __shfl_xor(v[i], 32);
    }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Element i of a 16-byte chunk, by value.  (__builtin_bit_cast applied
// directly to a subscripted ext_vector element reads element 0 whatever i
// is, so every reinterpretation below goes through this copy.)
__device__ __forceinline__ uint32_t lane_word(u32x4 v, int i) {
    const uint32_t w = v[i];
    return w;
}

// acc + <k chunk, q chunk> over one 16-byte chunk.
template <int KV> __device__ __forceinline__ float chunk_dot(u32x4 k, u32x4 q, float acc) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (KV == KV_F16)
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, lane_word(k, i)),
                                         __builtin_bit_cast(f16x2, lane_word(q, i)), acc, false);
        else if constexpr (KV == KV_BF16)
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, lane_word(k, i)),
                                                  __builtin_bit_cast(bf16x2, lane_word(q, i)), acc,
                                                  false);
        else
            acc = fmaf(__builtin_bit_cast(float, lane_word(k, i)),
                       __builtin_bit_cast(float, lane_word(q, i)), acc);
    }
    return acc;
}

// Widen one 16-byte chunk to fp32 (exact for every dtype).
template <int KV, int VEC>
__device__ __forceinline__ void chunk_to_float(u32x4 v, float (&f)[VEC]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (KV == KV_F16) {
            f16x2 h = __builtin_bit_cast(f16x2, lane_word(v, i));
            f[2 * i] = (float)h.x;
            f[2 * i + 1] = (float)h.y;
        } else if constexpr (KV == KV_BF16) {
            const uint32_t w = lane_word(v, i);
            f[2 * i] = __builtin_bit_cast(float, w << 16);
            f[2 * i + 1] = __builtin_bit_cast(float, w & 0xFFFF0000u);
        } else {
            f[i] = __builtin_bit_cast(float, lane_word(v, i));
        }
    }
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two fp32 values narrowed to the 16-bit type, round to nearest even (NaN
// stays NaN), packed low = a, high = b: one v_cvt_pk_{f16,bf16}_f32 on
// gfx950 (a software bf16 rounding with a NaN test compiled to divergent
// branches and made the bf16 kernels issue ~25% more instructions).
template <int KV> __device__ __forceinline__ uint32_t pack16(float a, float b) {
    const f32x2 v = {a, b};
    if constexpr (KV == KV_F16)
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    else
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// The two fp32 values a packed pair of the 16-bit type holds (exact).
template <int KV> __device__ __forceinline__ f32x2 unpack16(uint32_t w) {
    if constexpr (KV == KV_F16) {
        const f16x2 h = __builtin_bit_cast(f16x2, w);
        return f32x2{(float)h.x, (float)h.y};
    } else {
        return f32x2{__builtin_bit_cast(float, w << 16), __builtin_bit_cast(float, w & 0xFFFF0000u)};
    }
}

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
}

// Narrow VEC fp32 values to one 16-byte chunk of the element type (RNE).
template <int KV, int VEC> __device__ __forceinline__ u32x4 float_to_chunk(const float (&f)[VEC]) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (KV == KV_F32)
            r[i] = __builtin_bit_cast(uint32_t, f[i]);
        else
            r[i] = pack16<KV>(f[2 * i], f[2 * i + 1]);
    }
    return r;
}

template <int KV> __device__ __forceinline__ void store_elem(void *base, size_t idx, float x) {
    if constexpr (KV == KV_F16)
        ((_Float16 *)base)[idx] = (_Float16)x;
    else if constexpr (KV == KV_BF16)
        ((uint16_t *)base)[idx] = (uint16_t)f32_to_bf16_bits(x);
    else
        ((float *)base)[idx] = x;
}

__device__ __forceinline__ u32x4 load16(const char *p) { return *(const u32x4 *)p; }

// K/V pages are read once per launch: nontemporal (`nt`) loads, which stream
// better than the default policy on MI355X.
__device__ __forceinline__ u32x4 stream_load16(const char *p) {
    return __builtin_nontemporal_load((const u32x4 *)p);
}

// Per-wavefront state of one work item.
template <int KV, int D, int GT> struct ItemState {
    static constexpr int VEC = Geometry<KV, D>::kVec;
    u32x4 q[GT];
    float m[GT];     // running max, log2 units
    float l[GT];     // running sum of 2^(s - m)
    float o[GT][VEC];
};

// One tile's K and V registers, loaded and not yet used, and which of its
// kLoadsPerTile row groups hold tokens.
struct TileRegs {
    u32x4 k[kLoadsPerTile], v[kLoadsPerTile];
    bool tv[kLoadsPerTile];
};

// Issue one tile's loads: kLoadsPerTile loads of TPL rows each.  UNI: the TPL
// rows of every load sit in one page (block_size >= TPL), whose id blk[k] was
// read with a scalar load.  MASK: some token of the tile is past t_end or in a
// page with a negative id; such tokens are neither loaded nor counted.
template <int KV, int D, bool UNI, bool MASK>
__device__ __forceinline__ void tile_load(const DecodeParams &p, const int *bt, const char *kb,
                                          const char *vb, int t0, int t_end, int row, int col,
                                          bool col_ok, const int (&blk)[kLoadsPerTile],
                                          TileRegs &r) {
    using Geo = Geometry<KV, D>;
    constexpr int VEC = Geo::kVec;
    constexpr int EB = Geo::kElemBytes;
    constexpr int TPL = Geo::kRows;
    constexpr int LPT = kLoadsPerTile;
    const int bmask = p.block_size - 1;

    long long eoff[LPT];
#pragma unroll
    for (int k = 0; k < LPT; k++) {
        const int tok = t0 + k * TPL + row;
        if constexpr (UNI) {
            const int tk0 = t0 + k * TPL;
            r.tv[k] = !MASK || (tok < t_end && blk[k] >= 0);
            eoff[k] = (long long)blk[k] * p.kv_block_stride +
                      (long long)((((tk0 & bmask) + row) * D) + col * VEC);
        } else {
            const int bi = (tok < t_end ? tok : t_end - 1) >> p.bs_shift;
            const int b = bt[bi];
            r.tv[k] = tok < t_end && b >= 0;
            eoff[k] = (long long)b * p.kv_block_stride + (long long)(((tok & bmask) * D) + col * VEC);
        }
    }
#pragma unroll
    for (int k = 0; k < LPT; k++) {
        if ((!MASK || r.tv[k]) && col_ok)
            r.k[k] = stream_load16(kb + eoff[k] * EB);
        else
            r.k[k] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < LPT; k++) {
        if ((!MASK || r.tv[k]) && col_ok)
            r.v[k] = stream_load16(vb + eoff[k] * EB);
        else
            r.v[k] = u32x4{0, 0, 0, 0};
    }
}

// Fold one loaded tile into the row's state: scores, online softmax, o += P V.
template <int KV, int D, int GT, bool MASK>
__device__ __forceinline__ void tile_compute(const DecodeParams &p, const TileRegs &r,
                                             ItemState<KV, D, GT> &st) {
    using Geo = Geometry<KV, D>;
    constexpr int VEC = Geo::kVec;
    constexpr int RL = Geo::kRowLanes;
    constexpr int LPT = kLoadsPerTile;

    // Scores, log2 units: per-lane partial dots, then one interleaved row
    // reduction over all LPT*GT of them.
    float s[LPT][GT];
    float part[LPT * GT];
#pragma unroll
    for (int k = 0; k < LPT; k++) {
#pragma unroll
        for (int g = 0; g < GT; g++) part[k * GT + g] = chunk_dot<KV>(r.k[k], st.q[g], 0.0f);
    }
    row_sum_n<RL, LPT * GT>(part);
#pragma unroll
    for (int k = 0; k < LPT; k++) {
#pragma unroll
        for (int g = 0; g < GT; g++) {
            const float acc = part[k * GT + g] * p.scale_log2;
            s[k][g] = (MASK && !r.tv[k]) ? -INFINITY : acc;
        }
    }

    // Online softmax update of this row's state.
#pragma unroll
    for (int g = 0; g < GT; g++) {
        float mx = st.m[g];
#pragma unroll
        for (int k = 0; k < LPT; k++) mx = fmaxf(mx, s[k][g]);
        const float ms = (mx == -INFINITY) ? 0.0f : mx;
        const float alpha = fast_exp2(st.m[g] - ms);
        float ps = 0.0f;
#pragma unroll
        for (int k = 0; k < LPT; k++) {
            const float e = fast_exp2(s[k][g] - ms);
            s[k][g] = e;
            ps += e;
        }
        st.l[g] = st.l[g] * alpha + ps;
        st.m[g] = mx;
#pragma unroll
        for (int e = 0; e < VEC; e++) st.o[g][e] *= alpha;
    }

    // o += p * V.
#pragma unroll
    for (int k = 0; k < LPT; k++) {
        float vf[VEC];
        chunk_to_float<KV, VEC>(r.v[k], vf);
#pragma unroll
        for (int g = 0; g < GT; g++) {
#pragma unroll
            for (int e = 0; e < VEC; e++) st.o[g][e] = fmaf(s[k][g], vf[e], st.o[g][e]);
        }
    }
}

// One tile, loaded and folded in.
template <int KV, int D, int GT, bool UNI, bool MASK>
__device__ __forceinline__ void decode_tile(const DecodeParams &p, const int *bt, const char *kb,
                                            const char *vb, int t0, int t_end, int row, int col,
                                            bool col_ok, const int (&blk)[kLoadsPerTile],
                                            ItemState<KV, D, GT> &st) {
    TileRegs r;
    tile_load<KV, D, UNI, MASK>(p, bt, kb, vb, t0, t_end, row, col, col_ok, blk, r);
    tile_compute<KV, D, GT, MASK>(p, r, st);
}

// Block ids of the kLoadsPerTile loads of the tile at t0 (UNI geometry):
// indices are clamped to the last valid token so that a table entry past the
// sequence is never read.
template <int TPL>
__device__ __forceinline__ void tile_blocks(const int *bt, int t0, int t_end, int bs_shift,
                                            int (&blk)[kLoadsPerTile]) {
#pragma unroll
    for (int k = 0; k < kLoadsPerTile; k++) {
        const int tk0 = t0 + k * TPL;
        blk[k] = bt[(tk0 < t_end ? tk0 : t_end - 1) >> bs_shift];
    }
}

template <int KV, int D, int GT, bool UNI>
__device__ __forceinline__ void decode_partition(const DecodeParams &p, const int *bt,
                                                 const char *kb, const char *vb, int t_begin,
                                                 int t_end, int row, int col, bool col_ok,
                                                 ItemState<KV, D, GT> &st) {
    using Geo = Geometry<KV, D>;
    constexpr int TPL = Geo::kRows;
    constexpr int TT = Geo::kTileTokens;
    constexpr int LPT = kLoadsPerTile;
    int blk[LPT], nxt[LPT];
    if constexpr (UNI) tile_blocks<TPL>(bt, t_begin, t_end, p.bs_shift, nxt);
    for (int t0 = t_begin; t0 < t_end; t0 += TT) {
        if constexpr (UNI) {
            // Consume the ids fetched one tile ago, then fetch the next tile's
            // so their latency hides behind this tile.
            bool neg = false;
#pragma unroll
            for (int k = 0; k < LPT; k++) {
                blk[k] = __builtin_amdgcn_readfirstlane(nxt[k]);
                neg |= blk[k] < 0;
            }
            if (t0 + TT < t_end) tile_blocks<TPL>(bt, t0 + TT, t_end, p.bs_shift, nxt);
            if (t0 + TT <= t_end && !neg)
                decode_tile<KV, D, GT, true, false>(p, bt, kb, vb, t0, t_end, row, col, col_ok, blk, st);
            else
                decode_tile<KV, D, GT, true, true>(p, bt, kb, vb, t0, t_end, row, col, col_ok, blk, st);
        } else {
            decode_tile<KV, D, GT, false, true>(p, bt, kb, vb, t0, t_end, row, col, col_ok, blk, st);
        }
    }
}

// Query row of (sequence s, query head h) and output row of the same: from
// the per-sequence row tables when set, else the contiguous batch arrays.
// eb: bytes per element.
__device__ __forceinline__ const char *q_row(const DecodeParams &p, int s, int h, int D, int eb) {
    return p.q_rows ? p.q_rows[s] + (size_t)h * D * eb
                    : (const char *)p.q + ((size_t)s * p.num_heads + h) * D * eb;
}

__device__ __forceinline__ char *o_row(const DecodeParams &p, int s, int h, int D, int eb) {
    return p.o_rows ? p.o_rows[s] + (size_t)h * D * eb
                    : (char *)p.out + ((size_t)s * p.num_heads + h) * D * eb;
}

// Clamped length of sequence s.  Under the new-token fold
// (DecodeParams::nt_fold) the one sequence's cached length comes by value,
// nt_len - 1: no memory round trip.
__device__ __forceinline__ int seq_len_of(const DecodeParams &p, int s) {
    if (p.nt_fold) return p.nt_len - 1;
    const int L = p.seq_lens[s];
    return L < 0 ? 0 : (L > p.max_ctx ? p.max_ctx : L);
}

__device__ __forceinline__ int tiles_per_wave(int total, int num_waves, int min_tpw) {
    const int t = (total + num_waves - 1) / num_waves;
    return t > min_tpw ? t : min_tpw;
}

// Row of the prefix-fold state of (a sequence's fold base, kv head, query
// head g of the group); see DecodeParams::fold_row.
__device__ __forceinline__ size_t fold_state_row(const DecodeParams &p, int base, int kvh, int g) {
    const int q = base + g;
    const int v = q / p.fold_rows;
    return (size_t)v * p.fold_kr + (size_t)kvh * p.fold_rows + (size_t)(q - v * p.fold_rows);
}

// Logical index of workgroup b of a g-workgroup launch such that logical
// neighbours run on one XCD: the dispatcher deals workgroups to MI355X's 8
// XCDs round-robin (b on XCD b % 8), so XCD x's workgroups get one
// contiguous run of logical indices.  Neighbouring stream-K ranges then
// share an L2 (the cascade's prefix batch reads each shared page from two
// sequences of equal length, at the same offsets of neighbouring ranges).
__device__ __forceinline__ int xcd_local_block(int b, int g) {
    constexpr int kXcds = 8;
    const int q = g / kXcds, r = g % kXcds;
    const int x = b % kXcds, i = b / kXcds;
    return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

// Logical workgroup of this workgroup for a launch of `total` split units:
// XCD-local when the batch fills the launch (more than min_tiles_per_wave
// units per wavefront, so ranges reach the last wavefronts); otherwise
// (ranges on the lowest logical wavefronts only) the dispatch order, which
// spreads the busy ones over all XCDs.
__device__ __forceinline__ int logical_block(const DecodeParams &p, int total) {
    return (long long)total > (long long)p.num_waves * p.min_tiles_per_wave
               ? xcd_local_block(blockIdx.x, gridDim.x)
               : (int)blockIdx.x;
}

// Stream-K segments of one sequence: one per (kv head, head tile), or per kv
// head when the head tiles are paired (DecodeParams::pair_tiles).
__device__ __forceinline__ int seq_segments(const DecodeParams &p) {
    return p.num_kv_heads * (p.pair_tiles ? 1 : p.head_tiles);
}

// Split units of a segment of Ts tiles (paged_decode_params.h): its tiles
// plus the start-up cost; an empty segment costs nothing.
__device__ __forceinline__ int segment_units(const DecodeParams &p, int Ts) {
    return Ts > 0 ? Ts + p.seg_cost : 0;
}

// Exclusive prefix over sequences of the split units of all their segments,
// into LDS (num_seqs + 1 entries), by the whole workgroup.  Workgroup 0 also
// stores it for the merge kernel.
template <int TT, int WPG>
__device__ __forceinline__ void batch_prefix(const DecodeParams &p, int *pre) {
    __shared__ int part[WPG];
    const int nthr = 64 * WPG;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int B = p.num_seqs;
    const int per = (B + nthr - 1) / nthr;
    const int s0 = tid * per;
    const int segs = seq_segments(p);
    int local = 0;
    for (int i = 0; i < per; i++) {
        const int s = s0 + i;
        if (s < B) {
            const int t = segment_units(p, (seq_len_of(p, s) + TT - 1) / TT) * segs;
            pre[s] = t;  // units of sequence s, scanned below
            local += t;
        }
    }
    // Inclusive scan of the per-thread sums: within each wavefront with
    // shuffles, then the wavefronts' totals through LDS (one barrier; a
    // 256-thread Hillis-Steele scan took 16 and made the prologue longer).
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    if (lane == 63) part[wave] = incl;
    __syncthreads();
    int base = 0;
#pragma unroll
    for (int k = 0; k < WPG - 1; k++) base += k < wave ? part[k] : 0;
    int run = base + incl - local;  // exclusive prefix of this thread's first sequence
    for (int i = 0; i < per; i++) {
        const int s = s0 + i;
        if (s < B) {
            const int t = pre[s];
            pre[s] = run;
            run += t;
        }
    }
    if (tid == nthr - 1) pre[B] = base + incl;
    __syncthreads();
    if (blockIdx.x == 0) {
        for (int s = tid; s <= B; s += nthr) p.ws_prefix[s] = pre[s];
    }
}

// Walk this wavefront's stream-K range: for every segment piece in it call
// fn(s, L, kvh, ht, t_begin, t_end, whole, slot) where [t_begin, t_end) are
// the piece's tokens, `whole` says the piece is the entire segment (write the
// output) and `slot` is the partial slot otherwise.  `pre` is the LDS unit
// prefix (num_seqs + 1 ints); every thread of the workgroup (WPG wavefronts)
// must call this.  A range that ends inside a segment's start-up units holds
// none of its tiles and makes no piece of it.
template <int TT, int WPG, typename Fn>
__device__ __forceinline__ void stream_k_walk(const DecodeParams &p, int *pre, Fn &&fn) {
    batch_prefix<TT, WPG>(p, pre);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int B = p.num_seqs;
    const int total = pre[B];
    const int w = logical_block(p, total) * WPG + wave;
    const int tpw = tiles_per_wave(total, p.num_waves, p.min_tiles_per_wave);
    const long long g_lo = (long long)w * tpw;
    if (g_lo >= total) return;
    int g = (int)g_lo;
    const int g_end = min(total, g + tpw);

    // Sequence holding unit g: the last s with pre[s] <= g (empty sequences
    // share their successor's prefix, so this lands on one with tiles).
    int lo = 0, hi = B - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pre[mid] <= g) lo = mid; else hi = mid - 1;
    }
    int s = __builtin_amdgcn_readfirstlane(lo);
    const int segs = p.num_kv_heads * p.head_tiles;
    bool first = true;
    while (g < g_end) {
        const int L = seq_len_of(p, s);
        const int Ts = (L + TT - 1) / TT;  // tiles per segment of sequence s
        const int Cs = segment_units(p, Ts);
        const int local = g - pre[s];
        const int seg = local / Cs;
        const int u0 = local - seg * Cs;
        const int u1 = min(Cs, u0 + (g_end - g));
        const int t0 = max(u0 - p.seg_cost, 0), t1 = max(u1 - p.seg_cost, 0);
        if (t1 > t0) {
            const int kvh = seg / p.head_tiles;
            const int ht = seg - kvh * p.head_tiles;
            fn(s, L, kvh, ht, t0 * TT, min(L, t1 * TT), t0 == 0 && t1 == Ts,
               (size_t)w * 2 + (first ? 0 : 1));
            first = false;
        }
        g += u1 - u0;
        if (g - pre[s] >= Cs * segs) {  // sequence done: next one with tiles
            s++;
            while (s < B - 1 && pre[s + 1] == pre[s]) s++;
        }
    }
}

// Partition kernel, VALU tile path: kWavesPerGroup wavefronts per workgroup,
// each owning one stream-K range of tiles (see paged_decode_params.h).
template <int KV, int D, int GT>
__global__ __launch_bounds__(64 * kWavesPerGroup) void paged_decode_partition_kernel(
    const DecodeParams p) {
    using Geo = Geometry<KV, D>;
    constexpr int VEC = Geo::kVec;
    constexpr int EB = Geo::kElemBytes;
    constexpr int NCH = Geo::kChunks;
    constexpr int RL = Geo::kRowLanes;
    constexpr int TT = Geo::kTileTokens;
    extern __shared__ int pre[];  // num_seqs + 1 split-unit prefixes

    const int lane = threadIdx.x & 63;
    const int col = lane % RL;
    const int row = lane / RL;
    const bool col_ok = (NCH == RL) || (col < NCH);

    stream_k_walk<TT, kWavesPerGroup>(p, pre, [&](int s, int L, int kvh, int ht, int t_begin, int t_end,
                                  bool whole, size_t slot) {
        (void)L;
        const int g0 = ht * GT;
        const int nh = min(GT, p.group - g0);
        const size_t qrow0 = ((size_t)s * p.num_heads + (size_t)kvh * p.group + g0) * D;

        ItemState<KV, D, GT> st;
#pragma unroll
        for (int h = 0; h < GT; h++) {
            st.q[h] = (h < nh && col_ok)
                          ? load16(q_row(p, s, kvh * p.group + g0 + h, D, EB) + col * VEC * EB)
                          : u32x4{0, 0, 0, 0};
            st.m[h] = -INFINITY;
            st.l[h] = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; e++) st.o[h][e] = 0.0f;
        }
        if (p.fold_row && t_begin == 0 && row == 0) {  // row 0 lanes carry the prefix state
            const int base = p.fold_row[s];
            if (base >= 0) {
#pragma unroll
                for (int h = 0; h < GT; h++) {
                    if (h >= nh) continue;
                    const size_t r = fold_state_row(p, base, kvh, g0 + h);
                    st.m[h] = p.fold_lse[r];
                    st.l[h] = 1.0f;
                    if (col_ok) {
#pragma unroll
                        for (int e = 0; e < VEC; e++) st.o[h][e] = p.fold_out[r * D + col * VEC + e];
                    }
                }
            }
        }
        const int *bt = p.block_tables + (size_t)s * p.max_blocks;
        const char *kb = (const char *)p.k + (size_t)kvh * (size_t)p.kv_head_stride * EB;
        const char *vb = (const char *)p.v + (size_t)kvh * (size_t)p.kv_head_stride * EB;
        if (p.block_size >= Geo::kRows)
            decode_partition<KV, D, GT, true>(p, bt, kb, vb, t_begin, t_end, row, col, col_ok, st);
        else
            decode_partition<KV, D, GT, false>(p, bt, kb, vb, t_begin, t_end, row, col, col_ok, st);

        // Merge the row states (rows differ in lane bits >= log2 RL).
#pragma unroll
        for (int off = RL; off < 64; off <<= 1) {
#pragma unroll
            for (int h = 0; h < GT; h++) {
                const float mo = __shfl_xor(st.m[h], off);
                const float lo2 = __shfl_xor(st.l[h], off);
                const float M = fmaxf(st.m[h], mo);
                const float Ms = (M == -INFINITY) ? 0.0f : M;
                const float a = fast_exp2(st.m[h] - Ms);
                const float b = fast_exp2(mo - Ms);
                st.l[h] = st.l[h] * a + lo2 * b;
                st.m[h] = M;
#pragma unroll
                for (int e = 0; e < VEC; e++)
                    st.o[h][e] = st.o[h][e] * a + __shfl_xor(st.o[h][e], off) * b;
            }
        }

        if (row != 0 || !col_ok) return;
        if (whole && p.out_f32) {
#pragma unroll
            for (int h = 0; h < GT; h++) {
                if (h >= nh) continue;
                const float inv = st.l[h] > 0.0f ? 1.0f / st.l[h] : 0.0f;
                float *dst = p.out_f32 + qrow0 + (size_t)h * D + col * VEC;
#pragma unroll
                for (int e = 0; e < VEC; e += 4)
                    *(f32x4 *)(dst + e) = f32x4{st.o[h][e], st.o[h][e + 1], st.o[h][e + 2],
                                                st.o[h][e + 3]} * inv;
                if (col == 0)
                    p.out_lse[qrow0 / D + h] =
                        st.l[h] > 0.0f ? st.m[h] + log2f(st.l[h]) : -INFINITY;
            }
        } else if (whole) {
#pragma unroll
            for (int h = 0; h < GT; h++) {
                if (h >= nh) continue;
                const float inv = st.l[h] > 0.0f ? 1.0f / st.l[h] : 0.0f;
                float f[VEC];
#pragma unroll
                for (int e = 0; e < VEC; e++) f[e] = st.o[h][e] * inv;
                *(u32x4 *)(o_row(p, s, kvh * p.group + g0 + h, D, EB) + col * VEC * EB) =
                    float_to_chunk<KV, VEC>(f);
            }
        } else {
#pragma unroll
            for (int h = 0; h < GT; h++) {
                if (h >= nh) continue;
                float *dst = p.ws_o + (slot * GT + h) * D + col * VEC;
#pragma unroll
                for (int e = 0; e < VEC; e += 4)
                    *(f32x4 *)(dst + e) =
                        f32x4{st.o[h][e], st.o[h][e + 1], st.o[h][e + 2], st.o[h][e + 3]};
                if (col == 0) {
                    p.ws_ml[(slot * GT + h) * 2] = st.m[h];
                    p.ws_ml[(slot * GT + h) * 2 + 1] = st.l[h];
                }
            }
        }
    });
}

// Small batches on the VALU tile path (DecodeParams::segment_launch): S =
// DecodeParams::segment_split workgroups of kSegWaves wavefronts per segment
// (sequence, kv head, head tile), one round of workgroups for the batch.
// Workgroup j of a segment takes its tiles j, j + S, ...; of those, wavefront
// w takes the w-th, (w + kSegWaves)-th, ..., kSegTiles of them in flight at a
// time.  The sequence length, the query rows and the first tiles' block ids
// are requested together, the block ids without waiting for the length
// (entries past the sequence are read, within the table row, but their
// tokens are masked).  The wavefronts' states are combined through LDS; with
// S = 1 the workgroup writes the output rows (no merge launch), else its
// fp32 partial for paged_decode_segment_merge_kernel.
template <int KV, int D, int GT>
__global__ __launch_bounds__(64 * kSegWaves) void paged_decode_segment_kernel(
    const DecodeParams p) {
    using Geo = Geometry<KV, D>;
    constexpr int VEC = Geo::kVec;
    constexpr int EB = Geo::kElemBytes;
    constexpr int NCH = Geo::kChunks;
    constexpr int RL = Geo::kRowLanes;
    constexpr int TT = Geo::kTileTokens;
    constexpr int TPL = Geo::kRows;
    constexpr int LPT = kLoadsPerTile;
    __shared__ float s_o[kSegWaves][GT][D];
    __shared__ float s_m[kSegWaves][GT], s_l[kSegWaves][GT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane % RL;
    const int row = lane / RL;
    const bool col_ok = (NCH == RL) || (col < NCH);
    XHIP_WG_BEGIN(p);
    const int segs = p.num_kv_heads * p.head_tiles;
    const int S = p.segment_split;
    const int gseg = blockIdx.x / S;         // segment of the batch
    const int part = blockIdx.x - gseg * S;  // this workgroup's share of its tiles
    const int s = gseg / segs;
    const int seg = gseg - s * segs;
    const int kvh = seg / p.head_tiles;
    const int ht = seg - kvh * p.head_tiles;
    const int g0 = ht * GT;
    const int nh = min(GT, p.group - g0);
    const int *bt = p.block_tables + (size_t)s * p.max_blocks;
    const char *kb = (const char *)p.k + (size_t)kvh * (size_t)p.kv_head_stride * EB;
    const char *vb = (const char *)p.v + (size_t)kvh * (size_t)p.kv_head_stride * EB;

    const int L = seq_len_of(p, s);
    ItemState<KV, D, GT> st;
#pragma unroll
    for (int h = 0; h < GT; h++) {
        st.q[h] = (h < nh && col_ok)
                      ? load16(q_row(p, s, kvh * p.group + g0 + h, D, EB) + col * VEC * EB)
                      : u32x4{0, 0, 0, 0};
        st.m[h] = -INFINITY;
        st.l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; e++) st.o[h][e] = 0.0f;
    }
    // The workgroup's tiles are u * S + part for u = 0, 1, ...: wavefront w
    // takes u = w + kSegWaves * j in round 0, and kSegWaves * kSegTiles more
    // in each later round.
    int nxt[kSegTiles][LPT];
#pragma unroll
    for (int j = 0; j < kSegTiles; j++)
        tile_blocks<TPL>(bt, ((wave + kSegWaves * j) * S + part) * TT, p.max_ctx, p.bs_shift,
                         nxt[j]);
    const int Ts = (L + TT - 1) / TT;
    for (int r = 0; r < kSegRounds; r++) {
        const int ub = wave + kSegWaves * kSegTiles * r;  // this wavefront's first tile of the round
        if (ub * S + part >= Ts) break;
        if (r == 0 && wave == 0) XHIP_WG_STAMP(p, 7);
        TileRegs regs[kSegTiles];
#pragma unroll
        for (int j = 0; j < kSegTiles; j++) {
            int blk[LPT];
#pragma unroll
            for (int k = 0; k < LPT; k++) blk[k] = __builtin_amdgcn_readfirstlane(nxt[j][k]);
            tile_load<KV, D, true, true>(p, bt, kb, vb, ((ub + kSegWaves * j) * S + part) * TT, L,
                                         row, col, col_ok, blk, regs[j]);
        }
        if (r + 1 < kSegRounds) {
#pragma unroll
            for (int j = 0; j < kSegTiles; j++)
                tile_blocks<TPL>(bt, ((ub + kSegWaves * (kSegTiles + j)) * S + part) * TT,
                                 p.max_ctx, p.bs_shift, nxt[j]);
        }
#pragma unroll
        for (int j = 0; j < kSegTiles; j++) tile_compute<KV, D, GT, true>(p, regs[j], st);
    }

    if (wave == 0) XHIP_WG_STAMP(p, 8);
    // This wavefront's state: its rows merged (lane bits >= log2 RL), then
    // through LDS to the workgroup's combine.
#pragma unroll
    for (int off = RL; off < 64; off <<= 1) {
#pragma unroll
        for (int h = 0; h < GT; h++) {
            const float mo = __shfl_xor(st.m[h], off);
            const float lo2 = __shfl_xor(st.l[h], off);
            const float M = fmaxf(st.m[h], mo);
            const float Ms = (M == -INFINITY) ? 0.0f : M;
            const float a = fast_exp2(st.m[h] - Ms);
            const float b = fast_exp2(mo - Ms);
            st.l[h] = st.l[h] * a + lo2 * b;
            st.m[h] = M;
#pragma unroll
            for (int e = 0; e < VEC; e++)
                st.o[h][e] = st.o[h][e] * a + __shfl_xor(st.o[h][e], off) * b;
        }
    }
    if (row == 0 && col_ok) {
#pragma unroll
        for (int h = 0; h < GT; h++) {
#pragma unroll
            for (int e = 0; e < VEC; e++) s_o[wave][h][col * VEC + e] = st.o[h][e];
            if (col == 0) {
                s_m[wave][h] = st.m[h];
                s_l[wave][h] = st.l[h];
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nh * D; i += 64 * kSegWaves) {
        const int h = i / D, d = i - h * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kSegWaves; w++) M = fmaxf(M, s_m[w][h]);
        const float Ms = (M == -INFINITY) ? 0.0f : M;
        float l = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < kSegWaves; w++) {
            const float a = fast_exp2(s_m[w][h] - Ms);
            l += s_l[w][h] * a;
            o += s_o[w][h][d] * a;
        }
        if (S > 1) {
            // this workgroup's fp32 partial (m, l, o), combined by
            // paged_decode_segment_merge_kernel
            const size_t slot = (size_t)blockIdx.x * GT + h;
            p.ws_o[slot * D + d] = o;
            if (d == 0) {
                p.ws_ml[slot * 2] = M;
                p.ws_ml[slot * 2 + 1] = l;
            }
            continue;
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        store_elem<KV>(o_row(p, s, kvh * p.group + g0 + h, D, EB), d, o * inv);
    }
    XHIP_WG_FLUSH(p);
}

// The rows of the segments paged_decode_segment_kernel split over S =
// DecodeParams::segment_split workgroups: one workgroup per segment
// combines their fp32 partials (slots segment * S + j) by the online
// log-sum-exp rule and writes the output rows.
template <int KV, int D, int GT>
__global__ __launch_bounds__(256) void paged_decode_segment_merge_kernel(const DecodeParams p) {
    XHIP_MERGE_SCOPE(p);
    constexpr int EB = Geometry<KV, D>::kElemBytes;
    const int segs = p.num_kv_heads * p.head_tiles;
    const int S = p.segment_split;
    const int s = blockIdx.x / segs;
    const int seg = blockIdx.x - s * segs;
    const int kvh = seg / p.head_tiles;
    const int g0 = (seg - kvh * p.head_tiles) * GT;
    const int nh = min(GT, p.group - g0);
    for (int i = threadIdx.x; i < nh * D; i += 256) {
        const int h = i / D, d = i - h * D;
        float m = -INFINITY, l = 0.0f, o = 0.0f;
        for (int j = 0; j < S; j++) {
            const size_t slot = ((size_t)blockIdx.x * S + j) * GT + h;
            const float mj = p.ws_ml[slot * 2];
            const float M = fmaxf(m, mj);
            const float Ms = (M == -INFINITY) ? 0.0f : M;
            const float a = fast_exp2(m - Ms), w = fast_exp2(mj - Ms);
            l = l * a + p.ws_ml[slot * 2 + 1] * w;
            o = o * a + p.ws_o[slot * D + d] * w;
            m = M;
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        store_elem<KV>(o_row(p, s, kvh * p.group + g0 + h, D, EB), d, o * inv);
    }
}

// The slots of a cut segment's partials: partial 0 in slot s0, partial
// j >= 1 in slot sb + sstride * j.
struct PartialSlots {
    size_t s0, sb;
    int sstride, np;
};

// The partials of the segment whose first tile is split unit first_tile
// (Ts tiles, starting at unit seg_start) under a plan of tpw units per
// wavefront; false when the partition kernel finished it (it lay in one
// wavefront's range, or in one workgroup's under wg_fix).
template <int WPG>
__device__ __forceinline__ bool segment_partials(const DecodeParams &p, int seg_start,
                                                 int first_tile, int Ts, int tpw,
                                                 PartialSlots &ps) {
    const int w_first = first_tile / tpw;
    const int w_last = (first_tile + Ts - 1) / tpw;
    // the segment is w_first's first piece when w_first's range begins in the
    // segment's start-up units or at its first tile
    const int slot0 = (w_first * tpw >= seg_start) ? 0 : 1;
    ps.s0 = (size_t)w_first * 2 + slot0;
    if (p.wg_fix) {
        const int wg0 = w_first / WPG, wg1 = w_last / WPG;
        if (wg0 == wg1) return false;
        ps.np = wg1 - wg0 + 1;
        ps.sb = (size_t)wg0 * 2 * WPG;
        ps.sstride = 2 * WPG;
    } else {
        if (w_first == w_last) return false;
        ps.np = w_last - w_first + 1;
        ps.sb = (size_t)w_first * 2;
        ps.sstride = 2;
    }
    return true;
}

// segment_partials for a batch with paired head tiles (pair_tiles, no
// wg_fix): the partials of head tile ht of the segment, under a plan of tpw
// units per range (a range is two wavefronts).
__device__ __forceinline__ bool segment_partials_paired(int seg_start, int first_tile, int Ts,
                                                        int tpw, int ht, PartialSlots &ps) {
    const int r_first = first_tile / tpw;
    const int r_last = (first_tile + Ts - 1) / tpw;
    if (r_first == r_last) return false;
    const int slot0 = (r_first * tpw >= seg_start) ? 0 : 1;
    ps.np = r_last - r_first + 1;
    ps.sb = (size_t)(2 * r_first + ht) * 2;
    ps.s0 = ps.sb + slot0;
    ps.sstride = 4;
    return true;
}

// Four fp16 values as fp32.
__device__ __forceinline__ f32x4 unpack_h4(u32x2 h) {
    const f32x2 a = unpack16<KV_F16>(h.x), b = unpack16<KV_F16>(h.y);
    return f32x4{a.x, a.y, b.x, b.y};
}

// Four consecutive values of a partial's o at float index `at` of the
// split-K workspace: fp32, or HS: fp16 states (DecodeParams::ws_h).
template <bool HS>
__device__ __forceinline__ f32x4 partial_f32x4(const DecodeParams &p, size_t at) {
    if constexpr (HS) return unpack_h4(*(const u32x2 *)((const char *)p.ws_h + at * 2));
    else return *(const f32x4 *)(p.ws_o + at);
}

// Online log-sum-exp merge, into (m, l, acc) of one float4 column, of a
// segment's partials j = j0, j0 + step, ... < np (slots as in PartialSlots).
// The partials go in batches of up to NB whose loads are all issued before
// any is used, so a thread waits for one memory round trip per batch, not
// per partial; batch slots past np load and combine nothing.  The column's
// (m, l) and float4 of o sit at off_ml and off_o floats into a slot.  HS:
// fp16 states (DecodeParams::ws_h), whose o is read at the same index.
template <int GT, int D, int NB, bool HS = false>
__device__ __forceinline__ void merge_partials(const DecodeParams &p, const PartialSlots &ps,
                                               int j0, int step, int off_ml, int off_o,
                                               float &m, float &l, f32x4 &acc) {
    const int np = ps.np;
    for (int jb = j0; jb < np; jb += NB * step) {
        f32x2 mlv[NB];
        f32x4 ov[NB];
        u32x2 hv[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int j = jb + b * step;
            mlv[b] = f32x2{-INFINITY, 0.0f};  // (defined values for the slots left unread)
            ov[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            hv[b] = u32x2{0u, 0u};
            if (j < np) {
                const size_t slot = j == 0 ? ps.s0 : ps.sb + (size_t)ps.sstride * j;
                mlv[b] = *(const f32x2 *)(p.ws_ml + slot * GT * 2 + off_ml);
                if constexpr (HS)
                    hv[b] = *(const u32x2 *)((const char *)p.ws_h + (slot * GT * D + off_o) * 2);
                else
                    ov[b] = *(const f32x4 *)(p.ws_o + slot * GT * D + off_o);
            }
        }
        // keep the scheduler from starting the combine (and waiting on the
        // first loads) before the whole batch is issued
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (jb + b * step >= np) break;
            if constexpr (HS) ov[b] = unpack_h4(hv[b]);
            const float mj = mlv[b].x;
            const float M = fmaxf(m, mj);
            const float Ms = (M == -INFINITY) ? 0.0f : M;
            const float a = fast_exp2(m - Ms), w = fast_exp2(mj - Ms);
            l = l * a + mlv[b].y * w;
            acc = acc * a + ov[b] * w;
            m = M;
        }
    }
}

// Output float4 column `col` (head col / (D/4), head-major) of an empty
// sequence s: zeros (log-sum-exp -inf), or the prefix row under a prefix
// fold (the sequence's whole context was the shared prefix).
template <int KV, int D>
__device__ __forceinline__ void write_empty_column(const DecodeParams &p, int s, int kvh, int g0,
                                                   size_t qrow0, int col) {
    constexpr int C4 = D / 4;
    const size_t base = qrow0 + (size_t)col * 4;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    float lse = -INFINITY;
    const int fb = p.fold_row ? p.fold_row[s] : -1;
    if (fb >= 0) {
        const size_t r = fold_state_row(p, fb, kvh, g0 + col / C4);
        o = *(const f32x4 *)(p.fold_out + r * D + (col % C4) * 4);
        lse = p.fold_lse[r];
    }
    if (p.out_f32) {
        *(f32x4 *)(p.out_f32 + base) = o;
        if (col % C4 == 0) p.out_lse[qrow0 / D + col / C4] = lse;
    } else {
        char *orow = o_row(p, s, kvh * p.group + g0 + col / C4, D, KV == KV_F32 ? 4 : 2);
#pragma unroll
        for (int e = 0; e < 4; e++) store_elem<KV>(orow, (col % C4) * 4 + e, o[e]);
    }
}

// Four consecutive elements of a row (element type), as fp32.
template <int KV>
__device__ __forceinline__ f32x4 load4_elem(const char *row, int i) {
    if constexpr (KV == KV_F32) {
        return *(const f32x4 *)(row + (size_t)i * 4);
    } else {
        const u32x2 w = *(const u32x2 *)(row + (size_t)i * 2);
        const f32x2 a = unpack16<KV>(w.x), b = unpack16<KV>(w.y);
        return f32x4{a.x, a.y, b.x, b.y};
    }
}

// The new token's inputs of output float4 column c (dims 4c..4c+3) of query
// head `head` (kv head kvh) of sequence s: the query's four values and the
// token's K and V (DecodeParams::nt_fold).  Loaded when the merge starts, so
// that their round trip overlaps the partials'.
struct FoldIn {
    f32x4 q, k, v;
};

template <int KV, int D>
__device__ __forceinline__ FoldIn fold_load(const DecodeParams &p, int s, int kvh, int head, int c) {
    constexpr int EB = KV == KV_F32 ? 4 : 2;
    FoldIn f;
    f.q = load4_elem<KV>(q_row(p, s, head, D, EB), 4 * c);
    f.k = load4_elem<KV>((const char *)p.nt_k + (size_t)kvh * D * EB, 4 * c);
    f.v = load4_elem<KV>((const char *)p.nt_v + (size_t)kvh * D * EB, 4 * c);
    return f;
}

// New-token fold of one output column whose state over the cached tokens is
// (m, l, acc) (log2 units; acc = l * the row): the new token's score, q .
// k_new over the head's C4 = D/4 columns held by an aligned group of C4
// consecutive lanes (xor butterfly), then the online log-sum-exp update with
// v_new.  Returns the finished column.
template <int D>
__device__ __forceinline__ f32x4 fold_new_token(const DecodeParams &p, const FoldIn &f, float m,
                                                float l, f32x4 acc) {
    constexpr int C4 = D / 4;
    static_assert((C4 & (C4 - 1)) == 0 && C4 <= 32, "a head's columns in one aligned lane group");
    float dot = f.q.x * f.k.x + f.q.y * f.k.y + f.q.z * f.k.z + f.q.w * f.k.w;
#pragma unroll
    for (int off = 1; off < C4; off <<= 1) dot += __shfl_xor(dot, off);
    const float sc = dot * p.scale_log2;
    const float M = fmaxf(m, sc);
    const float a = fast_exp2(m - M), b = fast_exp2(sc - M);
    return (acc * a + f.v * b) * (1.0f / (l * a + b));
}

// New-token fold: the token's K/V rows of kv head kvh into its cache slot
// (16-byte chunks, threads of one workgroup), and, by one thread of the
// launch, the sequence's new page id and length.
template <int D, int EB>
__device__ __forceinline__ void store_new_token(const DecodeParams &p, int kvh, bool lead) {
    constexpr int kChunks = D * EB / 16;
    const int page = p.nt_slot >> p.bs_shift;
    const int off = p.nt_slot & (p.block_size - 1);
    const size_t at = ((size_t)page * p.kv_block_stride + (size_t)kvh * p.kv_head_stride +
                       (size_t)off * D) * EB;
    const size_t src = (size_t)kvh * D * EB;
    for (int i = threadIdx.x; i < 2 * kChunks; i += blockDim.x) {
        const bool is_v = i >= kChunks;
        const int ch = is_v ? i - kChunks : i;
        const char *from = (const char *)(is_v ? p.nt_v : p.nt_k) + src + (size_t)ch * 16;
        char *to = (char *)(is_v ? p.v : p.k) + at + (size_t)ch * 16;
        *(u32x4 *)to = *(const u32x4 *)from;
    }
    if (lead && threadIdx.x == 0) {
        if (p.nt_table) *p.nt_table = p.nt_page;
        *p.nt_lens = p.nt_len;
    }
}

// Merge kernel: one workgroup per (segment, chunk of kMergeCols output
// float4 columns), where a segment is (sequence, kv head, head tile) and the
// columns run over (head h < nh, dims 4c..4c+3).  It writes zeros for an
// empty sequence, does nothing for a segment finished inside one wavefront
// range, and otherwise combines the partials of every wavefront that touched
// the segment in one pass: each of the kMergeSplit threads of a column runs
// an online log-sum-exp merge over every kMergeSplit-th partial (running max,
// rescaled denominator and float4 numerator), and the splits are combined in
// LDS the same way.  TT is the tile length (tokens) of the partition kernel
// that produced the partials: the range arithmetic must match it exactly.
constexpr int kMergeSplit = 8;

template <int KV, int D, int GT, int TT>
__global__ __launch_bounds__(kMergeCols * kMergeSplit) void paged_decode_merge_kernel(
    const DecodeParams p) {
    XHIP_MERGE_SCOPE(p);
    constexpr int C4 = D / 4;
    __shared__ f32x4 s_acc[kMergeSplit][kMergeCols];
    __shared__ float s_m[kMergeSplit][kMergeCols];
    __shared__ float s_l[kMergeSplit][kMergeCols];
    const int segs = p.num_kv_heads * p.head_tiles;
    const int s = blockIdx.x / segs;
    const int seg = blockIdx.x - s * segs;
    const int kvh = seg / p.head_tiles;
    const int ht = seg - kvh * p.head_tiles;
    const int g0 = ht * GT;
    const int nh = min(GT, p.group - g0);
    const int ncols = nh * C4;
    const int col0 = blockIdx.y * kMergeCols;
    constexpr int EB = KV == KV_F32 ? 4 : 2;
    // the new-token fold needs a head's columns in one aligned lane group
    constexpr bool kFold = (C4 & (C4 - 1)) == 0 && C4 <= 32;
    if (kFold && p.nt_fold && blockIdx.y == 0 && ht == 0)
        store_new_token<D, EB>(p, kvh, blockIdx.x == 0);
    if (col0 >= ncols) return;
    const int tid = threadIdx.x;
    // the new-token fold's threads: the first kMergeCols, one per column
    FoldIn fi;
    if constexpr (kFold) {
        if (p.nt_fold && tid < kMergeCols && col0 + tid < ncols) {
            const int h = (col0 + tid) / C4;
            fi = fold_load<KV, D>(p, s, kvh, kvh * p.group + g0 + h, col0 + tid - h * C4);
        }
    }
    // the three scalars the merge needs, requested together (the empty asm
    // keeps the compiler from sinking the prefix loads past the L == 0 exit,
    // which would cost a second round trip).  Under the new-token fold (one
    // sequence, its cached length by value) they need no load at all.
    const int L = seq_len_of(p, s);
    int total, pre_s;
    if (kFold && p.nt_fold) {
        total = segs * segment_units(p, (L + TT - 1) / TT);
        pre_s = 0;
    } else {
        total = p.ws_prefix[p.num_seqs];
        pre_s = p.ws_prefix[s];
    }
    asm volatile("" ::"s"(total), "s"(pre_s));
    const size_t qrow0 = ((size_t)s * p.num_heads + (size_t)kvh * p.group + g0) * D;

    if (L == 0) {
        if constexpr (kFold) {
            if (p.nt_fold) {  // no cached token: the output is the new token's V
                const int col = col0 + tid;
                if (tid < kMergeCols && col < ncols) {
                    const int h = col / C4, c = col - h * C4;
                    const f32x4 o = fold_new_token<D>(p, fi, -INFINITY, 0.0f,
                                                      f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                    char *orow = o_row(p, s, kvh * p.group + g0 + h, D, EB);
#pragma unroll
                    for (int e = 0; e < 4; e++) store_elem<KV>(orow, c * 4 + e, o[e]);
                }
                return;
            }
        }
        if (tid < kMergeCols && col0 + tid < ncols && !p.skip_empty)
            write_empty_column<KV, D>(p, s, kvh, g0, qrow0, col0 + tid);
        return;
    }
    const int tpw = tiles_per_wave(total, p.num_waves, p.min_tiles_per_wave);
    const int Ts = (L + TT - 1) / TT;
    const int seg_start = pre_s + seg * segment_units(p, Ts);  // in split units
    PartialSlots ps;
    if (!segment_partials<kMfmaWavesPerGroup>(p, seg_start, seg_start + p.seg_cost, Ts, tpw, ps)) {
        if constexpr (kFold) {
            if (p.nt_fold) {
                // a segment the partition kernel finished: its row and
                // log-sum-exp (partial-output mode), folded with the new token
                const int col = col0 + tid;
                if (tid < kMergeCols && col < ncols) {
                    const int h = col / C4, c = col - h * C4;
                    const float lse = p.out_lse[qrow0 / D + h];
                    const f32x4 row = *(const f32x4 *)(p.out_f32 + qrow0 + (size_t)h * D + c * 4);
                    const f32x4 o =
                        fold_new_token<D>(p, fi, lse, lse == -INFINITY ? 0.0f : 1.0f, row);
                    char *orow = o_row(p, s, kvh * p.group + g0 + h, D, EB);
#pragma unroll
                    for (int e = 0; e < 4; e++) store_elem<KV>(orow, c * 4 + e, o[e]);
                }
            }
        }
        return;
    }

    const int cl = tid % kMergeCols;
    const int psplit = tid / kMergeCols;
    const int col = col0 + cl;
    const bool active = col < ncols;
    const int h = active ? col / C4 : 0;
    const int c = active ? col - h * C4 : 0;
    float m = -INFINITY, l = 0.0f;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (active) merge_partials<GT, D, 8>(p, ps, psplit, kMergeSplit, h * 2, h * D + c * 4, m, l, acc);
    s_acc[psplit][cl] = acc;
    s_m[psplit][cl] = m;
    s_l[psplit][cl] = l;
    __syncthreads();
    if (psplit != 0 || !active) return;
    float mm = m, ll = l;
    f32x4 aa = acc;
#pragma unroll
    for (int k = 1; k < kMergeSplit; k++) {
        const float mk = s_m[k][cl];
        const float M = fmaxf(mm, mk);
        const float Ms = (M == -INFINITY) ? 0.0f : M;
        const float a = fast_exp2(mm - Ms), b = fast_exp2(mk - Ms);
        ll = ll * a + s_l[k][cl] * b;
        aa = aa * a + s_acc[k][cl] * b;
        mm = M;
    }
    if constexpr (kFold) {
        if (p.nt_fold) {
            const f32x4 o = fold_new_token<D>(p, fi, mm, ll, aa);
            char *orow = o_row(p, s, kvh * p.group + g0 + h, D, EB);
#pragma unroll
            for (int e = 0; e < 4; e++) store_elem<KV>(orow, c * 4 + e, o[e]);
            return;
        }
    }
    const float inv = ll > 0.0f ? 1.0f / ll : 0.0f;
    const size_t base = qrow0 + (size_t)h * D + c * 4;
    if (p.out_f32) {
        *(f32x4 *)(p.out_f32 + base) = aa * inv;
        if (c == 0) p.out_lse[qrow0 / D + h] = ll > 0.0f ? mm + log2f(ll) : -INFINITY;
        return;
    }
    char *orow = o_row(p, s, kvh * p.group + g0 + h, D, EB);
#pragma unroll
    for (int e = 0; e < 4; e++) store_elem<KV>(orow, c * 4 + e, aa[e] * inv);
}


// Merge kernel, one workgroup per segment: for batches with enough segments
// to fill the GPU (where the (segment, chunk) grid above would launch several
// thousand short workgroups, each costing ~2 ns of dispatch).  NT threads
// (64 to 1024, chosen at launch as the first head tile's float4 columns
// rounded up to a power of two, at least 64) cover the columns, one each;
// where a segment has at most NT / 2 columns (fewer than 64, or the partly
// filled last head tile of a group), the S = NT / pow2(ncols) threads of a
// column split its partials (every S-th one) and combine in LDS.  Each thread runs
// the online log-sum-exp merge over its partials with a batch of their loads
// in flight at a time.
constexpr int kMergeSegThreads = 64;  // the smallest NT (LDS split below that many columns)

template <int KV, int D, int GT, int TT, int NT>
__global__ __launch_bounds__(NT) void paged_decode_merge_segment_kernel(const DecodeParams p) {
    XHIP_MERGE_SCOPE(p);
    constexpr int C4 = D / 4;
    __shared__ f32x4 s_acc[NT];
    __shared__ float s_m[NT];
    __shared__ float s_l[NT];
    const int segs = p.num_kv_heads * p.head_tiles;
    const int s = blockIdx.x / segs;
    const int seg = blockIdx.x - s * segs;
    const int kvh = seg / p.head_tiles;
    const int g0 = (seg - kvh * p.head_tiles) * GT;
    const int nh = min(GT, p.group - g0);
    const int ncols = nh * C4;
    // a head tile with no heads has nothing to merge (the host never plans
    // one; the column-span loop below needs ncols >= 1 to end)
    if (ncols <= 0) return;
    const int tid = threadIdx.x;
    // the three scalars the merge needs, requested together (the empty asm
    // keeps the compiler from sinking the prefix loads past the L == 0 exit,
    // which would cost a second round trip)
    const int L = seq_len_of(p, s);
    const int total = p.ws_prefix[p.num_seqs];
    const int pre_s = p.ws_prefix[s];
    asm volatile("" ::"s"(total), "s"(pre_s));
    const size_t qrow0 = ((size_t)s * p.num_heads + (size_t)kvh * p.group + g0) * D;

    if (L == 0) {
        if (!p.skip_empty)
            for (int col = tid; col < ncols; col += NT) write_empty_column<KV, D>(p, s, kvh, g0, qrow0, col);
        return;
    }
    const int tpw = tiles_per_wave(total, p.num_waves, p.min_tiles_per_wave);
    const int Ts = (L + TT - 1) / TT;
    const int seg_start = pre_s + seg * segment_units(p, Ts);  // in split units
    PartialSlots ps;
    if (!segment_partials<kMfmaWavesPerGroup>(p, seg_start, seg_start + p.seg_cost, Ts, tpw, ps))
        return;

    // Column span per split: all NT threads when ncols > NT / 2, else pow2(ncols).
    int span = NT;
    while ((span >> 1) >= ncols) span >>= 1;
    const int split = tid / span;  // 0 .. S-1
    const int nsplit = NT / span;
    const int cl = tid - split * span;

    float m = -INFINITY, l = 0.0f;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (cl < ncols) {
        const int h = cl / C4;
        merge_partials<GT, D, 8>(p, ps, split, nsplit, h * 2, h * D + (cl - h * C4) * 4, m, l, acc);
    }
    if (nsplit > 1) {  // ncols <= NT / 2: fewer than 64 columns, or a partly filled last head tile
        s_acc[tid] = acc;
        s_m[tid] = m;
        s_l[tid] = l;
        __syncthreads();
        if (split != 0) return;
        for (int k = 1; k < nsplit; k++) {
            const int o = k * span + cl;
            const float mk = s_m[o];
            const float M = fmaxf(m, mk);
            const float Ms = (M == -INFINITY) ? 0.0f : M;
            const float a = fast_exp2(m - Ms), b = fast_exp2(mk - Ms);
            l = l * a + s_l[o] * b;
            acc = acc * a + s_acc[o] * b;
            m = M;
        }
    }
    if (cl >= ncols) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const size_t base = qrow0 + (size_t)cl * 4;  // head-major columns
    if (p.out_f32) {
        *(f32x4 *)(p.out_f32 + base) = acc * inv;
        if (cl % C4 == 0) p.out_lse[qrow0 / D + cl / C4] = l > 0.0f ? m + log2f(l) : -INFINITY;
        return;
    }
    char *orow = o_row(p, s, kvh * p.group + g0 + cl / C4, D, KV == KV_F32 ? 4 : 2);
#pragma unroll
    for (int e = 0; e < 4; e++) store_elem<KV>(orow, (cl % C4) * 4 + e, acc[e] * inv);
}

}  // namespace xhip
