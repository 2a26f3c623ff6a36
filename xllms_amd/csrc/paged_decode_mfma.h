// MFMA tile path of the paged-decode attention (fp16 / bf16 K/V, head_size a
// multiple of 32, block_size >= 16).  One wavefront serves R row blocks of 16
// query heads of one kv head (R = 1, or 2 for groups of 17-32 heads at
// head_size <= 128): every K/V tile it loads is used by all 16R heads.
// Below, one row block; with R = 2 the QK^T MFMAs run once per block on the
// same K registers, and each V^T operand read from LDS feeds both blocks' PV
// MFMAs.
//
// Per 16-token tile (one page when block_size = 16), with g = lane/16 and
// j = lane%16 (v_mfma_f32_16x16x{32,16} operand layouts, checked on gfx950):
//   QK^T  S[token][head] = sum_d K[token][d] Q[head][d]
//         D/32 x v_mfma_f32_16x16x32: A = K rows (lane: token j, dims
//         32c+8g..+7, a 16-byte load straight from the page), B = Q of the 16
//         heads (lane: head j, same dims).  C: lane holds S[4g+r][j].
//   softmax per head j: the 16 scores of head j sit in lanes j, j+16, j+32,
//         j+48 (4 each): in-lane max, two xor shuffles, exp2, running sum.
//   PV    O^T[dim][head] += sum_t V[t][dim] P[head][t]
//         D/16 x v_mfma_f32_16x16x16 (twice: P = P_hi + P_lo in the 16-bit
//         type, so the product keeps ~22 bits of P): B = P, which is exactly
//         the C layout of the QK^T step (lane: head j, tokens 4g..4g+3);
//         A = V^T (lane: dim 16n+j, tokens 4g..4g+3), read from the V tile
//         staged in LDS.  C: lane holds O^T[16n+4g+r][j].
// The V tile goes global -> registers -> LDS (row stride 2*D+8 bytes so the
// four token groups of a V^T read fall in different LDS banks).  Loads are
// buffer loads: a token past the end of the range, or in a page with a
// negative id, gets an out-of-range offset and reads as zero without touching
// memory; its score is masked to -inf.  The next tile's K/V loads are issued
// before the current tile is computed.
#pragma once

#include "paged_decode_kernels.h"
#include "wg_trace.h"

namespace xhip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOobOffset = 0x80000000u;

template <int D> struct MfmaGeometry {
    static constexpr int kTile = 16;             // tokens per tile
    static constexpr int kChunks = D / 8;        // 16-byte chunks per 16-bit row
    static constexpr int kQkSteps = D / 32;      // QK^T MFMAs = K loads per lane
    static constexpr int kVLoads = D / 32;       // V 16-byte loads per lane (16 rows)
    static constexpr int kDimBlocks = D / 16;    // PV MFMAs per P half
    static constexpr int kLdsRow = 2 * D + 8;    // bytes per staged V row
    static constexpr int kLdsTile = 16 * kLdsRow;
    static_assert(D % 32 == 0, "MFMA path needs head_size % 32 == 0");
};

template <int KV> __device__ __forceinline__ f32x4 mfma_qk(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (KV == KV_F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <int KV> __device__ __forceinline__ f32x4 mfma_pv(u32x2 a, u32x2 b, f32x4 c) {
    if constexpr (KV == KV_F16)
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                     __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                         __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}


__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char *base) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7FFFFFFF, 0x00020000);
}

// K/V pages are streamed once per launch: nontemporal loads (cache policy
// `nt`).  On MI355X they raise the read rate of this access pattern (random
// 4 KB runs, 16-byte lane loads) from ~5.9 to ~6.6 TB/s.
constexpr int kStreamPolicy = 2;

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kStreamPolicy);
}

__device__ __forceinline__ u32x4 buf_load16_cached(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

template <int D> struct MfmaTileRegs {
    u32x4 k[MfmaGeometry<D>::kQkSteps];
    u32x4 v[MfmaGeometry<D>::kVLoads];
};

// Issue the K and V loads of the tile starting at token t0 (block id blk):
// rows past t_end or in a negative page read as zero.
template <int D>
__device__ __forceinline__ void mfma_load_tile(const DecodeParams &p, const char *kb,
                                               const char *vb, int t0, int t_end, int blk,
                                               int lane, bool cached, MfmaTileRegs<D> &r) {
    using G = MfmaGeometry<D>;
    const int bmask = p.block_size - 1;
    const bool page_ok = blk >= 0;
    const long long page = (long long)blk * p.kv_block_stride + (long long)(t0 & bmask) * D;
    const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kb + page * 2);
    const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vb + page * 2);
    const int j = lane & 15, g = lane >> 4;
    const bool krow_ok = page_ok && (t0 + j < t_end);
    uint32_t koff[G::kQkSteps], voff[G::kVLoads];
#pragma unroll
    for (int c = 0; c < G::kQkSteps; c++)
        koff[c] = krow_ok ? (uint32_t)(j * 2 * D + 64 * c + 16 * g) : kOobOffset;
#pragma unroll
    for (int c = 0; c < G::kVLoads; c++) {
        const int q = 64 * c + lane;
        const int row = q / G::kChunks;
        const int chunk = q - row * G::kChunks;
        const bool ok = page_ok && (t0 + row < t_end);
        voff[c] = ok ? (uint32_t)(row * 2 * D + 16 * chunk) : kOobOffset;
    }
    if (cached) {
#pragma unroll
        for (int c = 0; c < G::kQkSteps; c++) r.k[c] = buf_load16_cached(rk, koff[c]);
#pragma unroll
        for (int c = 0; c < G::kVLoads; c++) r.v[c] = buf_load16_cached(rv, voff[c]);
    } else {
#pragma unroll
        for (int c = 0; c < G::kQkSteps; c++) r.k[c] = buf_load16(rk, koff[c]);
#pragma unroll
        for (int c = 0; c < G::kVLoads; c++) r.v[c] = buf_load16(rv, voff[c]);
    }
}

// Running state of one wavefront over one segment: lane (g, j) owns head j.
template <int D> struct MfmaState {
    f32x4 o[MfmaGeometry<D>::kDimBlocks];  // O^T[16n + 4g + r][j]
    float m;                               // running max of head j (log2 units)
    float l;                               // this lane's part of the running sum
};

template <int KV, int D, int R>
__device__ __forceinline__ void mfma_tile(const DecodeParams &p, const u32x4 (*q)[MfmaGeometry<D>::kQkSteps],
                                          int t0, int t_end, bool page_ok, int lane, char *lds,
                                          const MfmaTileRegs<D> &r, MfmaState<D> (&st)[R]) {
    using G = MfmaGeometry<D>;
    const int j = lane & 15, g = lane >> 4;

    // V tile -> LDS (row-major, padded rows), two 8-byte writes per chunk.
#pragma unroll
    for (int c = 0; c < G::kVLoads; c++) {
        const int qi = 64 * c + lane;
        const int row = qi / G::kChunks;
        const int chunk = qi - row * G::kChunks;
        u32x2 *dst = (u32x2 *)(lds + row * G::kLdsRow + 16 * chunk);
        dst[0] = u32x2{r.v[c][0], r.v[c][1]};
        dst[1] = u32x2{r.v[c][2], r.v[c][3]};
    }

    // S = K Q^T for 16 tokens x 16 heads, per row block.
    f32x4 s[R];
#pragma unroll
    for (int b = 0; b < R; b++) s[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < G::kQkSteps; c++)
#pragma unroll
        for (int b = 0; b < R; b++) s[b] = mfma_qk<KV>(r.k[c], q[b][c], s[b]);

    bool ok[4];
#pragma unroll
    for (int i = 0; i < 4; i++) ok[i] = page_ok && (t0 + 4 * g + i < t_end);

    // Online softmax of head j over tokens 4g..4g+3 of this lane; P in the
    // 16-bit type as hi + lo parts (B operand of the PV MFMA).
    u32x2 p_hi[R], p_lo[R];
#pragma unroll
    for (int b = 0; b < R; b++) {
        float sc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) sc[i] = ok[i] ? s[b][i] * p.scale_log2 : -INFINITY;
        float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(st[b].m, mx);
        const float ms = (m_new == -INFINITY) ? 0.0f : m_new;
        const float alpha = fast_exp2(st[b].m - ms);
        float pe[4];
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pe[i] = fast_exp2(sc[i] - ms);
            psum += pe[i];
        }
        st[b].l = st[b].l * alpha + psum;
        st[b].m = m_new;
        // P = hi + lo in the 16-bit type (lo = the exact fp32 remainder of hi)
        const uint32_t h01 = pack16<KV>(pe[0], pe[1]), h23 = pack16<KV>(pe[2], pe[3]);
        const f32x2 r01 = unpack16<KV>(h01), r23 = unpack16<KV>(h23);
        p_hi[b] = u32x2{h01, h23};
        p_lo[b] = u32x2{pack16<KV>(pe[0] - r01.x, pe[1] - r01.y),
                        pack16<KV>(pe[2] - r23.x, pe[3] - r23.y)};
        // Rescale only when some head's running max moved: alpha is then
        // exactly 1 in every lane, and x * 1 == x, so skipping is exact (past
        // the first few hundred tokens most tiles skip).
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int n = 0; n < G::kDimBlocks; n++) st[b].o[n] *= alpha;
        }
    }

    // O^T += V^T P for every 16-dim block.
    const char *vrow = lds + (4 * g) * G::kLdsRow + 2 * j;
#pragma unroll
    for (int n = 0; n < G::kDimBlocks; n++) {
        const char *src = vrow + 32 * n;
        const uint32_t v0 = *(const uint16_t *)(src);
        const uint32_t v1 = *(const uint16_t *)(src + G::kLdsRow);
        const uint32_t v2 = *(const uint16_t *)(src + 2 * G::kLdsRow);
        const uint32_t v3 = *(const uint16_t *)(src + 3 * G::kLdsRow);
        const u32x2 a = {v0 | (v1 << 16), v2 | (v3 << 16)};
#pragma unroll
        for (int b = 0; b < R; b++) {
            st[b].o[n] = mfma_pv<KV>(a, p_hi[b], st[b].o[n]);
            st[b].o[n] = mfma_pv<KV>(a, p_lo[b], st[b].o[n]);
        }
    }
}

// Where the partition body finds a sequence's length, block table and query
// rows.  kSrcBatch: the batch's own arrays (DecodeParams and the lens /
// tables kernel arguments).  The cascade's in-kernel plan
// (paged_decode_cascade_attn.h) keeps the per-sequence data of its two
// batches in LDS (CascadeLdsPlan) and reads the caller's block tables and
// query rows in place: kSrcSuffix, the suffix of each caller sequence (its
// length past the shared prefix, its pages from its first private one);
// kSrcPrefix, the prefix-batch sequences (a group's shared pages, from its
// lowest member's table row, and query rows gathered from its members).
enum { kSrcBatch = 0, kSrcSuffix = 1, kSrcPrefix = 2 };

struct CascadeLdsPlan {
    const int *slen;    // [num_seqs] suffix length of caller sequence s
    const int *soff;    // [num_seqs] its shared prefix pages (the suffix's first page)
    const int *vlen;    // [v_max] length of prefix-batch sequence v (0: unused)
    const int *vrow;    // [v_max] block-table row of v's pages (its group's lowest member)
    const int *vdesc;   // [v_max][4] v's group: its first prefix-batch sequence, its
                        // members, -, the group id (-1: v unused)
    const int *grp;     // [num_seqs] group of caller sequence s (-1: none)
    int *win;           // [waves per workgroup][32] each wavefront's members of a piece
    int *p_row;         // [num_seqs] (global) a member's first row in the prefix batch
    const char *q;      // caller's query rows: [num_seqs][num_heads][head_size]
    const char *const *q_rows;  // or, when set, sequence s's rows at q_rows[s]
    int num_heads;      // caller's query heads
    int group;          // caller's query heads per kv head
    int rows;           // query rows per kv head of a prefix-batch sequence
    int num_seqs;       // caller's sequences
};

// Clamped length of sequence s of the batch under source SRC.
template <int SRC>
__device__ __forceinline__ int src_len(const DecodeParams &p, const int *__restrict__ lens, int s,
                                       const CascadeLdsPlan *cp) {
    if constexpr (SRC == kSrcBatch)
        return p.nt_fold ? p.nt_len - 1 : min(max(lens[s], 0), p.max_ctx);
    else if constexpr (SRC == kSrcSuffix) return __builtin_amdgcn_readfirstlane(cp->slen[s]);
    else return __builtin_amdgcn_readfirstlane(cp->vlen[s]);
}

// Block table of sequence s of the batch under source SRC.
template <int SRC>
__device__ __forceinline__ const int *src_table(const DecodeParams &p,
                                                const int *__restrict__ tables, int s,
                                                const CascadeLdsPlan *cp) {
    if constexpr (SRC == kSrcBatch) return tables + (size_t)s * p.max_blocks;
    else if constexpr (SRC == kSrcSuffix)
        return tables + (size_t)s * p.max_blocks + __builtin_amdgcn_readfirstlane(cp->soff[s]);
    else return tables + (size_t)__builtin_amdgcn_readfirstlane(cp->vrow[s]) * p.max_blocks;
}

// One piece of a wavefront's stream-K range: tokens [t_begin, t_end) of the
// segment (sequence s, kv head kvh, head tile ht).  `whole`: the piece is the
// entire segment (the output is written directly); else its partial goes to
// `slot`.  All fields are wavefront-uniform.
struct MfmaPiece {
    int s, kvh, ht, t_begin, t_end, L, whole, slot;
};

// Cursor over the pieces of one wavefront's range [g, g_end) of the batch's
// split units; s is the sequence holding unit g, w the wavefront (its
// partial slots), ht its head tile under paired head tiles (else -1).
struct RangeCursor {
    int g, g_end, s, first, w, ht;
};

// The next piece of the range (false at its end).  Same decomposition as
// stream_k_walk, one piece at a time, so the kernel can look one piece ahead.
// A range that ends inside a segment's start-up units makes no piece of it.
template <int TT, int SRC = kSrcBatch>
__device__ __forceinline__ bool next_piece(const DecodeParams &p, const int *__restrict__ lens,
                                           const int *pre, RangeCursor &c, MfmaPiece &pc,
                                           const CascadeLdsPlan *cp = nullptr) {
    const int segs = seq_segments(p);
    while (c.g < c.g_end) {
        const int L = src_len<SRC>(p, lens, c.s, cp);
        const int Ts = (L + TT - 1) / TT;
        const int Cs = segment_units(p, Ts);
        const int base = __builtin_amdgcn_readfirstlane(pre[c.s]);
        const int local = c.g - base;
        const int seg = local / Cs;
        const int u0 = local - seg * Cs;
        const int u1 = min(Cs, u0 + (c.g_end - c.g));
        const int t0 = max(u0 - p.seg_cost, 0), t1 = max(u1 - p.seg_cost, 0);
        c.g += u1 - u0;
        const int cur_s = c.s;
        if (c.g - base >= Cs * segs) {  // sequence done: next one with tiles
            int s = c.s + 1;
            while (s < p.num_seqs - 1 && pre[s + 1] == pre[s]) s++;
            c.s = __builtin_amdgcn_readfirstlane(s);
        }
        if (t1 <= t0) continue;  // only start-up units of this segment (the range's end)
        pc.s = cur_s;
        if (c.ht >= 0) {  // paired head tiles: a segment per kv head
            pc.kvh = seg;
            pc.ht = c.ht;
        } else {
            pc.kvh = seg / p.head_tiles;
            pc.ht = seg - pc.kvh * p.head_tiles;
        }
        pc.t_begin = t0 * TT;
        pc.t_end = min(L, t1 * TT);
        pc.L = L;
        pc.whole = t0 == 0 && t1 == Ts;
        pc.slot = c.w * 2 + (c.first ? 0 : 1);
        c.first = 0;
        return true;
    }
    return false;
}

// Q rows of the piece's (up to) 16R query heads in the MFMA B layout (row
// block b, lane: head 16b + j, dims 32c+8g..+7); heads past the group read
// as zero.  kSrcPrefix: with the group's rows laid end to end (rows per
// prefix-batch sequence), row k is query head k % G (of the kv head's G) of
// the group's member of rank k / G, members ranked in sequence order; rows
// past the last member read as zero.  The wavefront finds the (at most 16R)
// members of its rows with one ballot per 64 caller sequences, and the piece
// that starts its sequence's kv head 0 stores each member's first row
// (p_row).
template <int D, int R, int SRC = kSrcBatch>
__device__ __forceinline__ void mfma_load_q(const DecodeParams &p, const MfmaPiece &pc, int lane,
                                            u32x4 (&q)[R][MfmaGeometry<D>::kQkSteps],
                                            const CascadeLdsPlan *cp = nullptr) {
    const int j = lane & 15, g = lane >> 4;
    const int g0 = pc.ht * kMfmaHeads * R;
    if constexpr (SRC == kSrcPrefix) {
        const int *d = cp->vdesc + 4 * pc.s;
        const int vbase = __builtin_amdgcn_readfirstlane(d[0]);
        const int count = __builtin_amdgcn_readfirstlane(d[1]);
        const int gid = __builtin_amdgcn_readfirstlane(d[3]);
        const int G = cp->group;
        const int row0 = (pc.s - vbase) * cp->rows + g0;
        const int r_lo = row0 / G, r_hi = min((row0 + 16 * R - 1) / G, count - 1);
        int *win = cp->win + (threadIdx.x >> 6) * (16 * R);
        int acc = 0;
        for (int c0 = 0; c0 < cp->num_seqs && acc <= r_hi; c0 += 64) {
            const int s = c0 + lane;
            const bool in = s < cp->num_seqs && cp->grp[s] == gid;
            const unsigned long long m = __ballot(in);
            const int rk = acc + (int)__builtin_amdgcn_mbcnt_hi(
                                     (unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u));
            if (in && rk >= r_lo && rk <= r_hi) win[rk - r_lo] = s;
            acc += __popcll(m);
        }
        // (the window is written and read by this wavefront: its LDS
        // accesses complete in order)
        __builtin_amdgcn_wave_barrier();
        const size_t row_bytes = (size_t)D * 2;
        const bool first = pc.kvh == 0 && pc.t_begin == 0;
#pragma unroll
        for (int b = 0; b < R; b++) {
            const int rig = row0 + 16 * b + j;
            const int r = rig / G, gq = rig - r * G;
            const char *src = nullptr;
            if (r < count) {
                const int s = win[r - r_lo];
                const size_t h = (size_t)pc.kvh * G + gq;
                src = cp->q_rows ? cp->q_rows[s] + h * row_bytes
                                 : cp->q + ((size_t)s * cp->num_heads + h) * row_bytes;
                if (first && gq == 0 && g == 0) cp->p_row[s] = vbase * cp->rows + r * G;
            }
#pragma unroll
            for (int c = 0; c < MfmaGeometry<D>::kQkSteps; c++)
                q[b][c] = src ? load16(src + (size_t)(32 * c + 8 * g) * 2) : u32x4{0, 0, 0, 0};
        }
        return;
    }
    const int nh = min(kMfmaHeads * R, p.group - g0);
    const char *q0 = q_row(p, pc.s, pc.kvh * p.group + g0, D, 2);
#pragma unroll
    for (int b = 0; b < R; b++)
#pragma unroll
        for (int c = 0; c < MfmaGeometry<D>::kQkSteps; c++)
            q[b][c] = (16 * b + j < nh)
                          ? load16(q0 + ((size_t)(16 * b + j) * D + 32 * c + 8 * g) * 2)
                          : u32x4{0, 0, 0, 0};
}

// Prefix fold (DecodeParams::fold_row) of a piece that starts its segment:
// the prefix pass's result for each head, (m = lse, l = 1, O^T = the
// normalized prefix row), is merged into the piece's state after its last
// tile, like one more partial.  Its loads are issued when the piece begins
// (R = 1), so their latency hides behind the piece's tiles; with R = 2 the 32
// extra registers would not fit, and they are loaded at the end.
template <int D, int R> struct MfmaFold {
    f32x4 o[R][MfmaGeometry<D>::kDimBlocks];
    float m[R];
    int base;  // the sequence's fold base, < 0: no fold
};

template <int D, int R>
__device__ __forceinline__ void mfma_fold_load(const DecodeParams &p, const MfmaPiece &pc,
                                               int lane, MfmaFold<D, R> &f) {
    const int j = lane & 15, g = lane >> 4;
    const int g0 = pc.ht * kMfmaHeads * R;
    const int nh = min(kMfmaHeads * R, p.group - g0);
#pragma unroll
    for (int b = 0; b < R; b++) {
        // heads past the group read head g0 (valid) and are never written
        const size_t r = fold_state_row(p, f.base, pc.kvh, g0 + (16 * b + j < nh ? 16 * b + j : 0));
        f.m[b] = p.fold_lse[r];
#pragma unroll
        for (int n = 0; n < MfmaGeometry<D>::kDimBlocks; n++)
            f.o[b][n] = *(const f32x4 *)(p.fold_out + r * D + 16 * n + 4 * g);
    }
}

template <int D, int R>
__device__ __forceinline__ void mfma_fold_apply(const MfmaFold<D, R> &f, int lane,
                                                MfmaState<D> (&st)[R]) {
    const int g = lane >> 4;
#pragma unroll
    for (int b = 0; b < R; b++) {
        const float M = fmaxf(st[b].m, f.m[b]);
        const float Ms = (M == -INFINITY) ? 0.0f : M;
        const float a = fast_exp2(st[b].m - Ms), w = fast_exp2(f.m[b] - Ms);
        st[b].l = st[b].l * a + (g == 0 ? w : 0.0f);  // l is summed over the 4 lane groups
#pragma unroll
        for (int n = 0; n < MfmaGeometry<D>::kDimBlocks; n++)
            st[b].o[n] = st[b].o[n] * a + f.o[b][n] * w;
        st[b].m = M;
    }
}

// Block ids of the piece's tiles first .. first+63, lane i holding tile
// first+i (clamped to the piece's last tile).
template <int SRC = kSrcBatch>
__device__ __forceinline__ int mfma_load_ids(const DecodeParams &p, const int *__restrict__ tables,
                                             const MfmaPiece &pc, int first, int lane,
                                             const CascadeLdsPlan *cp = nullptr) {
    const int *bt = src_table<SRC>(p, tables, pc.s, cp);
    const int ti = pc.t_begin + 16 * (first + lane);
    return bt[(ti < pc.t_end ? ti : pc.t_end - 1) >> p.bs_shift];
}

}  // namespace xhip

namespace xhip {

// Where a finished segment's rows go: its output rows (element type), or in
// partial-output mode its fp32 rows and log-sum-exp.  st holds unreduced
// per-lane sums (lane group g of head j); they are reduced here.
template <int KV, int D, int R, bool HS = false>
__device__ __forceinline__ void mfma_write_rows(const DecodeParams &p, const MfmaPiece &pc,
                                                int lane, const MfmaState<D> (&st)[R]) {
    using G = MfmaGeometry<D>;
    constexpr int GT = kMfmaHeads * R;
    const int j = lane & 15, gq = lane >> 4;
    const int g0 = pc.ht * GT;
    const int nh = min(GT, p.group - g0);
    const size_t qrow0 = ((size_t)pc.s * p.num_heads + (size_t)pc.kvh * p.group + g0) * D;
#pragma unroll
    for (int b = 0; b < R; b++) {
        float l = st[b].l;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const int hj = 16 * b + j;  // head of this lane in the tile
        if (hj >= nh) continue;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        if constexpr (HS) {
            char *dst = (char *)p.out_h + (qrow0 + (size_t)hj * D + 4 * gq) * 2;
#pragma unroll
            for (int n = 0; n < G::kDimBlocks; n++) {
                const f32x4 o = st[b].o[n] * inv;
                *(u32x2 *)(dst + 32 * n) =
                    u32x2{pack16<KV_F16>(o[0], o[1]), pack16<KV_F16>(o[2], o[3])};
            }
            if (gq == 0) p.out_lse[qrow0 / D + hj] = l > 0.0f ? st[b].m + log2f(l) : -INFINITY;
        } else if (p.out_f32) {
            float *dst = p.out_f32 + qrow0 + (size_t)hj * D + 4 * gq;
#pragma unroll
            for (int n = 0; n < G::kDimBlocks; n++) *(f32x4 *)(dst + 16 * n) = st[b].o[n] * inv;
            if (gq == 0) p.out_lse[qrow0 / D + hj] = l > 0.0f ? st[b].m + log2f(l) : -INFINITY;
        } else {
            char *dst = o_row(p, pc.s, pc.kvh * p.group + g0 + hj, D, 2) + 4 * gq * 2;
#pragma unroll
            for (int n = 0; n < G::kDimBlocks; n++) {
                const f32x4 o = st[b].o[n] * inv;
                *(u32x2 *)(dst + 32 * n) = u32x2{pack16<KV>(o[0], o[1]), pack16<KV>(o[2], o[3])};
            }
        }
    }
}

// The partial of a cut segment's piece, in the piece's slot of the split-K
// workspace: fp32 (m, l, unnormalized o), or HS: an fp16 state
// (DecodeParams::ws_h) (m + log2 l, 1, o / l in fp16).
template <int D, int R, bool HS = false>
__device__ __forceinline__ void mfma_write_partial(const DecodeParams &p, const MfmaPiece &pc,
                                                   int lane, const MfmaState<D> (&st)[R]) {
    using G = MfmaGeometry<D>;
    constexpr int GT = kMfmaHeads * R;
    const int j = lane & 15, gq = lane >> 4;
    const int nh = min(GT, p.group - pc.ht * GT);
#pragma unroll
    for (int b = 0; b < R; b++) {
        float l = st[b].l;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const int hj = 16 * b + j;
        if (hj >= nh) continue;
        if constexpr (HS) {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            char *dst = (char *)p.ws_h + (((size_t)pc.slot * GT + hj) * D + 4 * gq) * 2;
#pragma unroll
            for (int n = 0; n < G::kDimBlocks; n++) {
                const f32x4 o = st[b].o[n] * inv;
                *(u32x2 *)(dst + 32 * n) =
                    u32x2{pack16<KV_F16>(o[0], o[1]), pack16<KV_F16>(o[2], o[3])};
            }
            if (gq == 0) {
                p.ws_ml[((size_t)pc.slot * GT + hj) * 2] =
                    l > 0.0f ? st[b].m + log2f(l) : -INFINITY;
                p.ws_ml[((size_t)pc.slot * GT + hj) * 2 + 1] = l > 0.0f ? 1.0f : 0.0f;
            }
            continue;
        }
        float *dst = p.ws_o + ((size_t)pc.slot * GT + hj) * D + 4 * gq;
#pragma unroll
        for (int n = 0; n < G::kDimBlocks; n++) *(f32x4 *)(dst + 16 * n) = st[b].o[n];
        if (gq == 0) {
            p.ws_ml[((size_t)pc.slot * GT + hj) * 2] = st[b].m;
            p.ws_ml[((size_t)pc.slot * GT + hj) * 2 + 1] = l;
        }
    }
}

// LDS slot of one wavefront for the workgroup-level combine (mfma_wg_fixup):
// a state in the lane layout of MfmaState (per-lane o, m and unreduced l),
// so two states merge lane by lane.
template <int D> struct MfmaFixSlot {
    f32x4 o[MfmaGeometry<D>::kDimBlocks][64];
    float m[64], l[64];
    int ends;  // the state reaches the end of its segment
};

template <int D>
__device__ __forceinline__ void fix_store(MfmaFixSlot<D> &slot, int lane, const MfmaState<D> &st) {
#pragma unroll
    for (int n = 0; n < MfmaGeometry<D>::kDimBlocks; n++) slot.o[n][lane] = st.o[n];
    slot.m[lane] = st.m;
    slot.l[lane] = st.l;
}

template <int D>
__device__ __forceinline__ void fix_load(const MfmaFixSlot<D> &slot, int lane, MfmaState<D> &st) {
#pragma unroll
    for (int n = 0; n < MfmaGeometry<D>::kDimBlocks; n++) st.o[n] = slot.o[n][lane];
    st.m = slot.m[lane];
    st.l = slot.l[lane];
}

// st <- st (+) the state in slot (online log-sum-exp, per lane).
template <int D>
__device__ __forceinline__ void fix_absorb(const MfmaFixSlot<D> &slot, int lane, MfmaState<D> &st) {
    const float mo = slot.m[lane];
    const float M = fmaxf(st.m, mo);
    const float Ms = (M == -INFINITY) ? 0.0f : M;
    const float a = fast_exp2(st.m - Ms), b = fast_exp2(mo - Ms);
    st.l = st.l * a + slot.l[lane] * b;
#pragma unroll
    for (int n = 0; n < MfmaGeometry<D>::kDimBlocks; n++) st.o[n] = st.o[n] * a + slot.o[n][lane] * b;
    st.m = M;
}

// The workgroup's relay slot of the mode-2 combine: one state of R row
// blocks in the lane layout, and per wavefront whether it relayed its state
// there (and whether that state reaches the end of its segment).
template <int D, int R> struct MfmaRelaySlot {
    f32x4 o[R][MfmaGeometry<D>::kDimBlocks][64];
    float m[R][64], l[R][64];
    int relayed[kMfmaWavesPerGroup];
    int ends[kMfmaWavesPerGroup];
};

// LDS of one workgroup of the partition kernel: the V tile staging of each
// wavefront, and the slots of the workgroup-level combine (by mode).
template <int FIX, int D, int R> struct MfmaSweepLds {
    int unused;
};
template <int D, int R> struct MfmaSweepLds<1, D, R> {
    MfmaFixSlot<D> fix[kMfmaWavesPerGroup];
};
template <int D, int R> struct MfmaSweepLds<2, D, R> {
    MfmaRelaySlot<D, R> relay;
};
template <int D, int R, int FIX = mfma_wg_fixup(kMfmaHeads * R, D)> struct MfmaLds {
    __attribute__((aligned(16))) char vtile[kMfmaWavesPerGroup][MfmaGeometry<D>::kLdsTile];
    MfmaSweepLds<FIX, D, R> sw;
};

// st <- st (+) the partial in workspace slot `slot` (its l is the reduced
// sum: lane group 0 takes it; fp32, or HS: an fp16 state).  Rows past the group
// were never written; they are left alone.
template <int D, int R, bool HS = false>
__device__ __forceinline__ void absorb_partial(const DecodeParams &p, int slot, int ht, int lane,
                                               MfmaState<D> (&st)[R]) {
    constexpr int GT = kMfmaHeads * R;
    const int j = lane & 15, gq = lane >> 4;
    const int nh = min(GT, p.group - ht * GT);
#pragma unroll
    for (int b = 0; b < R; b++) {
        const int hj = 16 * b + j;
        if (hj >= nh) continue;
        const size_t at = ((size_t)slot * GT + hj) * D + 4 * gq;
        const float mo = p.ws_ml[((size_t)slot * GT + hj) * 2];
        const float lo = gq == 0 ? p.ws_ml[((size_t)slot * GT + hj) * 2 + 1] : 0.0f;
        const float M = fmaxf(st[b].m, mo);
        const float Ms = (M == -INFINITY) ? 0.0f : M;
        const float a = fast_exp2(st[b].m - Ms), w = fast_exp2(mo - Ms);
        st[b].l = st[b].l * a + lo * w;
#pragma unroll
        for (int n = 0; n < MfmaGeometry<D>::kDimBlocks; n++)
            st[b].o[n] = st[b].o[n] * a + partial_f32x4<HS>(p, at + 16 * n) * w;
        st[b].m = M;
    }
}

// Partition kernel, MFMA tile path (head tile of 16R query heads).
//
// A wavefront walks the pieces of its stream-K range (usually one or two
// segments) as one pipeline: while the last tile of a piece is computed, the
// next piece's first K/V tile is already in flight, and its block ids were
// requested when the current piece began.  Without this look-ahead a
// wavefront whose range crosses a segment boundary waited on a chain of
// dependent loads (block ids, then the first tile) at the crossing, and those
// wavefronts finished the launch last (measured on MI355X: 3 us later on
// average at config 2).  Q is loaded when its piece begins: requesting the
// next piece's Q a piece early as well gained ~1% at configs 2-4 but cost 5%
// (cascade) to 10% (plain decode) at config 5 (measured, same box).
//
// Cut segments (mfma_wg_fixup instantiations).  A piece that is not a whole
// segment is cut at the start (it continues the previous wavefront's range),
// at the end (the next wavefront continues it), or both.  Writing each such
// piece's fp32 partial to memory put ~16-20 MB of stores at config 4b into
// the wavefronts' critical paths (a cut first piece's stores delay the next
// piece's loads, which share the memory counter; every wavefront ends with
// one), measured at 8.6 us of a 76 us kernel.  Instead: a cut first piece
// followed by more pieces goes to the wavefront's LDS slot; the last piece's
// state stays in registers; at the end, a last piece that continues the
// left neighbour's goes to the slot too, and after one workgroup barrier
// the leftmost holder of each segment in the workgroup absorbs the slots of
// the neighbours its piece continues into and writes it: finished rows when
// the whole segment lay in the workgroup, else one partial.  (A sweep from
// the last wavefront down to the first, one barrier per wavefront, kept the
// workgroup ~1.8 us past its last tile, measured on MI355X.)  The first
// wavefront's cut first piece (its left neighbour is in another workgroup)
// is written as a partial after its range, from its slot.
// Mode 2 (two row blocks) keeps one relay slot per workgroup: cut first
// pieces followed by more pieces are written as partials by every
// wavefront, and a left neighbour absorbs such a partial from memory (the
// workgroup barrier orders it) instead of from the relay slot.
//
// The body runs one workgroup's four ranges: logical workgroup `wg` of a
// plan of `waves` wavefronts over the batch of p, whose split-unit prefix
// `pre` is in LDS.  PAIR: the batch's head tiles are paired
// (DecodeParams::pair_tiles): the workgroup's two pairs of wavefronts walk
// two ranges, one head tile per wavefront, and every cut piece leaves its
// own partial (no workgroup combine).  SRC: where the batch's per-sequence
// data is (kSrcBatch: lens / tables and p; else the in-kernel cascade plan
// cp).  HS: partial-output rows and partials are fp16 states
// (DecodeParams::out_h, ws_h).
template <int KV, int D, int R, bool PAIR = false, int SRC = kSrcBatch, bool HS = false>
__device__ __forceinline__ void mfma_partition_body(
    const DecodeParams &p, const int *__restrict__ lens, const int *__restrict__ tables,
    const int *pre, int wg, int waves,
    MfmaLds<D, R, PAIR ? 0 : mfma_wg_fixup(kMfmaHeads * R, D)> &sm,
    const CascadeLdsPlan *cp = nullptr) {
    using G = MfmaGeometry<D>;
    constexpr int FIX = PAIR ? 0 : mfma_wg_fixup(kMfmaHeads * R, D);
    constexpr int NW = kMfmaWavesPerGroup;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    char *lds = sm.vtile[wave];
    if constexpr (FIX == 2) {
        // ordered before any read by the sweep's first barrier
        if (lane == 0) sm.sw.relay.relayed[wave] = 0;
    }

    const int B = p.num_seqs;
    const int total = pre[B];
    const int w = wg * NW + wave;
    const int wr = PAIR ? w >> 1 : w;  // this wavefront's range
    const int tpw = tiles_per_wave(total, PAIR ? waves >> 1 : waves, p.min_tiles_per_wave);
    const long long g_lo = (long long)wr * tpw;

    MfmaState<D> st[R];   // the state of the piece being computed; after the loop, the last one's
    MfmaPiece pc;         // the piece being computed; after the loop, the last one
    bool have_last = false;  // FIX: the last piece is cut (its state is kept for the sweep)
    MfmaPiece pc_first;      // FIX == 1, first wavefront: its cut first piece, saved in its slot
    bool first_saved = false;
#if XHIP_TRACING
    int n_tiles = 0, n_pieces = 0;
#endif
    RangeCursor cur;
    cur.g = (int)g_lo;
    cur.g_end = g_lo < total ? min(total, cur.g + tpw) : cur.g;
    cur.first = 1;
    cur.w = w;
    cur.ht = PAIR ? (w & 1) : -1;
    {
        // the sequence holding unit g: the last s with pre[s] <= g (empty
        // sequences share their successor's prefix, so this lands on one
        // with tiles)
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pre[mid] <= cur.g) lo = mid; else hi = mid - 1;
        }
        cur.s = __builtin_amdgcn_readfirstlane(lo);
    }

    // A range inside one segment's start-up units holds no tile (only when
    // tpw <= seg_cost); the segment's tiles belong to the next wavefront.
    if (g_lo < total && next_piece<16, SRC>(p, lens, pre, cur, pc, cp)) {
        u32x4 q[R][G::kQkSteps];
        int ids;
        if constexpr (SRC == kSrcPrefix) {
            // (the block ids' round trip overlaps the members' lookup)
            ids = mfma_load_ids<SRC>(p, tables, pc, 0, lane, cp);
            mfma_load_q<D, R, SRC>(p, pc, lane, q, cp);
        } else {
            mfma_load_q<D, R, SRC>(p, pc, lane, q, cp);
            ids = mfma_load_ids<SRC>(p, tables, pc, 0, lane, cp);
        }
        // fold base of the current piece (requested a piece ahead from here on)
        int fold_base = (p.fold_row && pc.t_begin == 0) ? p.fold_row[pc.s] : -1;
        MfmaTileRegs<D> ra, rb;
        int blk_a = __builtin_amdgcn_readlane(ids, 0);
        XHIP_WAVE_STAMP(p, wave, 0);
        {
            const char *kb = (const char *)p.k + (size_t)pc.kvh * (size_t)p.kv_head_stride * 2;
            const char *vb = (const char *)p.v + (size_t)pc.kvh * (size_t)p.kv_head_stride * 2;
            mfma_load_tile<D>(p, kb, vb, pc.t_begin, pc.t_end, blk_a, lane, pc.s < p.cached_seqs,
                              ra);
        }

        while (true) {
            MfmaPiece pn = pc;
            const bool has_next = next_piece<16, SRC>(p, lens, pre, cur, pn, cp);
            // Issued whether or not there is a next piece (pn is then the
            // current one again), so every path through the loop below has
            // the same loads in flight and the compiler's wait counts stay
            // exact.
            const int ids_n = mfma_load_ids<SRC>(p, tables, pn, 0, lane, cp);
            const int fold_base_n =
                (p.fold_row && has_next && pn.t_begin == 0) ? p.fold_row[pn.s] : -1;
            const char *kb = (const char *)p.k + (size_t)pc.kvh * (size_t)p.kv_head_stride * 2;
            const char *vb = (const char *)p.v + (size_t)pc.kvh * (size_t)p.kv_head_stride * 2;
            const char *kb_n = (const char *)p.k + (size_t)pn.kvh * (size_t)p.kv_head_stride * 2;
            const char *vb_n = (const char *)p.v + (size_t)pn.kvh * (size_t)p.kv_head_stride * 2;
            const bool cached = pc.s < p.cached_seqs;
            const bool cached_n = has_next && pn.s < p.cached_seqs;
            const int *bt = src_table<SRC>(p, tables, pc.s, cp);

#pragma unroll
            for (int b = 0; b < R; b++) {
#pragma unroll
                for (int n = 0; n < G::kDimBlocks; n++) st[b].o[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                st[b].m = -INFINITY;
                st[b].l = 0.0f;
            }
            MfmaFold<D, R> fold;
            fold.base = fold_base;
            if (R == 1 && fold.base >= 0) mfma_fold_load<D, R>(p, pc, lane, fold);
            const int ntiles = (pc.t_end - pc.t_begin + 15) >> 4;
#if XHIP_TRACING
            n_tiles += ntiles;
            n_pieces++;
#endif
            for (int i = 0; i < ntiles; i++) {
                if (i > 0 && (i & 63) == 0) ids = mfma_load_ids<SRC>(p, tables, pc, i, lane, cp);
                const int t0 = pc.t_begin + 16 * i;
                // The next tile: this piece's, else the next piece's first (all
                // rows out of range when there is none).
                const int nl = (i + 1) & 63;
                const bool in_piece = i + 1 < ntiles;
                int blk_b;
                if (in_piece)
                    blk_b = nl != 0 ? __builtin_amdgcn_readlane(ids, nl) : bt[(t0 + 16) >> p.bs_shift];
                else
                    blk_b = has_next ? __builtin_amdgcn_readlane(ids_n, 0) : -1;
                mfma_load_tile<D>(p, in_piece ? kb : kb_n, in_piece ? vb : vb_n,
                                  in_piece ? t0 + 16 : pn.t_begin,
                                  in_piece ? pc.t_end : (has_next ? pn.t_end : 0), blk_b, lane,
                                  in_piece ? cached : cached_n, rb);
                mfma_tile<KV, D, R>(p, q, t0, pc.t_end, blk_a >= 0, lane, lds, ra, st);
                ra = rb;
                blk_a = blk_b;
            }

            if (fold.base >= 0) {
                if (R != 1) mfma_fold_load<D, R>(p, pc, lane, fold);
                mfma_fold_apply<D, R>(fold, lane, st);
            }
            if (pc.whole) {
                mfma_write_rows<KV, D, R, HS>(p, pc, lane, st);
            } else if constexpr (FIX == 1) {
                if (has_next) {
                    // a cut piece with more pieces after it: the wavefront's
                    // first piece, a continuation that ends its segment here.
                    // It goes to the wavefront's slot; the first wavefront's
                    // (whose left neighbour is in another workgroup) is
                    // written as a partial after the range, so that its
                    // stores do not sit in front of the next piece's loads.
                    fix_store<D>(sm.sw.fix[wave], lane, st[0]);
                    if (lane == 0) sm.sw.fix[wave].ends = 1;
                    if (wave == 0) {
                        pc_first = pc;
                        first_saved = true;
                    }
                } else {
                    have_last = true;  // the sweep below decides where it goes
                }
            } else if constexpr (FIX == 2) {
                if (has_next)
                    mfma_write_partial<D, R, HS>(p, pc, lane, st);
                else
                    have_last = true;
            } else {
                mfma_write_partial<D, R, HS>(p, pc, lane, st);
            }
            if (!has_next) break;
            pc = pn;
            ids = ids_n;
            fold_base = fold_base_n;
            mfma_load_q<D, R, SRC>(p, pc, lane, q, cp);
        }
        XHIP_WAVE_STAMP(p, wave, 1);
    }
#if XHIP_TRACING
    XHIP_WAVE_PUT(p, wave, 2, (unsigned long long)n_tiles | ((unsigned long long)n_pieces << 32));
#endif

    if constexpr (FIX == 2) {
        // As below, with the one relay slot.
        __syncthreads();
        for (int i = NW - 1; i >= 0; i--) {
            if (wave == i && have_last) {
                const bool cut_start = pc.t_begin > 0;
                bool ends = pc.t_end >= pc.L;
                if (!ends && i < NW - 1) {
                    if (sm.sw.relay.relayed[i + 1]) {
#pragma unroll
                        for (int b = 0; b < R; b++) {
                            const float mo = sm.sw.relay.m[b][lane];
                            const float M = fmaxf(st[b].m, mo);
                            const float Ms = (M == -INFINITY) ? 0.0f : M;
                            const float a = fast_exp2(st[b].m - Ms), wt = fast_exp2(mo - Ms);
                            st[b].l = st[b].l * a + sm.sw.relay.l[b][lane] * wt;
#pragma unroll
                            for (int n = 0; n < G::kDimBlocks; n++)
                                st[b].o[n] = st[b].o[n] * a + sm.sw.relay.o[b][n][lane] * wt;
                            st[b].m = M;
                        }
                        ends = sm.sw.relay.ends[i + 1] != 0;
                    } else {
                        // the neighbour's first piece, followed by more
                        // pieces, was written as a partial in its slot 0;
                        // it ends the segment in that range
                        absorb_partial<D, R, HS>(p, (w + 1) * 2, pc.ht, lane, st);
                        ends = true;
                    }
                }
                if (cut_start && i > 0) {
#pragma unroll
                    for (int b = 0; b < R; b++) {
#pragma unroll
                        for (int n = 0; n < G::kDimBlocks; n++) sm.sw.relay.o[b][n][lane] = st[b].o[n];
                        sm.sw.relay.m[b][lane] = st[b].m;
                        sm.sw.relay.l[b][lane] = st[b].l;
                    }
                    if (lane == 0) {
                        sm.sw.relay.relayed[i] = 1;
                        sm.sw.relay.ends[i] = ends ? 1 : 0;
                    }
                } else if (!cut_start && ends) {
                    mfma_write_rows<KV, D, R, HS>(p, pc, lane, st);
                } else {
                    mfma_write_partial<D, R, HS>(p, pc, lane, st);
                }
            }
            __syncthreads();
        }
    }
    if constexpr (FIX == 1) {
        // The wavefronts of a workgroup hold consecutive ranges.  First, a
        // wavefront whose last piece continues its left neighbour's (cut at
        // the start; its range is that one piece) puts the state in its slot,
        // as a cut first piece followed by more pieces already did in the
        // loop.  Then, after one barrier, the leftmost holder of each
        // segment in the workgroup absorbs the slots of the neighbours its
        // piece continues into, left to right, and writes the segment:
        // finished rows when it lay in the workgroup, else one partial.
        const bool cut_start = have_last && pc.t_begin > 0;
        if (have_last && cut_start && wave > 0) {
            fix_store<D>(sm.sw.fix[wave], lane, st[0]);
            if (lane == 0) sm.sw.fix[wave].ends = pc.t_end >= pc.L ? 1 : 0;
        }
        __syncthreads();
        if (first_saved) {
            MfmaState<D> sf[R];
            fix_load<D>(sm.sw.fix[0], lane, sf[0]);
            mfma_write_partial<D, R, HS>(p, pc_first, lane, sf);
        }
        if (have_last && !(cut_start && wave > 0)) {
            bool ends = pc.t_end >= pc.L;
            for (int j = wave + 1; !ends && j < NW; j++) {
                fix_absorb<D>(sm.sw.fix[j], lane, st[0]);
                ends = sm.sw.fix[j].ends != 0;
            }
            if (!cut_start && ends)
                mfma_write_rows<KV, D, R, HS>(p, pc, lane, st);
            else
                mfma_write_partial<D, R, HS>(p, pc, lane, st);
        }
    }
}


// Two wavefronts per SIMD (the plan's occupancy) up to head_size 128: at
// most 256 registers each.  Larger heads need more and run one per SIMD.
template <int KV, int D, int R>
__global__ __launch_bounds__(64 * kMfmaWavesPerGroup, D <= 128 ? 2 : 1) void paged_decode_partition_mfma_kernel(
    const DecodeParams p, const int *__restrict__ lens, const int *__restrict__ tables) {
    // lens / tables are p.seq_lens / p.block_tables again: as restrict
    // kernel arguments their wavefront-uniform reads become scalar loads,
    // which do not wait behind the K/V loads in flight.
    extern __shared__ int pre[];  // num_seqs + 1 split-unit prefixes
    __shared__ MfmaLds<D, R> sm;
    XHIP_WG_BEGIN(p);
    batch_prefix<16, kMfmaWavesPerGroup>(p, pre);
    XHIP_WG_STAMP(p, 1);
    const int lb = logical_block(p, pre[p.num_seqs]);
    XHIP_WG_PUT(p, 3, lb);
    mfma_partition_body<KV, D, R>(p, lens, tables, pre, lb, p.num_waves, sm);
    XHIP_WG_FLUSH(p);
}

}  // namespace xhip
