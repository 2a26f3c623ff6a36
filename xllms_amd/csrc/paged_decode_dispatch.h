// Shared body of the per-dtype launch units: (tile path, head_size, head_tile)
// dispatch.  The MFMA path exists for the 16-bit types and head sizes that are
// multiples of 32; the VALU path covers every supported shape.
#pragma once

#include <hip/hip_ext.h>

#include "paged_decode_kernels.h"
#include "paged_decode_launch.h"
#include "paged_decode_mfma.h"

namespace xhip {

template <int KV, int D>
static const void *valu_fn(int head_tile) {
    switch (head_tile) {
    case 1: return reinterpret_cast<const void *>(&paged_decode_partition_kernel<KV, D, 1>);
    case 2: return reinterpret_cast<const void *>(&paged_decode_partition_kernel<KV, D, 2>);
    case 4: return reinterpret_cast<const void *>(&paged_decode_partition_kernel<KV, D, 4>);
    case 8: return reinterpret_cast<const void *>(&paged_decode_partition_kernel<KV, D, 8>);
    default: return nullptr;
    }
}

template <int KV, int D> constexpr bool has_mfma() {
    return KV != KV_F32 && D % 32 == 0;
}

// Two row blocks per wavefront (head tile 32) fit the register file at two
// wavefronts per SIMD up to head_size 128.
template <int KV, int D> constexpr bool has_mfma_wide() {
    return has_mfma<KV, D>() && D <= kMfmaWideMaxHeadSize;
}

template <int KV, int D>
static const void *partition_fn(int head_tile, bool mfma) {
    if (mfma) {
        if constexpr (has_mfma<KV, D>()) {
            if (head_tile == kMfmaHeads)
                return reinterpret_cast<const void *>(&paged_decode_partition_mfma_kernel<KV, D, 1>);
            if constexpr (has_mfma_wide<KV, D>())
                if (head_tile == 2 * kMfmaHeads)
                    return reinterpret_cast<const void *>(
                        &paged_decode_partition_mfma_kernel<KV, D, 2>);
        }
        return nullptr;
    }
    return valu_fn<KV, D>(head_tile);
}

// A partition kernel launch.  With trace events it goes through
// hipExtLaunchKernelGGL, which stamps them from the kernel's own dispatch
// (its start and its end), not from event packets queued around it, whose
// latency made the kernel read 2-6 us longer than rocprof's trace.
template <typename F, typename... Args>
static hipError_t launch_partition(F kernel, unsigned grid, unsigned block, size_t lds,
                                   hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop,
                                   Args... args) {
    if (ev_start || ev_stop)
        hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(block), (std::uint32_t)lds, st, ev_start,
                              ev_stop, 0u, args...);
    else
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), lds, st, args...);
    return hipGetLastError();
}

template <int KV, int D, int GT, int TT>
static hipError_t launch_merge(const DecodeParams &p, hipStream_t st) {
    const unsigned segs = (unsigned)(p.num_seqs * p.num_kv_heads * p.head_tiles);
    const int heads = p.group < GT ? p.group : GT;
    if (p.merge_per_segment) {
        // one thread per float4 column of the segment (heads * D/4), the
        // count rounded up to a power of two from 64 to 1024; the wider
        // instantiations exist only where a segment can have that many
        // columns (fewer than 64 columns: 64 threads split the partials)
        constexpr int kMaxCols = GT * (D / 4);
        constexpr int kNt128 = kMaxCols > 64 ? 128 : 64;
        constexpr int kNt256 = kMaxCols > 128 ? 256 : 64;
        constexpr int kNt512 = kMaxCols > 256 ? 512 : 64;
        constexpr int kNt1024 = kMaxCols > 512 ? 1024 : 64;
        const int cols = heads * (D / 4);
        if (cols <= 64)
            paged_decode_merge_segment_kernel<KV, D, GT, TT, 64><<<segs, 64, 0, st>>>(p);
        else if (cols <= 128)
            paged_decode_merge_segment_kernel<KV, D, GT, TT, kNt128><<<segs, kNt128, 0, st>>>(p);
        else if (cols <= 256)
            paged_decode_merge_segment_kernel<KV, D, GT, TT, kNt256><<<segs, kNt256, 0, st>>>(p);
        else if (cols <= 512)
            paged_decode_merge_segment_kernel<KV, D, GT, TT, kNt512><<<segs, kNt512, 0, st>>>(p);
        else
            paged_decode_merge_segment_kernel<KV, D, GT, TT, kNt1024><<<segs, kNt1024, 0, st>>>(p);
        return hipGetLastError();
    }
    const unsigned chunks = (unsigned)((heads * (D / 4) + kMergeCols - 1) / kMergeCols);
    paged_decode_merge_kernel<KV, D, GT, TT>
        <<<dim3(segs, chunks), kMergeCols * kMergeSplit, 0, st>>>(p);
    return hipGetLastError();
}

template <int KV, int D>
static hipError_t launch_for_head_size(const DecodeParams &p, int head_tile, bool mfma,
                                       hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
    constexpr int TT = Geometry<KV, D>::kTileTokens;
    const unsigned grid = (unsigned)(p.num_waves / kWavesPerGroup);
    const size_t lds = (size_t)(p.num_seqs + 1) * sizeof(int);
    if (mfma) {
        if constexpr (has_mfma<KV, D>()) {
            const unsigned mgrid = (unsigned)(p.num_waves / kMfmaWavesPerGroup);
            if (head_tile == kMfmaHeads) {
                const hipError_t e = launch_partition(
                    paged_decode_partition_mfma_kernel<KV, D, 1>, mgrid, 64 * kMfmaWavesPerGroup,
                    lds, st, ev_start, ev_stop, p, p.seq_lens, p.block_tables);
                if (e != hipSuccess) return e;
                return launch_merge<KV, D, kMfmaHeads, MfmaGeometry<D>::kTile>(p, st);
            }
            if constexpr (has_mfma_wide<KV, D>()) {
                if (head_tile == 2 * kMfmaHeads) {
                    const hipError_t e = launch_partition(
                        paged_decode_partition_mfma_kernel<KV, D, 2>, mgrid,
                        64 * kMfmaWavesPerGroup, lds, st, ev_start, ev_stop, p, p.seq_lens,
                        p.block_tables);
                    if (e != hipSuccess) return e;
                    return launch_merge<KV, D, 2 * kMfmaHeads, MfmaGeometry<D>::kTile>(p, st);
                }
            }
        }
        return hipErrorInvalidValue;
    }
    if (p.segment_launch) {
        // segment_split workgroups per segment; above one, a merge
        const unsigned segs = (unsigned)(p.num_seqs * p.num_kv_heads * p.head_tiles);
        const unsigned sgrid = segs * (unsigned)p.segment_split;
        hipError_t e = hipErrorInvalidValue;
        if (head_tile == 1)
            e = launch_partition(paged_decode_segment_kernel<KV, D, 1>, sgrid, 64 * kSegWaves, 0,
                                 st, ev_start, ev_stop, p);
        else if (head_tile == 2)
            e = launch_partition(paged_decode_segment_kernel<KV, D, 2>, sgrid, 64 * kSegWaves, 0,
                                 st, ev_start, ev_stop, p);
        if (e != hipSuccess || p.segment_split == 1) return e;
        if (head_tile == 1)
            paged_decode_segment_merge_kernel<KV, D, 1><<<segs, 256, 0, st>>>(p);
        else
            paged_decode_segment_merge_kernel<KV, D, 2><<<segs, 256, 0, st>>>(p);
        return hipGetLastError();
    }
    switch (head_tile) {
    case 1: {
        const hipError_t e = launch_partition(paged_decode_partition_kernel<KV, D, 1>, grid,
                                              64 * kWavesPerGroup, lds, st, ev_start, ev_stop, p);
        if (e != hipSuccess) return e;
        return launch_merge<KV, D, 1, TT>(p, st);
    }
    case 2: {
        const hipError_t e = launch_partition(paged_decode_partition_kernel<KV, D, 2>, grid,
                                              64 * kWavesPerGroup, lds, st, ev_start, ev_stop, p);
        if (e != hipSuccess) return e;
        return launch_merge<KV, D, 2, TT>(p, st);
    }
    case 4: {
        const hipError_t e = launch_partition(paged_decode_partition_kernel<KV, D, 4>, grid,
                                              64 * kWavesPerGroup, lds, st, ev_start, ev_stop, p);
        if (e != hipSuccess) return e;
        return launch_merge<KV, D, 4, TT>(p, st);
    }
    case 8: {
        const hipError_t e = launch_partition(paged_decode_partition_kernel<KV, D, 8>, grid,
                                              64 * kWavesPerGroup, lds, st, ev_start, ev_stop, p);
        if (e != hipSuccess) return e;
        return launch_merge<KV, D, 8, TT>(p, st);
    }
    default: return hipErrorInvalidValue;
    }
}

#define XHIP_FOR_HEAD_SIZES(X) X(32) X(64) X(80) X(96) X(112) X(128) X(192) X(256)

template <int KV>
static const void *partition_fn_dtype(int head_size, int head_tile, bool mfma) {
    switch (head_size) {
#define XHIP_CASE(d) case d: return partition_fn<KV, d>(head_tile, mfma);
        XHIP_FOR_HEAD_SIZES(XHIP_CASE)
#undef XHIP_CASE
    default: return nullptr;
    }
}

template <int KV>
static int occupancy_for_dtype(int head_size, int head_tile, bool mfma, size_t lds_bytes) {
    const void *fn = partition_fn_dtype<KV>(head_size, head_tile, mfma);
    if (!fn) return 0;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, fn, 64 * (mfma ? kMfmaWavesPerGroup : kWavesPerGroup), lds_bytes) !=
        hipSuccess)
        return 0;
    return blocks;
}

template <int KV>
static hipError_t launch_for_dtype(const DecodeParams &p, int head_size, int head_tile, bool mfma,
                                   hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
    switch (head_size) {
#define XHIP_CASE(d) \
    case d: return launch_for_head_size<KV, d>(p, head_tile, mfma, st, ev_start, ev_stop);
        XHIP_FOR_HEAD_SIZES(XHIP_CASE)
#undef XHIP_CASE
    default: return hipErrorInvalidValue;
    }
}

}  // namespace xhip
