// Shared body of the per-dtype launch units: head_size x head_tile dispatch.
#pragma once

#include "paged_decode_kernels.h"
#include "paged_decode_launch.h"

namespace xhip {

template <int KV, int D, int GT> static const void *partition_fn() {
    return reinterpret_cast<const void *>(&paged_decode_partition_kernel<KV, D, GT>);
}

template <int KV, int D>
static const void *partition_fn_for(int head_tile) {
    switch (head_tile) {
    case 1: return partition_fn<KV, D, 1>();
    case 2: return partition_fn<KV, D, 2>();
    case 4: return partition_fn<KV, D, 4>();
    case 8: return partition_fn<KV, D, 8>();
    default: return nullptr;
    }
}

template <int KV, int D, int GT>
static hipError_t launch_tile(const DecodeParams &p, hipStream_t st, hipEvent_t after_partition) {
    const unsigned grid = (unsigned)(p.num_waves / kWavesPerGroup);
    const size_t lds = (size_t)(p.num_seqs + 1) * sizeof(int);
    paged_decode_partition_kernel<KV, D, GT><<<grid, 64 * kWavesPerGroup, lds, st>>>(p);
    if (after_partition) {
        const hipError_t e = hipEventRecord(after_partition, st);
        if (e != hipSuccess) return e;
    }
    const unsigned segs = (unsigned)(p.num_seqs * p.num_kv_heads * p.head_tiles);
    paged_decode_merge_kernel<KV, D, GT><<<segs, 256, 0, st>>>(p);
    return hipGetLastError();
}

template <int KV, int D>
static hipError_t launch_for_head_size(const DecodeParams &p, int head_tile, hipStream_t st,
                                       hipEvent_t after_partition) {
    switch (head_tile) {
    case 1: return launch_tile<KV, D, 1>(p, st, after_partition);
    case 2: return launch_tile<KV, D, 2>(p, st, after_partition);
    case 4: return launch_tile<KV, D, 4>(p, st, after_partition);
    case 8: return launch_tile<KV, D, 8>(p, st, after_partition);
    default: return hipErrorInvalidValue;
    }
}

#define XHIP_FOR_HEAD_SIZES(X) X(32) X(64) X(80) X(96) X(112) X(128) X(192) X(256)

template <int KV>
static const void *partition_fn_dtype(int head_size, int head_tile) {
    switch (head_size) {
#define XHIP_CASE(d) case d: return partition_fn_for<KV, d>(head_tile);
        XHIP_FOR_HEAD_SIZES(XHIP_CASE)
#undef XHIP_CASE
    default: return nullptr;
    }
}

template <int KV>
static int occupancy_for_dtype(int head_size, int head_tile, size_t lds_bytes) {
    const void *fn = partition_fn_dtype<KV>(head_size, head_tile);
    if (!fn) return 0;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, 64 * kWavesPerGroup,
                                                     lds_bytes) != hipSuccess)
        return 0;
    return blocks;
}

template <int KV>
static hipError_t launch_for_dtype(const DecodeParams &p, int head_size, int head_tile,
                                   hipStream_t st, hipEvent_t after_partition) {
    switch (head_size) {
#define XHIP_CASE(d) case d: return launch_for_head_size<KV, d>(p, head_tile, st, after_partition);
        XHIP_FOR_HEAD_SIZES(XHIP_CASE)
#undef XHIP_CASE
    default: return hipErrorInvalidValue;
    }
}

}  // namespace xhip
