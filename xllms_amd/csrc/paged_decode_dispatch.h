// Shared body of the per-dtype launch units: head_size x head_tile dispatch.
#pragma once

#include "paged_decode_kernels.h"
#include "paged_decode_launch.h"

namespace xhip {

template <int KV, int D>
static hipError_t launch_for_head_size(const DecodeParams &p, int head_tile, unsigned grid,
                                       bool reduce, hipStream_t st) {
    const dim3 block(64 * kWavesPerGroup);
    switch (head_tile) {
    case 1: paged_decode_partition_kernel<KV, D, 1><<<grid, block, 0, st>>>(p); break;
    case 2: paged_decode_partition_kernel<KV, D, 2><<<grid, block, 0, st>>>(p); break;
    case 4: paged_decode_partition_kernel<KV, D, 4><<<grid, block, 0, st>>>(p); break;
    case 8: paged_decode_partition_kernel<KV, D, 8><<<grid, block, 0, st>>>(p); break;
    default: return hipErrorInvalidValue;
    }
    if (reduce) {
        const dim3 rgrid(p.num_heads, p.num_seqs);
        paged_decode_reduce_kernel<KV, D><<<rgrid, 64, (size_t)p.max_parts * sizeof(float), st>>>(p);
    }
    return hipGetLastError();
}

template <int KV>
static hipError_t launch_for_dtype(const DecodeParams &p, int head_size, int head_tile,
                                   unsigned grid, bool reduce, hipStream_t st) {
    switch (head_size) {
    case 32: return launch_for_head_size<KV, 32>(p, head_tile, grid, reduce, st);
    case 64: return launch_for_head_size<KV, 64>(p, head_tile, grid, reduce, st);
    case 80: return launch_for_head_size<KV, 80>(p, head_tile, grid, reduce, st);
    case 96: return launch_for_head_size<KV, 96>(p, head_tile, grid, reduce, st);
    case 112: return launch_for_head_size<KV, 112>(p, head_tile, grid, reduce, st);
    case 128: return launch_for_head_size<KV, 128>(p, head_tile, grid, reduce, st);
    case 192: return launch_for_head_size<KV, 192>(p, head_tile, grid, reduce, st);
    case 256: return launch_for_head_size<KV, 256>(p, head_tile, grid, reduce, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace xhip
