// Per-dtype launch entry points of the paged-decode kernels (one translation
// unit per dtype so the instantiations compile in parallel).
#pragma once

#include <hip/hip_runtime_api.h>

#include "paged_decode_params.h"

namespace xhip {

// Launches the partition kernel on `grid` workgroups and, when `reduce`, the
// partition-merge kernel over (num_heads, num_seqs).  head_tile is the query
// heads per wavefront (1, 2, 4 or 8).  Returns hipErrorInvalidValue for a
// head_size / head_tile with no instantiation, else the launch status.
hipError_t launch_decode_f16(const DecodeParams &p, int head_size, int head_tile, unsigned grid,
                             bool reduce, hipStream_t stream);
hipError_t launch_decode_bf16(const DecodeParams &p, int head_size, int head_tile, unsigned grid,
                              bool reduce, hipStream_t stream);
hipError_t launch_decode_f32(const DecodeParams &p, int head_size, int head_tile, unsigned grid,
                             bool reduce, hipStream_t stream);

}  // namespace xhip
