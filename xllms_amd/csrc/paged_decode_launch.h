// Per-dtype launch entry points of the paged-decode kernels (one translation
// unit per dtype so the instantiations compile in parallel).
#pragma once

#include <hip/hip_runtime_api.h>

#include "paged_decode_params.h"

namespace xhip {

// Resident workgroups per CU of the partition kernel for this
// (head_size, head_tile, tile path) with `lds_bytes` of dynamic LDS; 0 when
// there is no such instantiation.  A workgroup is kWavesPerGroup wavefronts
// on the VALU path and kMfmaWavesPerGroup on the MFMA path.  mfma selects the
// MFMA tile path (16-bit types, head_size % 32 == 0, head_tile 16).
int partition_occupancy_f16(int head_size, int head_tile, bool mfma, size_t lds_bytes);
int partition_occupancy_bf16(int head_size, int head_tile, bool mfma, size_t lds_bytes);
int partition_occupancy_f32(int head_size, int head_tile, bool mfma, size_t lds_bytes);

// Launches the partition kernel on num_waves / (wavefronts per workgroup)
// workgroups, then the merge kernel over every (sequence, kv head, head
// tile).  Non-null `ev_start` / `ev_stop` events are stamped with the
// partition kernel's start and end (hipExtLaunchKernel).  Returns
// hipErrorInvalidValue for a head_size / head_tile with no instantiation,
// else the launch status.
hipError_t launch_decode_f16(const DecodeParams &p, int head_size, int head_tile, bool mfma,
                             hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop);
hipError_t launch_decode_bf16(const DecodeParams &p, int head_size, int head_tile, bool mfma,
                              hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop);
hipError_t launch_decode_f32(const DecodeParams &p, int head_size, int head_tile, bool mfma,
                             hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop);

}  // namespace xhip
