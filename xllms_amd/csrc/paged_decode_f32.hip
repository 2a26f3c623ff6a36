// Instantiations of the paged-decode kernels for f32 K/V, Q and O.
#include "paged_decode_dispatch.h"

namespace xhip {

int partition_occupancy_f32(int head_size, int head_tile, bool mfma, size_t lds_bytes) {
    return occupancy_for_dtype<KV_F32>(head_size, head_tile, mfma, lds_bytes);
}

hipError_t launch_decode_f32(const DecodeParams &p, int head_size, int head_tile, bool mfma,
                             hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop) {
    return launch_for_dtype<KV_F32>(p, head_size, head_tile, mfma, stream, ev_start, ev_stop);
}

}  // namespace xhip
