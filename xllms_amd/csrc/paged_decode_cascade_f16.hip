// Instantiations of the cascade attention kernels for f16 K/V, Q and O.
#include "paged_decode_cascade_attn.h"

namespace xhip {

int cascade_attn_occupancy_f16(int head_size, int rs, size_t lds_bytes) {
    return cascade_occupancy_dtype<KV_F16>(head_size, rs, lds_bytes);
}

hipError_t launch_cascade_attn_f16(const DecodeParams &pp, const DecodeParams &ps,
                                   const int *p_row, int rows, int head_size, int rs,
                                   hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop) {
    return launch_cascade_attn_dtype<KV_F16>(pp, ps, p_row, rows, head_size, rs, stream,
                                             ev_start, ev_stop);
}

}  // namespace xhip
