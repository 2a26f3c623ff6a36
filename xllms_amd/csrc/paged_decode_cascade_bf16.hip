// Instantiations of the cascade attention kernels for bf16 K/V, Q and O.
#include "paged_decode_cascade_attn.h"

namespace xhip {

int cascade_attn_occupancy_bf16(int head_size, int rs, bool inplan, size_t lds_bytes) {
    return cascade_occupancy_dtype<KV_BF16>(head_size, rs, inplan, lds_bytes);
}

hipError_t launch_cascade_attn_bf16(const DecodeParams &pp, const DecodeParams &ps,
                                    const int *p_row, int rows, int head_size, int rs,
                                    const CascadeInPlan *ip, hipStream_t stream, hipEvent_t ev_start,
                                    hipEvent_t ev_stop) {
    return launch_cascade_attn_dtype<KV_BF16>(pp, ps, p_row, rows, head_size, rs, ip, stream,
                                           ev_start, ev_stop);
}

}  // namespace xhip
