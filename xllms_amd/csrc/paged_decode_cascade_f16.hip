// Instantiations of the cascade attention kernels for f16 K/V, Q and O.
#include "paged_decode_cascade_attn.h"

namespace xhip {

size_t inplan_lds_bytes(int num_seqs, int v_max, int num_groups) {
    return (size_t)inplan_lds_ints(num_seqs, v_max, num_groups) * sizeof(int);
}

int cascade_attn_occupancy_f16(int head_size, int rs, bool inplan, size_t lds_bytes) {
    return cascade_occupancy_dtype<KV_F16>(head_size, rs, inplan, lds_bytes);
}

hipError_t launch_cascade_attn_f16(const DecodeParams &pp, const DecodeParams &ps,
                                   const int *p_row, int rows, int head_size, int rs,
                                   const CascadeInPlan *ip, hipStream_t stream, hipEvent_t ev_start,
                                   hipEvent_t ev_stop) {
    return launch_cascade_attn_dtype<KV_F16>(pp, ps, p_row, rows, head_size, rs, ip, stream,
                                           ev_start, ev_stop);
}

}  // namespace xhip
