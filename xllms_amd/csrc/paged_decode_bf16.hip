// Instantiations of the paged-decode kernels for bf16 K/V, Q and O.
#include "paged_decode_dispatch.h"

namespace xhip {

hipError_t launch_decode_bf16(const DecodeParams &p, int head_size, int head_tile, unsigned grid,
                             bool reduce, hipStream_t stream) {
    return launch_for_dtype<KV_BF16>(p, head_size, head_tile, grid, reduce, stream);
}

}  // namespace xhip
