// Fixed device scratch of nxt_paged_attention_noalloc (paged_decode_scratch.hip).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>

namespace xhip {

// Size of the per-device scratch array, 66 MiB.  Every automatic plan fits
// on a 256-CU MI355X: the MFMA path's 2048 wavefronts need at most 64 MiB of
// split-K partials (2 slots x 16 heads x 256 dims, or 32 heads x 128 dims,
// x 4 B each) plus 1 MiB of (m, l) pairs and the unit prefix; the VALU
// path's head tiles of up to 8 heads run at most 2048 wavefronts for 8
// heads (32 MiB at 256 dims) and 4096 for 4 or fewer.  A plan that needs
// more (an explicit partition_tokens, or a larger device) is refused.
constexpr size_t kNoAllocScratchBytes = (size_t)66 << 20;

// This device's scratch address (looked up once per device, with it
// current) and size.  Allocates nothing.
hipError_t noalloc_scratch(int device, void **ptr, size_t *bytes);

}  // namespace xhip
