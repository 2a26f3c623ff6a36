// Launch parameters of the gated / element-wise activation kernels
// (activation.hip), the MLP ops of the reference's operator API
// (include/operator_api.h:122-150, operators/activation_kernels.cu:52-239).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "fast_div.h"

namespace xhip {

// Same values as NxtActivationOp in include/xllm_hip_operator_api.h.
enum ActOp : int {
    ACT_SILU_AND_MUL = 1,       // out = silu(gate) * up
    ACT_MUL_AND_SILU = 2,       // out = gate * silu(up)
    ACT_GELU_AND_MUL = 3,       // out = gelu(gate) * up       (erf form)
    ACT_GELU_TANH_AND_MUL = 4,  // out = gelu_tanh(gate) * up  (tanh form)
    ACT_GELU = 5,               // out = gelu(x)
    ACT_SILU = 6,               // out = silu(x)
};

// constexpr functions are callable from host and device code alike.
constexpr bool act_is_gated(int op) { return op >= ACT_SILU_AND_MUL && op <= ACT_GELU_TANH_AND_MUL; }

struct ActivationParams {
    void *out;              // [num_tokens][d]
    const void *input;      // [num_tokens][2d] (gated: gate | up) or [num_tokens][d]
    long long num_tokens;
    int d;
    int dtype;              // KV_F16 / KV_BF16 / KV_F32 (paged_decode_params.h codes)
    int op;                 // ActOp
    // Vector path (d * elem_bytes a multiple of 16, tensors 16-byte aligned):
    uint32_t chunks;        // 16-byte output chunks of this launch, < 2^32
    DivMagic row_chunks;    // division by d * elem_bytes / 16
};

// Enqueues one activation over params.num_tokens rows.  `vector_path` selects
// the 16-byte chunk kernel (its preconditions checked by the caller, with
// params.chunks / row_chunks filled in); otherwise the element kernel runs.
// num_cus sizes the grid.
hipError_t launch_activation(const ActivationParams &p, bool vector_path, int num_cus,
                             hipStream_t stream);

}  // namespace xhip
