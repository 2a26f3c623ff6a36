// Gated and element-wise activations of the MLP (the reference's
// operators/activation_kernels.cu:52-134 behind include/operator_api.h:
// 122-150), written for gfx950.
//
// Semantics, per element, as the reference computes them (its device
// functions silu / gelu / gelu_tanh, activation_kernels.cu:24-48):
//   silu(x)      = x / (1 + exp(-x))                          in fp32
//   gelu(x)      = (x * 0.5) * (1 + erf(x * sqrt(1/2)))         in fp32
//   gelu_tanh(x) = (0.5 * x) * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))
// the activation is rounded to the tensor's element type, and a gated op
// multiplies it by the other half of the row in that element type: for 16-bit
// types the fp32 product of two 16-bit values is exact, so rounding it once
// gives the correctly rounded 16-bit product, as the reference's half
// operator* does.  Gated rows are [gate (d) | up (d)]; silu_and_mul applies
// the activation to the gate, mul_and_silu to the up half.
//
// HBM-bound: a gated op reads 2d and writes d elements per row, an
// element-wise op reads d and writes d.  The vector kernel gives each lane
// whole 16-byte output chunks (8 fp16/bf16 or 4 fp32 elements) with the gate
// and up chunks it needs loaded first, kUnroll chunks per lane per pass so
// several 16-byte loads are in flight per lane; loads and stores are
// nontemporal (streamed once).  Output chunk i lies in row t = i / (d*e/16),
// and the gate chunk is at i + t*(d*e/16) of the input (the up chunk one row
// half later), so a single division per chunk (a multiply-high) is the only
// index work.  The element kernel covers every other shape (any d, any
// alignment) one element per lane.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "activation.h"
#include "paged_decode_params.h"

namespace xhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kBlock = 256;
constexpr int kUnroll = 4;

template <int OP> __device__ __forceinline__ float activation(float x) {
    if constexpr (OP == ACT_SILU_AND_MUL || OP == ACT_MUL_AND_SILU || OP == ACT_SILU) {
        return x / (1.0f + expf(-x));
    } else if constexpr (OP == ACT_GELU_AND_MUL || OP == ACT_GELU) {
        constexpr float kInvSqrt2 = 0.70710678118654752440f;
        return x * 0.5f * (1.0f + erff(x * kInvSqrt2));
    } else {
        constexpr float kSqrt2OverPi = 0.79788456080286535588f;
        constexpr float kCubic = 0.044715f;
        const float cube = x * x * x;
        const float inner = kSqrt2OverPi * fmaf(kCubic, cube, x);
        return 0.5f * x * (1.0f + tanhf(inner));
    }
}

// fp32 -> element type and back (round to nearest even; NaN stays NaN).
__device__ __forceinline__ uint32_t bf16_bits(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

template <int DT> __device__ __forceinline__ float round_to(float x) {
    if constexpr (DT == KV_F16) return (float)(_Float16)x;
    else if constexpr (DT == KV_BF16) return __builtin_bit_cast(float, bf16_bits(x) << 16);
    else return x;
}

// One output element from its input(s), fp32 in, fp32 out (already rounded
// to the element type).
template <int OP, int DT> __device__ __forceinline__ float apply(float g, float u) {
    if constexpr (OP == ACT_MUL_AND_SILU) return round_to<DT>(g * round_to<DT>(activation<OP>(u)));
    else if constexpr (act_is_gated(OP)) return round_to<DT>(round_to<DT>(activation<OP>(g)) * u);
    else return round_to<DT>(activation<OP>(g));
}

// 16-byte chunk <-> fp32 values.
template <int DT> struct Chunk {
    static constexpr int kVec = DT == KV_F32 ? 4 : 8;
};

template <int DT> __device__ __forceinline__ void unpack(const u32x4 &c, float (&f)[Chunk<DT>::kVec]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w = c[i];
        if constexpr (DT == KV_F16) {
            const f16x2 h = __builtin_bit_cast(f16x2, w);
            f[2 * i] = (float)h.x;
            f[2 * i + 1] = (float)h.y;
        } else if constexpr (DT == KV_BF16) {
            f[2 * i] = __builtin_bit_cast(float, w << 16);
            f[2 * i + 1] = __builtin_bit_cast(float, w & 0xFFFF0000u);
        } else {
            f[i] = __builtin_bit_cast(float, w);
        }
    }
}

template <int DT> __device__ __forceinline__ u32x4 pack(const float (&f)[Chunk<DT>::kVec]) {
    u32x4 c;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if constexpr (DT == KV_F16) {
            f16x2 h;
            h.x = (_Float16)f[2 * i];
            h.y = (_Float16)f[2 * i + 1];
            c[i] = __builtin_bit_cast(uint32_t, h);
        } else if constexpr (DT == KV_BF16) {
            // values are already bf16-exact: truncation keeps them
            c[i] = (__builtin_bit_cast(uint32_t, f[2 * i]) >> 16) |
                   (__builtin_bit_cast(uint32_t, f[2 * i + 1]) & 0xFFFF0000u);
        } else {
            c[i] = __builtin_bit_cast(uint32_t, f[i]);
        }
    }
    return c;
}

template <int OP, int DT>
__global__ __launch_bounds__(kBlock) void activation_vec_kernel(const ActivationParams p) {
    constexpr int V = Chunk<DT>::kVec;
    const u32x4 *in = (const u32x4 *)p.input;
    u32x4 *out = (u32x4 *)p.out;
    const uint32_t n = p.chunks;
    const uint32_t rc = p.row_chunks.d;
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t base = blockIdx.x * kBlock + threadIdx.x; base < n;
         base += stride * kUnroll) {
        u32x4 g[kUnroll], u[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const uint32_t i = base + k * stride;
            if (i < n) {
                if constexpr (act_is_gated(OP)) {
                    const uint32_t t = div_by(i, p.row_chunks);
                    const size_t gi = (size_t)i + (size_t)t * rc;
                    g[k] = __builtin_nontemporal_load(in + gi);
                    u[k] = __builtin_nontemporal_load(in + gi + rc);
                } else {
                    g[k] = __builtin_nontemporal_load(in + i);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const uint32_t i = base + k * stride;
            if (i < n) {
                float gf[V], uf[V], of[V];
                unpack<DT>(g[k], gf);
                if constexpr (act_is_gated(OP)) unpack<DT>(u[k], uf);
#pragma unroll
                for (int e = 0; e < V; e++)
                    of[e] = apply<OP, DT>(gf[e], act_is_gated(OP) ? uf[e] : 0.0f);
                __builtin_nontemporal_store(pack<DT>(of), out + i);
            }
        }
    }
}

template <int DT> __device__ __forceinline__ float load_elem(const void *base, size_t idx) {
    if constexpr (DT == KV_F16) return (float)((const _Float16 *)base)[idx];
    else if constexpr (DT == KV_BF16)
        return __builtin_bit_cast(float, (uint32_t)((const uint16_t *)base)[idx] << 16);
    else return ((const float *)base)[idx];
}

template <int DT> __device__ __forceinline__ void store_elem(void *base, size_t idx, float x) {
    if constexpr (DT == KV_F16) ((_Float16 *)base)[idx] = (_Float16)x;
    else if constexpr (DT == KV_BF16) ((uint16_t *)base)[idx] = (uint16_t)(__builtin_bit_cast(uint32_t, x) >> 16);
    else ((float *)base)[idx] = x;
}

template <int OP, int DT>
__global__ __launch_bounds__(kBlock) void activation_elem_kernel(const ActivationParams p) {
    const long long n = p.num_tokens * p.d;
    const long long stride = (long long)gridDim.x * kBlock;
    for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float g, u = 0.0f;
        if constexpr (act_is_gated(OP)) {
            const long long t = i / p.d;
            const long long gi = i + t * p.d;
            g = load_elem<DT>(p.input, (size_t)gi);
            u = load_elem<DT>(p.input, (size_t)(gi + p.d));
        } else {
            g = load_elem<DT>(p.input, (size_t)i);
        }
        store_elem<DT>(p.out, (size_t)i, apply<OP, DT>(g, u));
    }
}

template <int OP, int DT>
hipError_t launch_typed(const ActivationParams &p, bool vector_path, int num_cus,
                        hipStream_t stream) {
    // One resident round: 8 workgroups of 4 waves per CU (32 waves per CU).
    const long long cap = (long long)(num_cus > 0 ? num_cus : 256) * 8;
    if (vector_path) {
        long long blocks = ((long long)p.chunks + kBlock * kUnroll - 1) / (kBlock * kUnroll);
        if (blocks > cap) blocks = cap;
        if (blocks < 1) blocks = 1;
        activation_vec_kernel<OP, DT><<<(unsigned)blocks, kBlock, 0, stream>>>(p);
    } else {
        long long blocks = (p.num_tokens * p.d + kBlock - 1) / kBlock;
        if (blocks > cap) blocks = cap;
        if (blocks < 1) blocks = 1;
        activation_elem_kernel<OP, DT><<<(unsigned)blocks, kBlock, 0, stream>>>(p);
    }
    return hipGetLastError();
}

template <int OP>
hipError_t launch_op(const ActivationParams &p, bool vector_path, int num_cus, hipStream_t stream) {
    switch (p.dtype) {
        case KV_F16: return launch_typed<OP, KV_F16>(p, vector_path, num_cus, stream);
        case KV_BF16: return launch_typed<OP, KV_BF16>(p, vector_path, num_cus, stream);
        case KV_F32: return launch_typed<OP, KV_F32>(p, vector_path, num_cus, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_activation(const ActivationParams &p, bool vector_path, int num_cus,
                             hipStream_t stream) {
    switch (p.op) {
        case ACT_SILU_AND_MUL: return launch_op<ACT_SILU_AND_MUL>(p, vector_path, num_cus, stream);
        case ACT_MUL_AND_SILU: return launch_op<ACT_MUL_AND_SILU>(p, vector_path, num_cus, stream);
        case ACT_GELU_AND_MUL: return launch_op<ACT_GELU_AND_MUL>(p, vector_path, num_cus, stream);
        case ACT_GELU_TANH_AND_MUL:
            return launch_op<ACT_GELU_TANH_AND_MUL>(p, vector_path, num_cus, stream);
        case ACT_GELU: return launch_op<ACT_GELU>(p, vector_path, num_cus, stream);
        case ACT_SILU: return launch_op<ACT_SILU>(p, vector_path, num_cus, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace xhip
