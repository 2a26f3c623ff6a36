// Gated and element-wise activations of the MLP (the reference's
// operators/activation_kernels.cu:52-134 behind include/operator_api.h:
// 122-150), written for gfx950.
//
// Semantics, per element, as the reference computes them (its device
// functions silu / gelu / gelu_tanh, activation_kernels.cu:24-48):
//   silu(x)      = x / (1 + exp(-x))                          in fp32
//   gelu(x)      = (x * 0.5) * (1 + erf(x * sqrt(1/2)))         in fp32
//   gelu_tanh(x) = (0.5 * x) * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))
// (fp32 tensors evaluate exactly these expressions; fp16 / bf16 tensors use
// cheaper forms of the same functions, accurate to about 1e-7 relative,
// below the 16-bit rounding that follows), the activation is rounded to the
// tensor's element type, and a gated op
// multiplies it by the other half of the row in that element type: for 16-bit
// types the fp32 product of two 16-bit values is exact, so rounding it once
// gives the correctly rounded 16-bit product, as the reference's half
// operator* does.  Gated rows are [gate (d) | up (d)]; silu_and_mul applies
// the activation to the gate, mul_and_silu to the up half.
//
// HBM-bound: a gated op reads 2d and writes d elements per row, an
// element-wise op reads d and writes d.  The vector kernel gives each lane
// one 16-byte output chunk (8 fp16/bf16 or 4 fp32 elements) and the gate and
// up chunks it needs; loads and stores are nontemporal (streamed once).
// Output chunk i lies in row t = i / (d*e/16),
// and the gate chunk is at i + t*(d*e/16) of the input (the up chunk one row
// half later), so a single division per chunk (a multiply-high) is the only
// index work.  The element kernel covers every other shape (any d, any
// alignment) one element per lane.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "activation.h"
#include "paged_decode_params.h"

// No contraction: every product and sum rounds to fp32 as written (the one
// fused multiply-add of the formulas is an explicit fmaf).
#pragma clang fp contract(off)

namespace xhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kBlock = 256;     // element kernel
constexpr int kVecBlock = 64;   // vector kernel: one wavefront

// The reference's fp32 formulas, with the device library's expf / erff /
// tanhf and an IEEE divide.  Used for fp32 tensors (whose kernels are
// HBM-bound with room to spare) and for the rare 16-bit inputs the fast
// forms below cannot take.
template <int OP> __device__ __forceinline__ float activation_ref(float x) {
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

// Fast forms for fp16 / bf16 tensors, whose 16-bit rounding hides the last
// fp32 bits: about 10-20 VALU instructions an element instead of 30-40, so
// the kernels stay HBM-bound.  v_exp_f32 (2^x) and v_rcp_f32 are 1-ulp
// hardware approximations.
//   silu(x)      = x / (1 + 2^(-x log2 e))
//   gelu_tanh(x) = (x / 2) (1 + tanh u),  u = sqrt(2/pi) (x + 0.044715 x^3),
//                  with 1 + tanh u = 2 / (1 + 2^(-2 u log2 e)) exactly
//   gelu(x)      = (x / 2) (1 + erf(x / sqrt 2)), 1 + erf(z) = erfc(-z), with
//                  erfc(a) = t exp(-a^2 + P(t)), t = 1 / (1 + a/2), a >= 0, and
//                  2 - erfc(a) for positive x; P is a degree-9 Chebyshev fit
//                  (fit_erfc.py next to this file) with relative error
//                  1.2e-7 for every a >= 0.
// For negative x both keep the reference's fp32 cancellation in 1 + tanh u
// and 1 + erf z (which is 0 once tanh / erf round to -1) rather than the more
// accurate tiny values, so that, say, gelu(-9) * inf is NaN here as there.
// silu's rcp underflows below 2^-126 for x < -87.3 (|silu| < 1e-36), where
// fp16 rounds to zero anyway; bf16 can hold such values, so bf16 takes the
// reference formula there.
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kSiluFastMin = -87.0f;

template <int OP> __device__ __forceinline__ float activation_fast(float x) {
    if constexpr (OP == ACT_SILU_AND_MUL || OP == ACT_MUL_AND_SILU || OP == ACT_SILU) {
        return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -kLog2e));
    } else if constexpr (OP == ACT_GELU_AND_MUL || OP == ACT_GELU) {
        constexpr float kInvSqrt2 = 0.70710678118654752440f;
        const float a = fabsf(x * kInvSqrt2);
        const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, a, 1.0f));
        float p = 1.708930433e-01f;
        p = fmaf(p, t, -8.222485185e-01f);
        p = fmaf(p, t, 1.488708496e+00f);
        p = fmaf(p, t, -1.135414600e+00f);
        p = fmaf(p, t, 2.790049911e-01f);
        p = fmaf(p, t, -1.863418519e-01f);
        p = fmaf(p, t, 9.679660201e-02f);
        p = fmaf(p, t, 3.740904033e-01f);
        p = fmaf(p, t, 1.000023723e+00f);
        p = fmaf(p, t, -1.265512228e+00f);
        const float erfc_a = t * __builtin_amdgcn_exp2f(fmaf(-a, a, p) * kLog2e);
        // for x < 0, 1 - (1 - erfc): the reference's 1 + erf(z) in fp32, whose
        // erf(z) rounds next to -1 (so the sum is a multiple of 2^-24, and 0
        // once erfc < 2^-25)
        const float one_plus_erf = x < 0.0f ? 1.0f - (1.0f - erfc_a) : 2.0f - erfc_a;
        return x * 0.5f * one_plus_erf;
    } else {
        constexpr float kSqrt2OverPi = 0.79788456080286535588f;
        constexpr float kCubic = 0.044715f;
        const float cube = x * x * x;
        const float inner = kSqrt2OverPi * fmaf(kCubic, cube, x);
        // s = (1 + tanh u) / 2; 1 - (1 - 2s) is the reference's 1 + tanh(u) in
        // fp32, 0 once tanh(u) rounds to -1
        const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(inner * (-2.0f * kLog2e)));
        return 0.5f * x * (1.0f - (1.0f - 2.0f * s));
    }
}

constexpr bool act_is_silu(int op) {
    return op == ACT_SILU_AND_MUL || op == ACT_MUL_AND_SILU || op == ACT_SILU;
}

// REF: the reference formula; else fp32 tensors take it and 16-bit tensors
// the fast form.
template <int OP, int DT, bool REF> __device__ __forceinline__ float activation(float x) {
    if constexpr (REF || DT == KV_F32) return activation_ref<OP>(x);
    else return activation_fast<OP>(x);
}

// fp32 -> element type and back (round to nearest even; NaN stays NaN).
template <int DT> __device__ __forceinline__ float round_to(float x) {
    if constexpr (DT == KV_F16) return (float)(_Float16)x;
    else if constexpr (DT == KV_BF16) return (float)(__bf16)x;
    else return x;
}

// One output element from its input(s), fp32 in, fp32 out (already rounded
// to the element type; the product of two 16-bit values is exact in fp32, so
// rounding it once is the correctly rounded 16-bit product).
// The activation as an fp32 value, rounded: the empty asm hides the product
// that made it from the narrowing that follows, which the backend would
// otherwise fuse into one v_fma_mix (a single rounding to fp16 where the
// reference rounds to fp32 and then to fp16) in some kernels and not others.
template <int OP, int DT, bool REF> __device__ __forceinline__ float activation_f32(float x) {
    float r = activation<OP, DT, REF>(x);
    asm("" : "+v"(r));
    return r;
}

template <int OP, int DT, bool REF = false>
__device__ __forceinline__ float apply(float g, float u) {
    if constexpr (OP == ACT_MUL_AND_SILU)
        return round_to<DT>(g * round_to<DT>(activation_f32<OP, DT, REF>(u)));
    else if constexpr (act_is_gated(OP))
        return round_to<DT>(round_to<DT>(activation_f32<OP, DT, REF>(g)) * u);
    else return round_to<DT>(activation_f32<OP, DT, REF>(g));
}

// Whether these elements need the reference formula: bf16 silu arguments
// below kSiluFastMin (NaN compares false and stays on the fast path, which
// propagates it).
template <int OP, int DT, int N>
__device__ __forceinline__ bool needs_ref(const float (&g)[N], const float (&u)[N]) {
    if constexpr (DT == KV_BF16 && act_is_silu(OP)) {
        const float(&arg)[N] = OP == ACT_MUL_AND_SILU ? u : g;
        float m = arg[0];
#pragma unroll
        for (int e = 1; e < N; e++) m = fminf(m, arg[e]);
        return m < kSiluFastMin;
    } else {
        return false;
    }
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
            // values are already bf16-exact: the high halves are the bits
            c[i] = (__builtin_bit_cast(uint32_t, f[2 * i]) >> 16) |
                   (__builtin_bit_cast(uint32_t, f[2 * i + 1]) & 0xFFFF0000u);
        } else {
            c[i] = __builtin_bit_cast(uint32_t, f[i]);
        }
    }
    return c;
}

// One 16-byte output chunk per lane, one pass, one wavefront per workgroup.
// Measured on MI355X for fp16 silu_and_mul over 8192 x 14336 (704 MB): 104 us
// (6.8 TB/s) this way, against 109 us with 256-lane workgroups and 116-125 us
// for grid-stride loops of 2-8 chunks per lane; nontemporal loads and stores
// are worth 8% together.
template <int OP, int DT>
__global__ __launch_bounds__(kVecBlock) void activation_vec_kernel(const ActivationParams p) {
    constexpr int V = Chunk<DT>::kVec;
    const u32x4 *in = (const u32x4 *)p.input;
    u32x4 *out = (u32x4 *)p.out;
    const uint32_t i = blockIdx.x * kVecBlock + threadIdx.x;
    if (i >= p.chunks) return;
    u32x4 g, u;
    if constexpr (act_is_gated(OP)) {
        const uint32_t rc = p.row_chunks.d;
        const uint32_t t = div_by(i, p.row_chunks);
        const size_t gi = (size_t)i + (size_t)t * rc;
        g = __builtin_nontemporal_load(in + gi);
        u = __builtin_nontemporal_load(in + gi + rc);
    } else {
        g = __builtin_nontemporal_load(in + i);
    }
    float gf[V], uf[V], of[V];
    unpack<DT>(g, gf);
    if constexpr (act_is_gated(OP)) {
        unpack<DT>(u, uf);
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) uf[e] = 0.0f;
    }
    if (__builtin_expect(needs_ref<OP, DT>(gf, uf), 0)) {
#pragma unroll
        for (int e = 0; e < V; e++) of[e] = apply<OP, DT, true>(gf[e], uf[e]);
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) of[e] = apply<OP, DT>(gf[e], uf[e]);
    }
    __builtin_nontemporal_store(pack<DT>(of), out + i);
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
        float gv[1] = {g}, uv[1] = {u};
        const float r = needs_ref<OP, DT>(gv, uv) ? apply<OP, DT, true>(g, u) : apply<OP, DT>(g, u);
        store_elem<DT>(p.out, (size_t)i, r);
    }
}

template <int OP, int DT>
hipError_t launch_typed(const ActivationParams &p, bool vector_path, int num_cus,
                        hipStream_t stream) {
    // element kernel: a grid-stride loop over one resident round, 8
    // workgroups of 4 wavefronts per CU
    const long long cap = (long long)(num_cus > 0 ? num_cus : 256) * 8;
    if (vector_path) {
        const long long blocks = ((long long)p.chunks + kVecBlock - 1) / kVecBlock;
        if (blocks < 1) return hipSuccess;
        activation_vec_kernel<OP, DT><<<(unsigned)blocks, kVecBlock, 0, stream>>>(p);
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
