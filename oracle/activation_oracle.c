/*
 * CPU oracle for the MLP activation operators of the reference's operator API.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP plugin, the
 * Python host mirror) may link, load or call this file.  Only tests/ and
 * bench.py's cpu_baseline leg use it, as the checker (or as the timed CPU
 * baseline), never as the thing measured.
 *
 * What it restates (from the reference, read as text, not copied):
 *
 *  oracle_activation
 *      operators/activation_kernels.cu:24-134, the six kernels behind
 *      include/operator_api.h:122-150, element by element:
 *        silu(x)      = x / (1 + expf(-x))                        (:24-28)
 *        gelu(x)      = (x * 0.5f) * (1 + erff(x * (float)M_SQRT1_2))
 *                                                                 (:30-36)
 *        gelu_tanh(x) = (0.5f * x) * (1 + tanhf(inner)),          (:38-48)
 *          inner = (float)(sqrt(2)*(2/sqrt(pi))*0.5) * (x + 0.044715f*x^3)
 *          with x + 0.044715f*x^3 a fused multiply-add: the reference is
 *          compiled by nvcc, which contracts a*b+c into one FMA by default
 *          (--fmad=true), and this is the only such site in the three
 *          functions;
 *      each device function returns T (:27, :35, :47), so the activation is
 *      rounded to the element type; a gated kernel multiplies it by the other
 *      operand in T (:65-69, :86, :102): for fp16 the reference's half
 *      operator* is one correctly rounded fp16 multiply, which the exact
 *      fp32 product of two fp16 values rounded once reproduces.  Rows:
 *      input row t of a gated op is [gate (d) | up (d)] at t*2d (:58-60),
 *      silu_and_mul = silu(gate)*up, mul_and_silu = gate*silu(up) (:65-69),
 *      gelu(_tanh)_and_mul = act(gate)*up; element-wise ops read row t at
 *      t*d (:113).  dtype codes 1 fp16, 2 bf16 (this build's extension, the
 *      same rules with bf16 rounding), 3 fp32.
 *
 *  oracle_activation_mt
 *      The same, rows split over OpenMP threads (bit-identical); the
 *      multi-core CPU baseline.
 *
 *  oracle_float_to_half / oracle_float_to_bf16
 *      fp32 -> binary16 / bfloat16, round to nearest even, with subnormals,
 *      overflow to infinity and NaN kept NaN (the reference's __float2half).
 *
 * Pinning (tests/test_activation_oracle.py): the conversions against numpy /
 * torch; every op against its closed form in double precision (numpy, scipy's
 * erf) with the same roundings to the element type, special values, the
 * odd-part identities act(x) - act(-x) = x, and the gate / up order.
 */
#define _DEFAULT_SOURCE /* M_SQRT1_2, M_SQRT2, M_2_SQRTPI under -std=c11 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

enum { ACT_DT_F16 = 1, ACT_DT_BF16 = 2, ACT_DT_F32 = 3 };
enum {
    ACT_SILU_AND_MUL = 1,
    ACT_MUL_AND_SILU = 2,
    ACT_GELU_AND_MUL = 3,
    ACT_GELU_TANH_AND_MUL = 4,
    ACT_GELU = 5,
    ACT_SILU = 6,
};

static float f32_of_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t bits_of_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* binary16 -> binary32, exact. */
static float act_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1F) return f32_of_bits(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return f32_of_bits(sign);
        /* subnormal: man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return f32_of_bits(sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest even. */
uint16_t oracle_float_to_half(float f) {
    const uint32_t u = bits_of_f32(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu)); /* NaN */
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520: rounds to inf */
    if (a < 0x38800000u) {
        /* below the smallest normal 2^-14: a multiple of 2^-24 after rounding */
        const float mag = f32_of_bits(a);
        /* mag * 2^24 is exact in fp32 (a power-of-two scale); rint rounds
         * half to even in the default rounding mode */
        const float q = rintf(mag * 16777216.0f);
        return (uint16_t)(sign | (uint16_t)q); /* q <= 1024 = smallest normal */
    }
    /* normal: keep 10 of the 23 mantissa bits, round to nearest even */
    const uint32_t exp = ((a >> 23) - 127 + 15);
    uint32_t man = a & 0x7FFFFFu;
    uint32_t h = (exp << 10) | (man >> 13);
    const uint32_t rest = man & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++; /* may carry into exp: fine */
    return (uint16_t)(sign | h);
}

/* binary32 -> bfloat16, round to nearest even. */
uint16_t oracle_float_to_bf16(float f) {
    const uint32_t u = bits_of_f32(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static float round_to(float x, int dt) {
    if (dt == ACT_DT_F16) return act_half_to_float(oracle_float_to_half(x));
    if (dt == ACT_DT_BF16) return f32_of_bits((uint32_t)oracle_float_to_bf16(x) << 16);
    return x;
}

static float load(const void *base, size_t i, int dt) {
    if (dt == ACT_DT_F16) return act_half_to_float(((const uint16_t *)base)[i]);
    if (dt == ACT_DT_BF16) return f32_of_bits((uint32_t)((const uint16_t *)base)[i] << 16);
    return ((const float *)base)[i];
}

/* x is already representable in dt */
static void store(void *base, size_t i, float x, int dt) {
    if (dt == ACT_DT_F16) ((uint16_t *)base)[i] = oracle_float_to_half(x);
    else if (dt == ACT_DT_BF16) ((uint16_t *)base)[i] = oracle_float_to_bf16(x);
    else ((float *)base)[i] = x;
}

static float silu(float x) { return x / (1.0f + expf(-x)); }

static float gelu(float x) {
    const float alpha = (float)M_SQRT1_2;
    return x * 0.5f * (1.0f + erff(x * alpha));
}

static float gelu_tanh(float x) {
    const float beta = (float)(M_SQRT2 * M_2_SQRTPI * 0.5);
    const float kappa = 0.044715f;
    const float x_cube = x * x * x;
    const float inner = beta * fmaf(kappa, x_cube, x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

static int act_valid(int op, int dt) {
    return op >= ACT_SILU_AND_MUL && op <= ACT_SILU && dt >= ACT_DT_F16 && dt <= ACT_DT_F32;
}

static void act_row(int op, void *out, const void *input, long long t, int d, int dt) {
    const int gated = op <= ACT_GELU_TANH_AND_MUL;
    const size_t in0 = (size_t)t * (size_t)d * (gated ? 2u : 1u);
    const size_t out0 = (size_t)t * (size_t)d;
    for (int i = 0; i < d; i++) {
        const float x = load(input, in0 + (size_t)i, dt);
        float r;
        if (!gated) {
            r = round_to(op == ACT_SILU ? silu(x) : gelu(x), dt);
        } else {
            const float y = load(input, in0 + (size_t)d + (size_t)i, dt);
            switch (op) {
            case ACT_SILU_AND_MUL: r = round_to(round_to(silu(x), dt) * y, dt); break;
            case ACT_MUL_AND_SILU: r = round_to(x * round_to(silu(y), dt), dt); break;
            case ACT_GELU_AND_MUL: r = round_to(round_to(gelu(x), dt) * y, dt); break;
            default: r = round_to(round_to(gelu_tanh(x), dt) * y, dt); break;
            }
        }
        store(out, out0 + (size_t)i, r, dt);
    }
}

/* out[num_tokens][d] from input[num_tokens][2d] (gated) or [num_tokens][d].
 * Returns 0, or -1 for an unknown op / dtype or negative sizes. */
int oracle_activation(int op, void *out, const void *input, long long num_tokens, int d, int dt) {
    if (!act_valid(op, dt) || num_tokens < 0 || d < 0) return -1;
    for (long long t = 0; t < num_tokens; t++) act_row(op, out, input, t, d, dt);
    return 0;
}

int oracle_activation_mt(int op, void *out, const void *input, long long num_tokens, int d, int dt,
                         int threads) {
    if (!act_valid(op, dt) || num_tokens < 0 || d < 0) return -1;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (long long t = 0; t < num_tokens; t++) act_row(op, out, input, t, d, dt);
    return 0;
}
