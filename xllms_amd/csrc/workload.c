/*
 * Seeded synthetic inputs for the paged-decode workloads (host only).
 *
 * One counter-based generator so that every consumer (GPU harness, CPU
 * baseline, tests) sees bit-identical host buffers: element i of a stream is a
 * pure function of (seed, i), so filling is embarrassingly parallel and
 * independent of thread count.
 *   uniform: SplitMix64 finaliser applied to seed + (ctr+1)*0x9E3779B97F4A7C15
 *            (Steele, Lea, Flood, "Fast splittable pseudorandom number
 *            generators", OOPSLA 2014; constants as published by Vigna).
 *   normal:  Box-Muller on the pair (2j, 2j+1): element 2j = r cos(theta),
 *            element 2j+1 = r sin(theta), r = sqrt(-2 ln u1),
 *            theta = 2 pi u2, evaluated in double and rounded to fp32; 16-bit
 *            outputs then round that fp32 value to nearest-even once.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { XW_FP16 = 1, XW_BF16 = 2, XW_FP32 = 3 };

static inline uint64_t xw_mix(uint64_t seed, uint64_t ctr) {
    uint64_t z = seed + (ctr + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t xw_uniform_u64(uint64_t seed, uint64_t ctr) { return xw_mix(seed, ctr); }

float xw_normal(uint64_t seed, uint64_t i) {
    uint64_t j = i >> 1;
    uint64_t a = xw_mix(seed, 2 * j), b = xw_mix(seed, 2 * j + 1);
    double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1.0p-53;         /* [0, 1) */
    double r = sqrt(-2.0 * log(u1));
    double th = 6.283185307179586476925286766559 * u2;
    return (float)((i & 1) ? r * sin(th) : r * cos(th));
}

/* fp32 -> IEEE binary16, round to nearest even (incl. subnormals, overflow to
 * inf, quiet NaN).  Normal range: add the exponent rebias plus a rounding
 * constant of 0xfff + (lsb of the kept mantissa) and shift; subnormal range:
 * let the FPU round by adding 0.5f, whose ulp is the binary16 subnormal
 * step 2^-24. */
uint16_t xw_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x47800000u) { /* >= 65536, inf or nan */
        if (ax > 0x7F800000u) return sign | 0x7E00u;
        return sign | 0x7C00u;
    }
    if (ax < 0x38800000u) { /* below 2^-14: binary16 subnormal or zero */
        float af;
        memcpy(&af, &ax, 4);
        volatile float t = af + 0.5f;
        uint32_t tb;
        float tv = t;
        memcpy(&tb, &tv, 4);
        return sign | (uint16_t)(tb - 0x3F000000u);
    }
    uint32_t odd = (ax >> 13) & 1u;
    ax += 0xC8000FFFu + odd; /* rebias exponent by (15-127)<<23, round */
    return sign | (uint16_t)(ax >> 13);
}

uint16_t xw_float_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

/* dst[k] = normal(seed, offset + k) * mul, stored as dtype, k < n. */
void xw_fill_normal(void *dst, size_t n, int dtype, uint64_t seed, uint64_t offset,
                    float mul, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
    for (size_t k = 0; k < n; k++) {
        float v = xw_normal(seed, offset + k) * mul;
        if (dtype == XW_FP16)
            ((uint16_t *)dst)[k] = xw_float_to_half(v);
        else if (dtype == XW_BF16)
            ((uint16_t *)dst)[k] = xw_float_to_bf16(v);
        else
            ((float *)dst)[k] = v;
    }
    (void)nthreads;
}

/* Scale selected rows of a row-major [nrows][row_len] buffer by `mul` before
 * the single rounding to dtype: rows[i] lists the row indices.  The values are
 * regenerated from the stream (seed, row*row_len + offset), so the result is
 * what xw_fill_normal(mul=1) followed by an exact fp32 multiply and one
 * rounding would give. */
void xw_scale_rows(void *dst, const int64_t *rows, size_t nrows_sel, size_t row_len,
                   int dtype, uint64_t seed, uint64_t offset, float mul, int nthreads) {
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
    for (size_t i = 0; i < nrows_sel; i++) {
        size_t base = (size_t)rows[i] * row_len;
        for (size_t e = 0; e < row_len; e++) {
            float v = xw_normal(seed, offset + base + e) * mul;
            if (dtype == XW_FP16)
                ((uint16_t *)dst)[base + e] = xw_float_to_half(v);
            else if (dtype == XW_BF16)
                ((uint16_t *)dst)[base + e] = xw_float_to_bf16(v);
            else
                ((float *)dst)[base + e] = v;
        }
    }
    (void)nthreads;
}

int xw_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
