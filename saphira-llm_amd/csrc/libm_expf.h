/*
 * libm_expf.h -- single-precision e^x with the bits of glibc's expf.
 *
 * The reference's softmax runs its scalar tail through the C library's expf
 * (src/ops.c:386-422, n % 8 trailing scores), so a decode step on the GPU
 * reproduces that function, not merely an accurate exponential. glibc (2.28
 * and later, sysdeps/ieee754/flt-32/e_expf.c, from Szabolcs Nagy's
 * optimized-routines) evaluates it in double:
 *
 *   x*32/ln2 = k + r, k the nearest integer (by adding and subtracting
 *   1.5*2^52), |r| <= 1/2;
 *   2^(k/32) = T[k mod 32] with k/32's integer part added to the exponent
 *   field, T[i] the double nearest 2^(i/32);
 *   e^x ~= 2^(k/32) * (1 + c2*r + c1*r^2 + c0*r^3), cubic coefficients of
 *   2^(r/32) from the published exp2f data;
 *
 * and rounds the double result to float once. On x86-64 with FMA glibc
 * selects the build of this code compiled for FMA, whose multiply-adds are
 * fused: z + shift and z - kd with z = x*32/ln2, c0*r + c1, c2*r + 1 and
 * z*r^2 + y; r*r and the final scaling stay plain products. That is the form
 * restated below, with every fusion written as an explicit fma so that any
 * compiler and any device produce the same bits.
 *
 * Pinned exhaustively: every one of the 2^32 float inputs against the host
 * C library's expf (saphira-llm_amd/host/expf_check.c, run by the tests).
 * The table entries are computed from 2^(i/32) to 60 digits and rounded to
 * nearest, not transcribed.
 *
 * Compiled as C (host) and as HIP (device); SLLM_HD marks the functions.
 */
#ifndef SLLM_LIBM_EXPF_H
#define SLLM_LIBM_EXPF_H

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define SLLM_HD __host__ __device__ static inline
#else
#define SLLM_HD static inline
#endif

/* T[i] = bits(2^(i/32)) - (i << 47): adding k << 47 then puts k/32 into the
 * exponent field and leaves 2^((k mod 32)/32) in the mantissa. */
#define SLLM_EXPF_TAB_INIT {                                                       \
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL,           \
    0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL,           \
    0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL,           \
    0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,           \
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL,           \
    0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL,           \
    0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL,           \
    0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,           \
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL,           \
    0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL,           \
    0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL }

SLLM_HD uint32_t sllm_f32_bits(float f) { uint32_t u; __builtin_memcpy(&u, &f, 4); return u; }
SLLM_HD double sllm_f64_from(uint64_t u) { double d; __builtin_memcpy(&d, &u, 8); return d; }
SLLM_HD uint64_t sllm_f64_bits(double d) { uint64_t u; __builtin_memcpy(&u, &d, 8); return u; }

/* tab: the 32 entries of SLLM_EXPF_TAB_INIT (a table in whichever memory the
 * caller keeps it). */
SLLM_HD float sllm_libm_expf(float x, const uint64_t *tab) {
    const uint32_t abstop = (sllm_f32_bits(x) >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                              /* |x| >= 88, or NaN */
        if (sllm_f32_bits(x) == 0xff800000u) return 0.0f;           /* -inf */
        if (abstop >= 0x7f8u) return x + x;                         /* inf / NaN */
        if (x > 0x1.62e42ep6f) return HUGE_VALF;                    /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                        /* underflow */
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double xd = (double) x;
    const double kd_s = fma(inv_ln2_n, xd, shift);                  /* z + shift */
    const uint64_t ki = sllm_f64_bits(kd_s);
    const double kd = kd_s - shift;
    const double r = fma(inv_ln2_n, xd, -kd);                       /* z - kd */
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = sllm_f64_from(t);
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float) y;
}

#endif /* SLLM_LIBM_EXPF_H */
