/*
 * gsx_math.h - scalar math shared by the gfx950 kernels and the host-side C code.
 *
 * The gsx CPU backend decides which Gaussians and which pixel contributions exist through
 * float thresholds on glibc expf results (gsx/src/gsx-cpu/render.c:106-111, :1055-1070):
 * a 1-ulp difference in exp(power) can flip a contribution whose alpha sits at 1/255. To
 * reproduce those decisions bit for bit on the GPU this header restates the published
 * expf algorithm of ARM's optimized-routines (the code glibc >= 2.27 ships as expf): an
 * exp2 table of 32 entries in double, a cubic polynomial, and the round-to-int via the
 * 0x1.8p52 shift. x86-64 glibc dispatches to its FMA build on FMA-capable CPUs, so the
 * reduction and the polynomial use fused multiply-adds at exactly the points that build
 * fuses them. The restatement was compared against the host's glibc expf for all 2^32
 * float inputs with zero mismatches; tests/test_oracle_cpu.py repeats that check.
 *
 * The same holds for logf, sinf, cosf and powf below (ARM optimized-routines logf, sincosf and
 * powf, also the code glibc ships, with their 16-entry log / log2 tables, the 2/pi bits of the
 * large-argument reduction and the exp2 table above): the ADC's split offsets, the MCMC noise
 * and relocation, randn fills and the sRGB curves use them, so those results are glibc's, bit
 * for bit. logf, sinf and cosf were compared against the host glibc for all 2^32 inputs, powf
 * over 1e8 random pairs and every x in [0, 1] with the exponents the ADC uses, with zero
 * mismatches.
 *
 * Every function here is pure IEEE arithmetic and must be compiled without floating-point
 * contraction (-ffp-contract=off): the explicit fma() calls are the only fused operations.
 *
 * Third-party notice. The lookup tables, polynomial coefficients, bit windows and reduction
 * steps of expf, logf, sincosf and powf below follow Arm's optimized-routines
 * (https://github.com/ARM-software/optimized-routines, math/), which carries:
 *   Copyright (c) 2017-2024, Arm Limited.
 *   SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception
 * Those parts are used under the MIT licence; its terms travel with this notice: permission
 * is granted to use, copy, modify, merge, publish, distribute, sublicense and/or sell copies,
 * provided that the copyright notice and this permission notice are included in all copies or
 * substantial portions; the software is provided "as is", without warranty of any kind.
 */
#ifndef GSX_AMD_MATH_H
#define GSX_AMD_MATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define GSX_HD __host__ __device__ inline
#define GSX_FMA(a, b, c) __builtin_fma((a), (b), (c))
#define GSX_FMAF(a, b, c) __builtin_fmaf((a), (b), (c))
#else
#include <math.h>
#include <string.h>
#define GSX_HD static inline
#define GSX_FMA(a, b, c) fma((a), (b), (c))
#define GSX_FMAF(a, b, c) fmaf((a), (b), (c))
#endif

/* 2^(i/32) rounded to nearest double, with i << 47 subtracted from the bit pattern so that
 * adding the scaled integer part of the reduced argument rebuilds 2^(k/32) directly. */
#define GSX_EXP2_TABLE_BITS 5
#define GSX_EXP2_TABLE_SIZE 32

/* The table entries (those of ARM's optimized-routines expf, which glibc ships). Host code reads
 * a static array; device code a constant array in each code object, so a lookup is one load
 * instead of a per-lane branch tree. Kernels with many expf calls per lane also copy
 * it to LDS once and use gsx_expf_table with that copy, or build gsx_expf_blend's folded
 * table (see below). */
#define GSX_EXP2_TABLE_INIT                                                                        \
  { \
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL, \
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, \
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL, \
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL, \
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, \
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL, \
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL, \
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL \
  }

static const uint64_t gsx_exp2_table_host[GSX_EXP2_TABLE_SIZE] = GSX_EXP2_TABLE_INIT;
#if defined(__HIPCC__)
static __device__ const uint64_t gsx_exp2_table_dev[GSX_EXP2_TABLE_SIZE] = GSX_EXP2_TABLE_INIT;

__host__ __device__ inline uint64_t gsx_exp2_table_entry(uint32_t i)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return gsx_exp2_table_dev[i & 31u];
#else
    return gsx_exp2_table_host[i & 31u];
#endif
}
#else
static inline uint64_t gsx_exp2_table_entry(uint32_t i)
{
    return gsx_exp2_table_host[i & 31u];
}
#endif

GSX_HD uint32_t gsx_f32_bits(float x)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint32_t, x);
#else
    uint32_t u;
    memcpy(&u, &x, sizeof(u));
    return u;
#endif
}

GSX_HD float gsx_f32_from_bits(uint32_t u)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(float, u);
#else
    float x;
    memcpy(&x, &u, sizeof(x));
    return x;
#endif
}

GSX_HD uint64_t gsx_f64_bits(double x)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint64_t, x);
#else
    uint64_t u;
    memcpy(&u, &x, sizeof(u));
    return u;
#endif
}

GSX_HD double gsx_f64_from_bits(uint64_t u)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(double, u);
#else
    double x;
    memcpy(&x, &u, sizeof(x));
    return x;
#endif
}

/* expf with glibc's (FMA build) results for every float input. `table` supplies the 32
 * entries of gsx_exp2_table_entry (a kernel stages them in LDS: a per-lane switch would become
 * a divergent branch tree); pass NULL to use the switch. */
GSX_HD float gsx_expf_table(float x, const uint64_t *table)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t abstop = (gsx_f32_bits(x) >> 20) & 0x7ffu;
    double xd = (double)x;
    double z;
    double kd;
    double r;
    double r2;
    double y;
    double s;
    uint64_t ki;
    uint64_t t;

    if(abstop >= 0x42bu) { /* |x| >= 88 (top 12 bits of 88.0f), inf or nan */
        if(gsx_f32_bits(x) == 0xff800000u) {
            return 0.0f;
        }
        if(abstop >= 0x7f8u) {
            return x + x;
        }
        if(x > 0x1.62e42ep6f) {
            return gsx_f32_from_bits(0x7f800000u);
        }
        if(x < -0x1.9fe368p6f) {
            return 0.0f;
        }
    }
    z = inv_ln2_n * xd;
    kd = z + shift;
    ki = gsx_f64_bits(kd);
    kd -= shift;
    r = GSX_FMA(inv_ln2_n, xd, -kd);
    t = table != 0 ? table[ki % 32u] : gsx_exp2_table_entry((uint32_t)(ki % 32u));
    t += ki << (52 - GSX_EXP2_TABLE_BITS);
    s = gsx_f64_from_bits(t);
    z = GSX_FMA(c0, r, c1);
    r2 = r * r;
    y = GSX_FMA(c2, r, 1.0);
    y = GSX_FMA(z, r2, y);
    y = y * s;
    return (float)y;
}

GSX_HD float gsx_expf(float x)
{
    return gsx_expf_table(x, 0);
}

/* gsx_expf_table on [-4.5, 0], the blend kernels' clamped powers, with the exponent folded into
 * the table: there round(x * 32/ln2) = k lies in [-208, 0], ki (the bits of kd) is
 * 0x4338000000000000 + k, so gsx_expf_table's  t = table[ki % 32] + (ki << 47)  equals
 * table[k mod 32] + (k << 47) (mod 2^64), a function of k alone. Entry k + 208 of a
 * GSX_EXPF_BLEND_TABLE_SIZE-entry table holds it (gsx_expf_blend_entry), and k + 208 is the low
 * word of ki plus 208: one add and one load instead of masking, shifting and a 64-bit add.
 * Bit-identical to gsx_expf for every float in [-4.5, 0] (checked exhaustively on the host). */
#define GSX_EXPF_BLEND_BIAS 208
#define GSX_EXPF_BLEND_TABLE_SIZE 209

GSX_HD uint64_t gsx_expf_blend_entry(uint32_t j)
{
    const int32_t k = (int32_t)j - GSX_EXPF_BLEND_BIAS;
    return gsx_exp2_table_entry((uint32_t)k & 31u) + ((uint64_t)(int64_t)k << (52 - GSX_EXP2_TABLE_BITS));
}

GSX_HD float gsx_expf_blend(float x, const uint64_t *table)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint32_t klo = (uint32_t)gsx_f64_bits(kd);
    double r;
    double r2;
    double y;
    uint64_t t;

    kd -= shift;
    r = GSX_FMA(inv_ln2_n, xd, -kd);
    t = table[klo + GSX_EXPF_BLEND_BIAS];
    z = GSX_FMA(c0, r, c1);
    r2 = r * r;
    y = GSX_FMA(c2, r, 1.0);
    y = GSX_FMA(z, r2, y);
    y = y * gsx_f64_from_bits(t);
    return (float)y;
}

/* ---- logf (ARM optimized-routines logf: 16 subintervals of [0x1.66p-1, 0x1.66p0)) --------------
 * Entry i: 1/c and log(c) for c near the centre of subinterval i, as double bit patterns. */
#define GSX_LOGF_TABLE_INIT                                                                         \
  { \
    0x3ff661ec79f8f3beULL, 0xbfd57bf7808caadeULL, 0x3ff571ed4aaf883dULL, 0xbfd2bef0a7c06ddbULL, \
    0x3ff49539f0f010b0ULL, 0xbfd01eae7f513a67ULL, 0x3ff3c995b0b80385ULL, 0xbfcb31d8a68224e9ULL, \
    0x3ff30d190c8864a5ULL, 0xbfc6574f0ac07758ULL, 0x3ff25e227b0b8ea0ULL, 0xbfc1aa2bc79c8100ULL, \
    0x3ff1bb4a4a1a343fULL, 0xbfba4e76ce8c0e5eULL, 0x3ff12358f08ae5baULL, 0xbfb1973c5a611cccULL, \
    0x3ff0953f419900a7ULL, 0xbfa252f438e10c1eULL, 0x3ff0000000000000ULL, 0x0000000000000000ULL, \
    0x3fee608cfd9a47acULL, 0x3faaa5aa5df25984ULL, 0x3feca4b31f026aa0ULL, 0x3fbc5e53aa362eb4ULL, \
    0x3feb2036576afce6ULL, 0x3fc526e57720db08ULL, 0x3fe9c2d163a1aa2dULL, 0x3fcbc2860d224770ULL, \
    0x3fe886e6037841edULL, 0x3fd1058bc8a07ee1ULL, 0x3fe767dcf5534862ULL, 0x3fd4043057b6ee09ULL  \
  }
/* log2(c) of the same c (powf's log2, ARM optimized-routines powf_log2_data) */
#define GSX_LOG2F_TABLE_INIT                                                                        \
  { \
    0xbfdefec65b963019ULL, 0xbfdb0b6832d4fca4ULL, 0xbfd7418b0a1fb77bULL, 0xbfd39de91a6dcf7bULL, \
    0xbfd01d9bf3f2b631ULL, 0xbfc97c1d1b3b7af0ULL, 0xbfc2f9e393af3c9fULL, 0xbfb960cbbf788d5cULL, \
    0xbfaa6f9db6475fceULL, 0x0000000000000000ULL, 0x3fb338ca9f24f53dULL, 0x3fc476a9543891baULL, \
    0x3fce840b4ac4e4d2ULL, 0x3fd40645f0c6651cULL, 0x3fd88e9c2c1b9ff8ULL, 0x3fdce0a44eb17bccULL  \
  }

static const uint64_t gsx_logf_table_host[32] = GSX_LOGF_TABLE_INIT;
static const uint64_t gsx_log2f_table_host[16] = GSX_LOG2F_TABLE_INIT;
#if defined(__HIPCC__)
static __device__ const uint64_t gsx_logf_table_dev[32] = GSX_LOGF_TABLE_INIT;
static __device__ const uint64_t gsx_log2f_table_dev[16] = GSX_LOG2F_TABLE_INIT;
#endif

/* entry j of the logf table (1/c at 2i, log(c) at 2i + 1) and entry i of the log2 table */
GSX_HD uint64_t gsx_logf_table_entry(uint32_t j)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return gsx_logf_table_dev[j & 31u];
#else
    return gsx_logf_table_host[j & 31u];
#endif
}

GSX_HD uint64_t gsx_log2f_table_entry(uint32_t i)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return gsx_log2f_table_dev[i & 15u];
#else
    return gsx_log2f_table_host[i & 15u];
#endif
}

/* logf with glibc's (FMA build) result for every float input. */
GSX_HD float gsx_logf(float x)
{
    const double ln2 = 0x1.62e42fefa39efp-1;
    const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2, a2 = -0x1.ffffef20a4123p-2;
    uint32_t ix = gsx_f32_bits(x);
    uint32_t tmp, iz, i;
    int32_t k;
    double z, r, r2, y, y0, invc, logc;

    if(ix == 0x3f800000u) {
        return 0.0f;
    }
    if(ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        if(ix * 2u == 0u) {
            return gsx_f32_from_bits(0xff800000u); /* -inf */
        }
        if(ix == 0x7f800000u) {
            return x;
        }
        if((ix & 0x80000000u) != 0u || ix * 2u >= 0xff000000u) {
            return gsx_f32_from_bits(0x7fc00000u); /* NaN */
        }
        ix = gsx_f32_bits(x * 0x1p23f) - (23u << 23); /* subnormal: normalise */
    }
    tmp = ix - 0x3f330000u;
    i = (tmp >> 19) & 15u;
    k = (int32_t)tmp >> 23;
    iz = ix - (tmp & 0xff800000u);
    invc = gsx_f64_from_bits(gsx_logf_table_entry(2u * i));
    logc = gsx_f64_from_bits(gsx_logf_table_entry(2u * i + 1u));
    z = (double)gsx_f32_from_bits(iz);
    r = GSX_FMA(z, invc, -1.0);
    y0 = GSX_FMA((double)k, ln2, logc);
    r2 = r * r;
    y = GSX_FMA(a1, r, a2);
    y = GSX_FMA(a0, r2, y);
    y = GSX_FMA(y, r2, y0 + r);
    return (float)y;
}

/* ---- sinf / cosf (ARM optimized-routines sincosf) ---------------------------------------------- */
/* 2/pi in 24 overlapping 32-bit windows, 8 bits apart (the large-argument reduction) */
#define GSX_INV_PIO4_INIT                                                                            \
  { \
    0xa2u, 0xa2f9u, 0xa2f983u, 0xa2f9836eu, 0xf9836e4eu, 0x836e4e44u, 0x6e4e4415u, 0x4e441529u, \
    0x441529fcu, 0x1529fc27u, 0x29fc2757u, 0xfc2757d1u, 0x2757d1f5u, 0x57d1f534u, 0xd1f534ddu,  \
    0xf534ddc0u, 0x34ddc0dbu, 0xddc0db62u, 0xc0db6295u, 0xdb629599u, 0x6295993cu, 0x95993c43u,  \
    0x993c4390u, 0x3c439041u                                                                    \
  }
static const uint32_t gsx_inv_pio4_host[24] = GSX_INV_PIO4_INIT;
#if defined(__HIPCC__)
static __device__ const uint32_t gsx_inv_pio4_dev[24] = GSX_INV_PIO4_INIT;
#endif

GSX_HD uint32_t gsx_abstop12(float x)
{
    return (gsx_f32_bits(x) >> 20) & 0x7ffu;
}

/* The polynomial of sincosf: odd n evaluates cos(x), even n sin(x), for |x| <= pi/4; `flip`
 * selects the sign-flipped cosine coefficients of the second table (quadrants 2 and 3). */
GSX_HD float gsx_sincosf_poly(double x, double x2, int n, int flip)
{
    const double c0 = flip ? -0x1p0 : 0x1p0;
    const double c1 = flip ? 0x1.ffffffd0c621cp-2 : -0x1.ffffffd0c621cp-2;
    const double c2 = flip ? -0x1.55553e1068f19p-5 : 0x1.55553e1068f19p-5;
    const double c3 = flip ? 0x1.6c087e89a359dp-10 : -0x1.6c087e89a359dp-10;
    const double c4 = flip ? -0x1.99343027bf8c3p-16 : 0x1.99343027bf8c3p-16;
    const double s1 = -0x1.555545995a603p-3, s2 = 0x1.1107605230bc4p-7, s3 = -0x1.994eb3774cf24p-13;

    if((n & 1) == 0) {
        const double x3 = x * x2;
        const double t1 = GSX_FMA(x2, s3, s2);
        const double x7 = x3 * x2;
        const double s = GSX_FMA(x3, s1, x);
        return (float)GSX_FMA(x7, t1, s);
    } else {
        const double x4 = x2 * x2;
        const double t2 = GSX_FMA(x2, c4, c3);
        const double t1 = GSX_FMA(x2, c1, c0);
        const double x6 = x4 * x2;
        const double c = GSX_FMA(x4, c2, t1);
        return (float)GSX_FMA(x6, t2, c);
    }
}

/* x - n pi/2 for |x| < 120, n = round(x 2/pi) from the top bits of x 2^24 2/pi */
GSX_HD double gsx_sincosf_reduce_fast(double x, int *np)
{
    const double r = x * 0x1.45F306DC9C883p+23;
    const int n = ((int32_t)r + 0x800000) >> 24;

    *np = n;
    return GSX_FMA(-(double)n, 0x1.921FB54442D18p0, x);
}

/* Payne-Hanek style reduction with 96 bits of 2/pi for |x| >= 120 */
GSX_HD double gsx_sincosf_reduce_large(uint32_t xi, int *np)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t *arr = &gsx_inv_pio4_dev[(xi >> 26) & 15u];
#else
    const uint32_t *arr = &gsx_inv_pio4_host[(xi >> 26) & 15u];
#endif
    const int shift = (int)((xi >> 23) & 7u);
    uint64_t n, res0, res1, res2;

    xi = (xi & 0xffffffu) | 0x800000u;
    xi <<= shift;
    res0 = (uint64_t)(uint32_t)(xi * arr[0]);
    res1 = (uint64_t)xi * arr[4];
    res2 = (uint64_t)xi * arr[8];
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    n = (res0 + (1ull << 61)) >> 62;
    res0 -= n << 62;
    *np = (int)n;
    return (double)(int64_t)res0 * 0x1.921FB54442D18p-62;
}

/* want_cos: 1 for cosf, 0 for sinf; glibc's result for every float input */
GSX_HD float gsx_sincosf_one(float y, int want_cos)
{
    const float pio4f = 0x1.921FB6p-1f;
    double x = (double)y;
    double s;
    int n = 0;

    if(gsx_abstop12(y) < gsx_abstop12(pio4f)) {
        const double x2 = x * x;

        if(gsx_abstop12(y) < gsx_abstop12(0x1p-12f)) {
            return want_cos ? 1.0f : y;
        }
        return gsx_sincosf_poly(x, x2, want_cos, 0);
    } else if(gsx_abstop12(y) < gsx_abstop12(120.0f)) {
        x = gsx_sincosf_reduce_fast(x, &n);
        s = (n & 3) == 0 || (n & 3) == 3 ? 1.0 : -1.0;
        return gsx_sincosf_poly(x * s, x * x, want_cos ? n ^ 1 : n, (n & 2) != 0);
    } else if(gsx_abstop12(y) < 0x7f8u) {
        const uint32_t xi = gsx_f32_bits(y);
        const int sign = (int)(xi >> 31);

        x = gsx_sincosf_reduce_large(xi, &n);
        s = ((n + sign) & 3) == 0 || ((n + sign) & 3) == 3 ? 1.0 : -1.0;
        return gsx_sincosf_poly(x * s, x * x, want_cos ? n ^ 1 : n, ((n + sign) & 2) != 0);
    }
    return gsx_f32_from_bits(0x7fc00000u); /* inf or NaN: NaN */
}

GSX_HD float gsx_cosf(float x) { return gsx_sincosf_one(x, 1); }
GSX_HD float gsx_sinf(float x) { return gsx_sincosf_one(x, 0); }

/* ---- powf (ARM optimized-routines powf: log2 in double, then exp2 with the table above) -------- */
GSX_HD double gsx_powf_log2(uint32_t ix)
{
    const double a0 = 0x1.27616c9496e0bp-2, a1 = -0x1.71969a075c67ap-2, a2 = 0x1.ec70a6ca7baddp-2;
    const double a3 = -0x1.7154748bef6c8p-1, a4 = 0x1.71547652ab82bp0;
    const uint32_t tmp = ix - 0x3f330000u;
    const uint32_t i = (tmp >> 19) & 15u;
    const uint32_t top = tmp & 0xff800000u;
    const uint32_t iz = ix - top;
    const int32_t k = (int32_t)top >> 23;
    const double invc = gsx_f64_from_bits(gsx_logf_table_entry(2u * i));
    const double logc = gsx_f64_from_bits(gsx_log2f_table_entry(i));
    const double z = (double)gsx_f32_from_bits(iz);
    const double r = GSX_FMA(z, invc, -1.0);
    const double y0 = logc + (double)k;
    const double r2 = r * r;
    double y = GSX_FMA(a0, r, a1);
    const double p = GSX_FMA(a2, r, a3);
    const double r4 = r2 * r2;
    double q = GSX_FMA(a4, r, y0);

    q = GSX_FMA(p, r2, q);
    y = GSX_FMA(y, r4, q);
    return y;
}

GSX_HD float gsx_powf_exp2(double xd, uint32_t sign_bias)
{
    const double shift = 0x1.8p+52 / 32.0;
    const double c0 = 0x1.c6af84b912394p-5, c1 = 0x1.ebfce50fac4f3p-3, c2 = 0x1.62e42ff0c52d6p-1;
    double kd = xd + shift;
    const uint64_t ki = gsx_f64_bits(kd);
    double r, z, r2, y;
    uint64_t t;

    kd -= shift;
    r = xd - kd;
    t = gsx_exp2_table_entry((uint32_t)(ki % 32u));
    t += (ki + sign_bias) << (52 - GSX_EXP2_TABLE_BITS);
    z = GSX_FMA(c0, r, c1);
    r2 = r * r;
    y = GSX_FMA(c2, r, 1.0);
    y = GSX_FMA(z, r2, y);
    y = y * gsx_f64_from_bits(t);
    return (float)y;
}

/* 0: y not an integer, 1: odd integer, 2: even integer */
GSX_HD int gsx_powf_checkint(uint32_t iy)
{
    const int e = (int)((iy >> 23) & 0xffu);

    if(e < 0x7f) return 0;
    if(e > 0x7f + 23) return 2;
    if((iy & ((1u << (0x7f + 23 - e)) - 1u)) != 0u) return 0;
    if((iy & (1u << (0x7f + 23 - e))) != 0u) return 1;
    return 2;
}

GSX_HD int gsx_powf_zeroinfnan(uint32_t ix)
{
    return 2u * ix - 1u >= 2u * 0x7f800000u - 1u;
}

/* powf with glibc's (FMA build) results (x, y finite, zero, inf and NaN handled as glibc) */
GSX_HD float gsx_powf(float x, float y)
{
    uint32_t sign_bias = 0u;
    uint32_t ix = gsx_f32_bits(x);
    const uint32_t iy = gsx_f32_bits(y);
    double logx, ylogx;

    if(ix - 0x00800000u >= 0x7f800000u - 0x00800000u || gsx_powf_zeroinfnan(iy)) {
        if(gsx_powf_zeroinfnan(iy)) {
            /* a signalling NaN still yields a (quiet) NaN where the result would be 1 */
            if(2u * iy == 0u) return 2u * (ix ^ 0x00400000u) > 2u * 0x7fc00000u ? x + y : 1.0f;
            if(ix == 0x3f800000u) return 2u * (iy ^ 0x00400000u) > 2u * 0x7fc00000u ? x + y : 1.0f;
            if(2u * ix > 2u * 0x7f800000u || 2u * iy > 2u * 0x7f800000u) return x + y;
            if(2u * ix == 2u * 0x3f800000u) return 1.0f;
            if((2u * ix < 2u * 0x3f800000u) == ((iy & 0x80000000u) == 0u)) return 0.0f;
            return y * y;
        }
        if(gsx_powf_zeroinfnan(ix)) {
            float x2 = x * x;

            if((ix & 0x80000000u) != 0u && gsx_powf_checkint(iy) == 1) x2 = -x2;
            return (iy & 0x80000000u) != 0u ? 1.0f / x2 : x2;
        }
        if((ix & 0x80000000u) != 0u) {
            const int yint = gsx_powf_checkint(iy);

            if(yint == 0) return gsx_f32_from_bits(0x7fc00000u);
            if(yint == 1) sign_bias = 1u << (GSX_EXP2_TABLE_BITS + 11);
            ix &= 0x7fffffffu;
        }
        if(ix < 0x00800000u) {
            ix = gsx_f32_bits(x * 0x1p23f) & 0x7fffffffu;
            ix -= 23u << 23;
        }
    }
    logx = gsx_powf_log2(ix);
    ylogx = (double)y * logx;
    if(((gsx_f64_bits(ylogx) >> 47) & 0xffffu) >= (gsx_f64_bits(126.0) >> 47)) {
        if(ylogx > 0x1.fffffffd1d571p+6) return gsx_f32_from_bits(sign_bias ? 0xff800000u : 0x7f800000u);
        if(ylogx <= -150.0) return sign_bias ? -0.0f : 0.0f;
    }
    return gsx_powf_exp2(ylogx, sign_bias);
}

/* PCG32 as in gsx/src/pcg32.h:41-119 (O'Neill's pcg32 with the tiny-cuda-nn packaging):
 * 64-bit LCG state, XSH-RR output, seeding init(seed, seed) as gsx/src/gsx-random.c:25. */
#define GSX_PCG32_MULT 0x5851f42d4c957f2dULL

typedef struct gsx_amd_pcg32 {
    uint64_t state;
    uint64_t inc;
} gsx_amd_pcg32;

GSX_HD uint32_t gsx_pcg32_next_u32(gsx_amd_pcg32 *rng)
{
    uint64_t old = rng->state;
    uint32_t xorshifted;
    uint32_t rot;

    rng->state = old * GSX_PCG32_MULT + rng->inc;
    xorshifted = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    rot = (uint32_t)(old >> 59u);
    return (xorshifted >> rot) | (xorshifted << ((~rot + 1u) & 31u));
}

GSX_HD void gsx_pcg32_seed2(gsx_amd_pcg32 *rng, uint64_t initstate, uint64_t initseq)
{
    rng->state = 0u;
    rng->inc = (initseq << 1u) | 1u;
    (void)gsx_pcg32_next_u32(rng);
    rng->state += initstate;
    (void)gsx_pcg32_next_u32(rng);
}

GSX_HD float gsx_pcg32_next_f32(gsx_amd_pcg32 *rng)
{
    return gsx_f32_from_bits((gsx_pcg32_next_u32(rng) >> 9u) | 0x3f800000u) - 1.0f;
}

/* Jump ahead by `delta` draws in O(log delta) (Brown, "Random number generation with
 * arbitrary strides", 1994), as pcg32_advance in gsx/src/pcg32.h:103-119. */
GSX_HD void gsx_pcg32_advance(gsx_amd_pcg32 *rng, uint64_t delta)
{
    uint64_t cur_mult = GSX_PCG32_MULT;
    uint64_t cur_plus = rng->inc;
    uint64_t acc_mult = 1u;
    uint64_t acc_plus = 0u;

    while(delta > 0u) {
        if((delta & 1u) != 0u) {
            acc_mult *= cur_mult;
            acc_plus = acc_plus * cur_mult + cur_plus;
        }
        cur_plus = (cur_mult + 1u) * cur_plus;
        cur_mult *= cur_mult;
        delta /= 2u;
    }
    rng->state = acc_mult * rng->state + acc_plus;
}

#endif /* GSX_AMD_MATH_H */
