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
 * Every function here is pure IEEE arithmetic and must be compiled without floating-point
 * contraction (-ffp-contract=off): the explicit fma() calls are the only fused operations.
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
