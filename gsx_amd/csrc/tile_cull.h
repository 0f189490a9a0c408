/*
 * tile_cull.h - the conservative tile test of key emission, shared by the gfx950 kernels and the
 * CPU restatement in oracle/ (both compile it with -ffp-contract=off and IEEE division, so they
 * take the same decision bit for bit).
 *
 * The gsx CPU backend visits every pixel of a Gaussian's 3-sigma box (gsx/src/gsx-cpu/render.c:
 * 1042-1079) and skips the pixel when power < -4.5 or opacity * expf(power) < 1/255, with
 * power = -0.5 * (inv_a dx^2 + 2 inv_b dx dy + inv_c dy^2) in float. A tile of the box whose
 * pixels all fail those tests contributes nothing to the image or to any gradient, so its
 * (tile, Gaussian) instance can be left out of the sort. The test drops an instance only when a
 * bound of power over the whole clipped tile rectangle (continuous, so it covers every pixel
 * centre) lies below the skip threshold with room to spare:
 *   thr    = max(-4.5, ln(1/255) - ln(opacity)) - 1e-3     (per Gaussian; the pixel is skipped
 *            when power < thr + 1e-3, and the 1e-3 dwarfs every float rounding in between),
 *   q_cut  = -2 * thr,
 *   q_min  = minimum of the quadratic form over the rectangle (0 when it holds the centre,
 *            otherwise the least of its four corner values and the values at the edges'
 *            interior stationary points),
 *   margin = 1e-4 * (largest term magnitude over the rectangle) + 1e-3, which exceeds the float
 *            rounding of both q_min and the per-pixel power by orders of magnitude,
 *   drop   iff q_min - margin > q_cut.
 * Then every pixel centre has power <= -0.5 * (q_min - margin) < thr, so it fails a cut.
 */
#ifndef GSX_AMD_TILE_CULL_H
#define GSX_AMD_TILE_CULL_H

#include "gsx_math.h"

/* min / max / |x| / clamp as the IEEE operations (one instruction each, or a free source
 * modifier on the GPU). The test's operands are finite, where these equal the compare-and-select
 * forms; a signed zero can differ, and a zero of either sign leaves every quantity below
 * unchanged. lo <= hi in every clamp. */
#if defined(__HIPCC__)
GSX_HD float gsx_cull_minf(float a, float b) { return __builtin_fminf(a, b); }
GSX_HD float gsx_cull_maxf(float a, float b) { return __builtin_fmaxf(a, b); }
GSX_HD float gsx_cull_absf(float a) { return __builtin_fabsf(a); }
#else
GSX_HD float gsx_cull_minf(float a, float b) { return fminf(a, b); }
GSX_HD float gsx_cull_maxf(float a, float b) { return fmaxf(a, b); }
GSX_HD float gsx_cull_absf(float a) { return fabsf(a); }
#endif
GSX_HD float gsx_cull_clampf(float v, float lo, float hi) { return gsx_cull_minf(gsx_cull_maxf(v, lo), hi); }

/* Natural logarithm of a positive normal float from IEEE operations only, so the CPU and the
 * GPU agree bit for bit: x = m 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s),
 * s = (m - 1) / (m + 1), |s| < 0.172, series to s^11 (relative error below 1e-7). */
GSX_HD float gsx_cull_logf(float x)
{
    uint32_t u = gsx_f32_bits(x);
    int e = (int)((u >> 23) & 0xffu) - 127;
    float m = gsx_f32_from_bits((u & 0x007fffffu) | 0x3f800000u);
    float s, s2, t;

    if(m > 1.41421356f) {
        m = m * 0.5f;
        e += 1;
    }
    s = (m - 1.0f) / (m + 1.0f);
    s2 = s * s;
    t = 1.0f / 11.0f;
    t = t * s2 + 1.0f / 9.0f;
    t = t * s2 + 1.0f / 7.0f;
    t = t * s2 + 1.0f / 5.0f;
    t = t * s2 + 1.0f / 3.0f;
    t = t * s2 + 1.0f;
    return 2.0f * s * t + (float)e * 0.693147180559945f;
}

/* q_cut of the Gaussian with activated opacity `opacity` (> 1/255 for every visible one). */
GSX_HD float gsx_tile_qcut(float opacity)
{
    float thr = -5.54126354f - gsx_cull_logf(opacity); /* ln(1/255) - ln(opacity) */

    if(thr < -4.5f) {
        thr = -4.5f;
    }
    return -2.0f * (thr - 1e-3f);
}

/* Per-Gaussian constants of the test: conic (A, B, C) = (inv_a, inv_b, inv_c), their
 * reciprocals for the edge minima, and q_cut. */
typedef struct gsx_tile_conic {
    float mx, my, A, B, C, rA, rC, qcut;
} gsx_tile_conic;

GSX_HD gsx_tile_conic gsx_tile_conic_make(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity)
{
    gsx_tile_conic k;

    k.mx = mx;
    k.my = my;
    k.A = inv_a;
    k.B = inv_b;
    k.C = inv_c;
    k.rA = 1.0f / inv_a;
    k.rC = 1.0f / inv_c;
    k.qcut = gsx_tile_qcut(opacity);
    return k;
}

/* Nonzero when some pixel centre of the inclusive pixel rectangle [px0, px1] x [py0, py1] (the
 * tile clipped to the Gaussian's box) may receive a contribution from the Gaussian.
 * q(u, v) = A u^2 + 2 B u v + C v^2 is evaluated as fma(C v, v, fma(2 B u, v, (A u) u)); the four
 * corner values are shared by the two edges through each corner, and each edge adds the value at
 * its interior stationary point (clamped to the edge) when the quadratic is convex along it. */
GSX_HD int gsx_tile_conic_test(const gsx_tile_conic *k, int px0, int px1, int py0, int py1)
{
    const float A = k->A, B = k->B, C = k->C, rA = k->rA, rC = k->rC, qcut = k->qcut;
    const float B2 = 2.0f * B;
    const float dx0 = ((float)px0 + 0.5f) - k->mx;
    const float dx1 = ((float)px1 + 0.5f) - k->mx;
    const float dy0 = ((float)py0 + 0.5f) - k->my;
    const float dy1 = ((float)py1 + 0.5f) - k->my;
    const float X = gsx_cull_maxf(gsx_cull_absf(dx0), gsx_cull_absf(dx1));
    const float Y = gsx_cull_maxf(gsx_cull_absf(dy0), gsx_cull_absf(dy1));
    const float scale = gsx_cull_absf(A) * X * X + 2.0f * gsx_cull_absf(B) * X * Y + gsx_cull_absf(C) * Y * Y;
    const float margin = 1e-4f * scale + 1e-3f;
    float au0, au1, bu0, bu1, cv0, cv1, qmin, s, q;

    if(dx0 <= 0.0f && dx1 >= 0.0f && dy0 <= 0.0f && dy1 >= 0.0f) {
        return 1;
    }
    au0 = (A * dx0) * dx0;
    au1 = (A * dx1) * dx1;
    bu0 = B2 * dx0;
    bu1 = B2 * dx1;
    cv0 = C * dy0;
    cv1 = C * dy1;
    /* corners */
    qmin = GSX_FMAF(cv0, dy0, GSX_FMAF(bu0, dy0, au0));
    qmin = gsx_cull_minf(qmin, GSX_FMAF(cv1, dy1, GSX_FMAF(bu0, dy1, au0)));
    qmin = gsx_cull_minf(qmin, GSX_FMAF(cv0, dy0, GSX_FMAF(bu1, dy0, au1)));
    qmin = gsx_cull_minf(qmin, GSX_FMAF(cv1, dy1, GSX_FMAF(bu1, dy1, au1)));
    /* vertical edges u = dx0, dx1: stationary point v = -(B u) / C */
    if(C > 0.0f) {
        s = gsx_cull_clampf(-(B * dx0) * rC, dy0, dy1);
        q = GSX_FMAF(C * s, s, GSX_FMAF(bu0, s, au0));
        qmin = gsx_cull_minf(qmin, q);
        s = gsx_cull_clampf(-(B * dx1) * rC, dy0, dy1);
        q = GSX_FMAF(C * s, s, GSX_FMAF(bu1, s, au1));
        qmin = gsx_cull_minf(qmin, q);
    }
    /* horizontal edges v = dy0, dy1: stationary point u = -(B v) / A */
    if(A > 0.0f) {
        s = gsx_cull_clampf(-(B * dy0) * rA, dx0, dx1);
        q = GSX_FMAF(cv0, dy0, GSX_FMAF(B2 * s, dy0, (A * s) * s));
        qmin = gsx_cull_minf(qmin, q);
        s = gsx_cull_clampf(-(B * dy1) * rA, dx0, dx1);
        q = GSX_FMAF(cv1, dy1, GSX_FMAF(B2 * s, dy1, (A * s) * s));
        qmin = gsx_cull_minf(qmin, q);
    }
    return !(qmin - margin > qcut); /* keeps the instance for NaN input too */
}

GSX_HD int gsx_tile_may_contribute(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity, int px0,
    int px1, int py0, int py1)
{
    const gsx_tile_conic k = gsx_tile_conic_make(mx, my, inv_a, inv_b, inv_c, opacity);

    return gsx_tile_conic_test(&k, px0, px1, py0, py1);
}

#endif /* GSX_AMD_TILE_CULL_H */
