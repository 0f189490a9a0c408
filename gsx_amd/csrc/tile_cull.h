/*
 * tile_cull.h - the conservative tile test of key emission, shared by the gfx950 kernels and the
 * CPU restatement in oracle/ (both compile it with -ffp-contract=off and correctly rounded
 * division and square root, so they take the same decision bit for bit).
 *
 * The gsx CPU backend visits every pixel of a Gaussian's 3-sigma box (gsx/src/gsx-cpu/render.c:
 * 1042-1079) and skips the pixel when power < -4.5 or opacity * expf(power) < 1/255, with
 * power = -0.5 * (inv_a dx^2 + 2 inv_b dx dy + inv_c dy^2) in float. A tile of the box whose
 * pixels all fail those tests contributes nothing to the image or to any gradient, so its
 * (tile, Gaussian) instance can be left out of the sort. With
 *   thr    = max(-4.5, ln(1/255) - ln(opacity)) - 1e-3     (per Gaussian; the pixel is skipped
 *            when power < thr + 1e-3, and the 1e-3 dwarfs every float rounding in between),
 *   q_cut  = -2 * thr,
 * a pixel that contributes has its quadratic form q = -2 power at most q_cut. The test keeps,
 * for each tile row of the box, the tiles that hold a pixel column where the set {q <= Q}
 * (Q = q_cut plus an allowance for rounding) meets the row's band of pixel rows: one contiguous
 * run of tiles per row, from a closed form (gsx_tile_band_columns). Every dropped tile's pixels
 * therefore fail a cut.
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

/* Per-Gaussian constants of the row-span test. Every kept tile of a tile row of the box is one
 * contiguous run: the pixel centres of the row's band (its pixel rows within the box) that may
 * receive a contribution lie inside the convex set {q(u, v) <= Q}, whose part over the band
 * projects onto one interval of columns. With q = A u^2 + 2 B u v + C v^2 (A, C > 0,
 * det = A C - B^2 > 0) and D(v) = A Q - det v^2, the set's right boundary at height v is
 * u+(v) = (sqrt(D(v)) - B v) / A, a concave function of v largest at vr = -B sqrt(Q / (det C))
 * (the ellipse's rightmost point), so over the band [v0, v1] it is largest at clamp(vr, v0, v1);
 * by symmetry (q(u, v) = q(-u, -v)) the left boundary is least at -clamp(vr, -v1, -v0) mirrored.
 * The band misses the set exactly when D < 0 at that point.
 *   Q    = q_cut + 1e-5 S + 1e-3, S = A X^2 + 2 |B| X Y + C Y^2 with X, Y the largest |offsets| of
 *          the box's pixel centres from the mean: the kernels' power evaluation at a pixel of the
 *          box is within 4 eps S of the exact form (eps = 2^-24), 1e-5 S covers it 40 times over;
 *   aqs  = A Q (1 + 2^-14 + kappa 2^-19), kappa = A C / det: the rounding of D(v) for |v| within
 *          the set is below (3 + 2 kappa) eps A Q, and the factor adds at least 8 times that, so
 *          the computed D is never below the exact one and sqrt(D) never short;
 *   the remaining roundings (of -B v + sqrt(D), of the product with 1 / A) are below
 *          3 eps (sqrt(kappa) + 1) sqrt(Q / A), and the factor widens the span by at least
 *          2^-15 sqrt(Q / A), 8 times more.
 * A pixel column x is kept when its centre offset fl(fl(x + 0.5) - mx), the value the kernels
 * evaluate, lies in [u-, u+]; fl is monotone, so the kept columns are one interval, found from
 * floor / ceil of mx + u -/+ 0.5 and one exact check on each side. A Gaussian whose form is not
 * positive definite, whose kappa exceeds 2^16 (det then carries more than 1% rounding) or whose
 * mean lies beyond 2^21 pixels, or any non-finite constant, keeps every column of its box:
 * aqs = +inf, det = vr = B = 0 and ra = 1 make every band span the box without a branch. */
typedef struct gsx_tile_span {
    float mx, my; /* mean2d */
    float b;      /* inv_b */
    float ra;     /* 1 / inv_a */
    float det;    /* inv_a inv_c - inv_b^2 */
    float vr;     /* v of the rightmost point of the set */
    float aqs;    /* inv_a Q with the rounding allowance */
} gsx_tile_span;

/* Constants of the Gaussian with conic (inv_a, inv_b, inv_c), activated opacity `opacity` and
 * inclusive pixel box [x0, x1] x [y0, y1]. */
GSX_HD gsx_tile_span gsx_tile_span_make(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity,
    int x0, int x1, int y0, int y1)
{
    gsx_tile_span k;
    const float A = inv_a, B = inv_b, C = inv_c;
    const float dx0 = ((float)x0 + 0.5f) - mx, dx1 = ((float)x1 + 0.5f) - mx;
    const float dy0 = ((float)y0 + 0.5f) - my, dy1 = ((float)y1 + 0.5f) - my;
    const float X = gsx_cull_maxf(gsx_cull_absf(dx0), gsx_cull_absf(dx1));
    const float Y = gsx_cull_maxf(gsx_cull_absf(dy0), gsx_cull_absf(dy1));
    const float S = gsx_cull_absf(A) * X * X + 2.0f * gsx_cull_absf(B) * X * Y + gsx_cull_absf(C) * Y * Y;
    const float Q = gsx_tile_qcut(opacity) + (1e-5f * S + 1e-3f);
    const float ac = A * C;
    const float det = ac - B * B;
    const float kappa = ac / det;
    const float slack = 6.103515625e-05f + kappa * 1.9073486328125e-06f; /* 2^-14 + kappa 2^-19 */

    k.mx = mx;
    k.my = my;
    k.b = B;
    k.ra = 1.0f / A;
    k.det = det;
    k.vr = -B * sqrtf(Q / (det * C));
    k.aqs = (A * Q) * (1.0f + slack);
    /* the comparisons are false for NaN, which therefore keeps every column too */
    if(!(A > 0.0f && C > 0.0f && det > 0.0f && det * 65536.0f >= ac && gsx_cull_absf(mx) < 2097152.0f &&
           gsx_cull_absf(my) < 2097152.0f && gsx_cull_absf(k.vr) <= 3.0e38f && k.aqs <= 3.0e38f && k.ra <= 3.0e38f)) {
        k.b = 0.0f;
        k.ra = 1.0f;
        k.det = 0.0f;
        k.vr = 0.0f;
        k.aqs = __builtin_inff();
    }
    return k;
}

/* The pixel columns [*xa, *xb] of the box [x0, x1] whose centres may receive a contribution in
 * the band of pixel rows [py0, py1] (within the box); *xa > *xb when none. */
GSX_HD void gsx_tile_band_columns(const gsx_tile_span *k, int x0, int x1, int py0, int py1, int *xa, int *xb)
{
    const float v0 = ((float)py0 + 0.5f) - k->my, v1 = ((float)py1 + 0.5f) - k->my;
    const float vh = gsx_cull_clampf(k->vr, v0, v1);
    const float vl = gsx_cull_clampf(k->vr, -v1, -v0);
    const float dh = k->aqs - (k->det * vh) * vh;
    const float dl = gsx_cull_maxf(k->aqs - (k->det * vl) * vl, 0.0f);
    const float uh = (sqrtf(dh) - k->b * vh) * k->ra;
    const float ul = -((sqrtf(dl) - k->b * vl) * k->ra);
    const float sh = (k->mx + uh) - 0.5f, sl = (k->mx + ul) - 0.5f;
    int c;

    if(dh < 0.0f) { /* the band misses the set */
        *xa = 1;
        *xb = 0;
        return;
    }
    /* last column whose centre offset is at most uh */
    if(!(sh < (float)x1)) {
        c = x1;
    } else if(!(sh >= (float)x0 - 1.0f)) {
        c = x0 - 1;
    } else {
        c = (int)floorf(sh);
        if(c + 1 <= x1 && (((float)(c + 1) + 0.5f) - k->mx) <= uh) c += 1;
        if(c >= x0 && !((((float)c + 0.5f) - k->mx) <= uh)) c -= 1;
    }
    *xb = c;
    /* first column whose centre offset is at least ul */
    if(!(sl > (float)x0)) {
        c = x0;
    } else if(!(sl <= (float)x1 + 1.0f)) {
        c = x1 + 1;
    } else {
        c = (int)ceilf(sl);
        if(c - 1 >= x0 && (((float)(c - 1) + 0.5f) - k->mx) >= ul) c -= 1;
        if(c <= x1 && !((((float)c + 0.5f) - k->mx) >= ul)) c += 1;
    }
    *xa = c;
}

/* The pixel rectangle [*xa, *xb] x [*ya, *yb] of the box [x0, x1] x [y0, y1] that holds every
 * pixel centre which may receive a contribution from the Gaussian: the columns from the row-span
 * test with the whole box as one band, the rows from the same test with the roles of x and y
 * exchanged (q(u, v) is the same form with A and C swapped, and the rounding allowances are
 * symmetric in u and v). Empty when *xa > *xb or *ya > *yb. The blend kernels test pixels
 * against this rectangle instead of the 3-sigma box: a pixel outside it fails the CPU's cuts. */
GSX_HD void gsx_contribution_box(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity, int x0,
    int x1, int y0, int y1, int *xa, int *xb, int *ya, int *yb)
{
    const gsx_tile_span kx = gsx_tile_span_make(mx, my, inv_a, inv_b, inv_c, opacity, x0, x1, y0, y1);
    const gsx_tile_span ky = gsx_tile_span_make(my, mx, inv_c, inv_b, inv_a, opacity, y0, y1, x0, x1);

    gsx_tile_band_columns(&kx, x0, x1, y0, y1, xa, xb);
    gsx_tile_band_columns(&ky, y0, y1, x0, x1, ya, yb);
}

/* Nonzero when some pixel centre of the inclusive pixel rectangle [px0, px1] x [py0, py1] may
 * receive a contribution from the Gaussian (the rectangle taken as its box). */
GSX_HD int gsx_tile_may_contribute(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity, int px0,
    int px1, int py0, int py1)
{
    const gsx_tile_span k = gsx_tile_span_make(mx, my, inv_a, inv_b, inv_c, opacity, px0, px1, py0, py1);
    int xa, xb;

    gsx_tile_band_columns(&k, px0, px1, py0, py1, &xa, &xb);
    return xa <= xb;
}

#endif /* GSX_AMD_TILE_CULL_H */
