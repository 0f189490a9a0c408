/*
 * scenes.c - seeded synthetic scenes, cameras and targets for the benchmark configurations.
 *
 * Randomness follows gsx's host conventions so the same bytes can be fed to the gsx CPU
 * backend and to the gfx950 path:
 *   - generator: pcg32 seeded as init(seed, seed)        (gsx/src/gsx-random.c:14-29);
 *   - uniform:   (next_u32 >> 9 | 0x3f800000) - 1.0f        (gsx/src/pcg32.h:85-92);
 *   - normal:    Box-Muller, cosine branch, 2 uniforms     (gsx/src/gsx-random.c:86-112).
 * Fields are filled field by field, Gaussian-major within a field, in the order mean3d,
 * rotation, logscale, opacity, sh0. Rotations are 4 normals normalised on the host.
 *
 * Scene kinds (the distributions of the benchmark configurations):
 *   0 "cube":   means U[-extent, extent]^3, logscale U[a, b] or N(a, b), opacity N(mu, sd);
 *   1 "plane":  image-fit init on z = 0 with N(0, 0.01) z-jitter, logit(0.1) opacity;
 *   2 "clusters": 64 anisotropic clusters in [-3, 3]^3 plus 20% on a radius-10 shell.
 * Host code only; no GPU involvement.
 */
#include "gsx_math.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float next_uniform(gsx_amd_pcg32 *rng)
{
    return gsx_pcg32_next_f32(rng);
}

static float next_normal(gsx_amd_pcg32 *rng)
{
    float u1 = gsx_pcg32_next_f32(rng);
    float u2 = gsx_pcg32_next_f32(rng);
    float mag;

    u1 = fmaxf(1e-7f, u1);
    mag = sqrtf(-2.0f * logf(u1));
    return mag * cosf(2.0f * (float)3.14159265358979323846264338327950288 * u2);
}

/* Raw pcg32 stream helpers, used by tests to pin this generator against gsx's own. */
void gsx_scene_pcg32_stream(uint64_t seed, int64_t count, int kind, float *out)
{
    gsx_amd_pcg32 rng;
    int64_t i;

    gsx_pcg32_seed2(&rng, seed, seed);
    for(i = 0; i < count; ++i) {
        out[i] = kind == 0 ? next_uniform(&rng) : next_normal(&rng);
    }
}

static void fill_rotations(gsx_amd_pcg32 *rng, int64_t n, float *rotation)
{
    int64_t i;

    for(i = 0; i < n * 4; ++i) {
        rotation[i] = next_normal(rng);
    }
    for(i = 0; i < n; ++i) {
        float *q = rotation + i * 4;
        float nrm = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);

        if(nrm > 0.0f) {
            q[0] /= nrm;
            q[1] /= nrm;
            q[2] /= nrm;
            q[3] /= nrm;
        } else {
            q[0] = 0.0f;
            q[1] = 0.0f;
            q[2] = 0.0f;
            q[3] = 1.0f;
        }
    }
}

/*
 * params (float[8]) by kind:
 *   kind 0: extent, ls_a, ls_b, ls_is_normal (0 => U[a,b], 1 => N(a,b)), op_mu, op_sd, sh_sd, unused
 *   kind 1: ls_a, ls_b, z_sd, sh_sd, unused...
 *   kind 2: ls_mu, ls_sd, op_sd, sh_sd, shell_fraction, shell_radius, unused...
 */
int gsx_scene_generate(int kind, uint64_t seed, int64_t n, const float *params, float *mean3d, float *rotation,
    float *logscale, float *opacity, float *sh0)
{
    gsx_amd_pcg32 rng;
    int64_t i;

    gsx_pcg32_seed2(&rng, seed, seed);
    if(kind == 0) {
        float extent = params[0];

        for(i = 0; i < n * 3; ++i) {
            mean3d[i] = (next_uniform(&rng) * 2.0f - 1.0f) * extent;
        }
        fill_rotations(&rng, n, rotation);
        for(i = 0; i < n * 3; ++i) {
            if(params[3] != 0.0f) {
                logscale[i] = params[1] + params[2] * next_normal(&rng);
            } else {
                logscale[i] = params[1] + (params[2] - params[1]) * next_uniform(&rng);
            }
        }
        for(i = 0; i < n; ++i) {
            opacity[i] = params[4] + params[5] * next_normal(&rng);
        }
        for(i = 0; i < n * 3; ++i) {
            sh0[i] = params[6] * next_normal(&rng);
        }
        return 0;
    }
    if(kind == 1) {
        float init_logit = logf(0.1f / (1.0f - 0.1f));

        for(i = 0; i < n; ++i) {
            mean3d[i * 3 + 0] = next_uniform(&rng) * 2.0f - 1.0f;
            mean3d[i * 3 + 1] = next_uniform(&rng) * 2.0f - 1.0f;
            mean3d[i * 3 + 2] = params[2] * next_normal(&rng);
        }
        fill_rotations(&rng, n, rotation);
        for(i = 0; i < n * 3; ++i) {
            logscale[i] = params[0] + (params[1] - params[0]) * next_uniform(&rng);
        }
        for(i = 0; i < n; ++i) {
            opacity[i] = init_logit;
        }
        for(i = 0; i < n * 3; ++i) {
            sh0[i] = params[3] * next_normal(&rng);
        }
        return 0;
    }
    if(kind == 2) {
        float centre[64][3];
        float sdev[64][3];
        int64_t shell_count = (int64_t)((double)n * (double)params[4]);
        int c;

        for(c = 0; c < 64; ++c) {
            centre[c][0] = next_uniform(&rng) * 6.0f - 3.0f;
            centre[c][1] = next_uniform(&rng) * 6.0f - 3.0f;
            centre[c][2] = next_uniform(&rng) * 6.0f - 3.0f;
            sdev[c][0] = 0.05f + 0.45f * next_uniform(&rng);
            sdev[c][1] = 0.05f + 0.45f * next_uniform(&rng);
            sdev[c][2] = 0.05f + 0.45f * next_uniform(&rng);
        }
        for(i = 0; i < n; ++i) {
            if(i < n - shell_count) {
                int k = (int)(gsx_pcg32_next_u32(&rng) % 64u);

                mean3d[i * 3 + 0] = centre[k][0] + sdev[k][0] * next_normal(&rng);
                mean3d[i * 3 + 1] = centre[k][1] + sdev[k][1] * next_normal(&rng);
                mean3d[i * 3 + 2] = centre[k][2] + sdev[k][2] * next_normal(&rng);
            } else {
                float x = next_normal(&rng);
                float y = next_normal(&rng);
                float z = next_normal(&rng);
                float r = sqrtf(x * x + y * y + z * z);

                if(r <= 0.0f) {
                    x = 1.0f;
                    r = 1.0f;
                }
                mean3d[i * 3 + 0] = x / r * params[5];
                mean3d[i * 3 + 1] = y / r * params[5];
                mean3d[i * 3 + 2] = z / r * params[5];
            }
        }
        fill_rotations(&rng, n, rotation);
        for(i = 0; i < n * 3; ++i) {
            logscale[i] = params[0] + params[1] * next_normal(&rng);
        }
        for(i = 0; i < n; ++i) {
            opacity[i] = params[2] * next_normal(&rng);
        }
        for(i = 0; i < n * 3; ++i) {
            sh0[i] = params[3] * next_normal(&rng);
        }
        return 0;
    }
    return -1;
}

/* World-to-camera pose of a camera at `eye` looking at `target`, image y down (+z forward,
 * gsx-base.h:207-216). out[7] = qx, qy, qz, qw, tx, ty, tz. */
void gsx_scene_look_at(const float *eye, const float *target, float *out)
{
    double f[3], up[3] = { 0.0, 1.0, 0.0 }, xr[3], yd[3], r[3][3], t[3], tr, qw, qx, qy, qz, s, len;
    int i;

    for(i = 0; i < 3; ++i) f[i] = (double)target[i] - (double)eye[i];
    len = sqrt(f[0] * f[0] + f[1] * f[1] + f[2] * f[2]);
    for(i = 0; i < 3; ++i) f[i] /= len;
    if(fabs(f[1]) > 0.999) {
        up[0] = 0.0;
        up[1] = 0.0;
        up[2] = 1.0;
    }
    /* image down = -(up - (up.f) f) */
    s = up[0] * f[0] + up[1] * f[1] + up[2] * f[2];
    for(i = 0; i < 3; ++i) yd[i] = -(up[i] - s * f[i]);
    len = sqrt(yd[0] * yd[0] + yd[1] * yd[1] + yd[2] * yd[2]);
    for(i = 0; i < 3; ++i) yd[i] /= len;
    /* right = down x forward keeps (right, down, forward) right-handed */
    xr[0] = yd[1] * f[2] - yd[2] * f[1];
    xr[1] = yd[2] * f[0] - yd[0] * f[2];
    xr[2] = yd[0] * f[1] - yd[1] * f[0];
    for(i = 0; i < 3; ++i) {
        r[0][i] = xr[i];
        r[1][i] = yd[i];
        r[2][i] = f[i];
    }
    for(i = 0; i < 3; ++i) {
        t[i] = -(r[i][0] * eye[0] + r[i][1] * eye[1] + r[i][2] * eye[2]);
    }
    /* rotation matrix -> quaternion (Shepperd) */
    tr = r[0][0] + r[1][1] + r[2][2];
    if(tr > 0.0) {
        s = sqrt(tr + 1.0) * 2.0;
        qw = 0.25 * s;
        qx = (r[2][1] - r[1][2]) / s;
        qy = (r[0][2] - r[2][0]) / s;
        qz = (r[1][0] - r[0][1]) / s;
    } else if(r[0][0] > r[1][1] && r[0][0] > r[2][2]) {
        s = sqrt(1.0 + r[0][0] - r[1][1] - r[2][2]) * 2.0;
        qw = (r[2][1] - r[1][2]) / s;
        qx = 0.25 * s;
        qy = (r[0][1] + r[1][0]) / s;
        qz = (r[0][2] + r[2][0]) / s;
    } else if(r[1][1] > r[2][2]) {
        s = sqrt(1.0 + r[1][1] - r[0][0] - r[2][2]) * 2.0;
        qw = (r[0][2] - r[2][0]) / s;
        qx = (r[0][1] + r[1][0]) / s;
        qy = 0.25 * s;
        qz = (r[1][2] + r[2][1]) / s;
    } else {
        s = sqrt(1.0 + r[2][2] - r[0][0] - r[1][1]) * 2.0;
        qw = (r[1][0] - r[0][1]) / s;
        qx = (r[0][2] + r[2][0]) / s;
        qy = (r[1][2] + r[2][1]) / s;
        qz = 0.25 * s;
    }
    out[0] = (float)qx;
    out[1] = (float)qy;
    out[2] = (float)qz;
    out[3] = (float)qw;
    out[4] = (float)t[0];
    out[5] = (float)t[1];
    out[6] = (float)t[2];
}

/* Seeded target image [3, H, W]: kind 0 = U[0,1] noise blurred by a box of (2*radius+1)^2
 * (zero-padded, normalised by the in-image tap count); kind 1 = per channel the sum of
 * `terms` random-frequency/phase sinusoids, normalised to [0, 1]. */
int gsx_scene_target(int kind, uint64_t seed, int32_t width, int32_t height, int32_t param, float *out)
{
    gsx_amd_pcg32 rng;
    int64_t plane = (int64_t)width * (int64_t)height;
    int64_t i;
    int c;

    gsx_pcg32_seed2(&rng, seed, seed);
    if(kind == 0) {
        float *noise = (float *)malloc(sizeof(float) * (size_t)(3 * plane));
        int32_t radius = param;

        if(noise == NULL) return -1;
        for(i = 0; i < 3 * plane; ++i) noise[i] = next_uniform(&rng);
        for(c = 0; c < 3; ++c) {
            int32_t x, y;

            for(y = 0; y < height; ++y) {
                for(x = 0; x < width; ++x) {
                    float acc = 0.0f;
                    int taps = 0;
                    int32_t dx, dy;

                    for(dy = -radius; dy <= radius; ++dy) {
                        for(dx = -radius; dx <= radius; ++dx) {
                            int32_t xx = x + dx, yy = y + dy;

                            if(xx >= 0 && yy >= 0 && xx < width && yy < height) {
                                acc += noise[c * plane + (int64_t)yy * width + xx];
                                taps += 1;
                            }
                        }
                    }
                    out[c * plane + (int64_t)y * width + x] = acc / (float)taps;
                }
            }
        }
        free(noise);
        return 0;
    }
    if(kind == 1) {
        int terms = param;

        for(c = 0; c < 3; ++c) {
            float fx[64], fy[64], ph[64];
            float lo = 1e30f, hi = -1e30f;
            int k;
            int32_t x, y;

            if(terms > 64) terms = 64;
            for(k = 0; k < terms; ++k) {
                fx[k] = (next_uniform(&rng) * 2.0f - 1.0f) * 12.0f;
                fy[k] = (next_uniform(&rng) * 2.0f - 1.0f) * 12.0f;
                ph[k] = next_uniform(&rng) * 6.2831853f;
            }
            for(y = 0; y < height; ++y) {
                for(x = 0; x < width; ++x) {
                    float u = (float)x / (float)width, v = (float)y / (float)height, s = 0.0f;

                    for(k = 0; k < terms; ++k) {
                        s += sinf(6.2831853f * (fx[k] * u + fy[k] * v) + ph[k]);
                    }
                    out[c * plane + (int64_t)y * width + x] = s;
                    if(s < lo) lo = s;
                    if(s > hi) hi = s;
                }
            }
            for(i = 0; i < plane; ++i) {
                out[c * plane + i] = (out[c * plane + i] - lo) / (hi - lo > 0.0f ? hi - lo : 1.0f);
            }
        }
        return 0;
    }
    return -1;
}
