// adc.hip - adaptive density control (default / ABSGS refine and opacity reset) and the
// row gather it is built on, as data-parallel kernels.
//
// The gsx CPU backend (the parity oracle) runs ADC as sequential loops
// (gsx/src/gsx-cpu/adc/default.c:160-527, gsx/src/gsx-cpu/adc.c:380-559):
//   1. grow candidates in index order until the budget max_num_gaussians - n is spent;
//   2. gather rows [0, n) ++ candidates, zero the optimizer moments of the appended rows;
//   3. duplicate (the gathered copy) or split: 2 children at scale / 1.6, opacity
//      1 - sqrt(1 - sigmoid(o)), offsets R * ((s + 1e-5) * N(0,1)) from one sequential pcg32
//      stream, 6 normals (12 uniforms) per split;
//   4. keep rows with sigmoid(o) > threshold, (size OK or not prune_large) and non-degenerate
//      rotation, in order (stable compaction; at least one row survives);
//   5. zero the auxiliary statistics; in a reset window clamp opacity and reset its moments.
// Here each step is a kernel over rows: ranks come from exclusive scans (so "first-come by
// index" becomes rank < budget), and split k draws from the stream advanced by 12 * k, which
// is exactly where the CPU's sequential stream stands at that split. Classification and keep
// decisions use the glibc-exact expf, so counts and row order match the CPU bit for bit.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <new>

#include "../../include/gsx_hip.h"
#include "common.hpp"

namespace gsx_amd {

// Thread-local message behind gsx_hip_last_error_message (defined in abi.hip).
void set_last_error(const char* what);

constexpr int kAdcThreads = 256;

// gsx_sigmoid / gsx_logit (gsx/src/gsx-core.c:2920-2935), used by the ADC (not the renderer's
// two-branch sigmoid).
__device__ inline float adc_sigmoid(float x) { return 1.0f / (1.0f + gsx_expf(-x)); }

// glibc's logf and cosf, bit for bit (the restatements of gsx_math.h)
__device__ inline float adc_logf(float x) { return gsx_logf(x); }
__device__ inline float adc_cosf(float x) { return gsx_cosf(x); }

__device__ inline float adc_prob_to_logit(float p) {
    // gsx/src/gsx-cpu/adc.c:230-240
    float c = p;
    if (c <= 1e-6f) c = 1e-6f;
    if (c >= 1.0f - 1e-6f) c = 1.0f - 1e-6f;
    return adc_logf(c / (1.0f - c));
}

__device__ inline float adc_next_normal(gsx_amd_pcg32* rng) {
    // gsx/src/gsx-random.c:86-112 (cosine branch, two uniforms)
    float u1 = gsx_pcg32_next_f32(rng);
    const float u2 = gsx_pcg32_next_f32(rng);
    u1 = fmaxf(1e-7f, u1);
    const float mag = sqrtf(-2.0f * adc_logf(u1));
    return mag * adc_cosf(2.0f * (float)3.14159265358979323846264338327950288 * u2);
}

// mode: 0 none, 1 duplicate, 2 split (default.c:160-219)
__global__ __launch_bounds__(kAdcThreads) void adc_classify_kernel(int64_t n, gsx_hip_adc_params p,
                                                                   const float* __restrict__ logscale,
                                                                   const float* __restrict__ grad_acc,
                                                                   const float* __restrict__ visible_counter,
                                                                   uint8_t* __restrict__ mode, uint32_t* __restrict__ grow,
                                                                   uint32_t* __restrict__ split) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint8_t m = 0;
    const float counter = visible_counter != nullptr ? visible_counter[i] : 1.0f;
    if (counter > 0.0f) {
        const float g = grad_acc[i] / (counter > 1.0f ? counter : 1.0f);
        const float thr = p.algorithm == 1 ? p.duplicate_absgrad_threshold : p.duplicate_grad_threshold;
        if (g > thr) {
            const float sx = gsx_expf(logscale[i * 3 + 0]);
            const float sy = gsx_expf(logscale[i * 3 + 1]);
            const float sz = gsx_expf(logscale[i * 3 + 2]);
            float mx = sx;
            if (sy > mx) mx = sy;
            if (sz > mx) mx = sz;
            m = mx > p.duplicate_scale_threshold * p.scene_scale ? 2 : 1;
        }
    }
    mode[i] = m;
    grow[i] = m != 0 ? 1u : 0u;
    split[i] = m == 2 ? 1u : 0u;
}

// Rows of a Gaussian set, addressed uniformly: field f has width w[f] floats per row.
struct RowSet {
    float* f[GSX_HIP_ADC_MAX_FIELDS];
    int32_t w[GSX_HIP_ADC_MAX_FIELDS];
    int32_t count;
};

// Appends row src as row n + rank for every granted candidate, zeroes the appended optimizer
// moments, then applies the split mutation (default.c:38-158) to both rows.
__global__ __launch_bounds__(kAdcThreads) void adc_grow_kernel(int64_t n, uint64_t budget, gsx_hip_adc_params p,
                                                               const uint8_t* __restrict__ mode,
                                                               const uint32_t* __restrict__ grow_rank,
                                                               const uint32_t* __restrict__ split_rank, RowSet rows,
                                                               RowSet moments, uint64_t rng_state, uint64_t rng_inc,
                                                               int32_t mean_f, int32_t rot_f, int32_t ls_f,
                                                               int32_t op_f) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint8_t m = mode[i];
    if (m == 0 || (uint64_t)grow_rank[i] >= budget) return;
    const int64_t t = n + (int64_t)grow_rank[i];
    for (int f = 0; f < rows.count; ++f) {
        const int w = rows.w[f];
        for (int c = 0; c < w; ++c) rows.f[f][t * w + c] = rows.f[f][i * w + c];
    }
    for (int f = 0; f < moments.count; ++f) {
        const int w = moments.w[f];
        for (int c = 0; c < w; ++c) moments.f[f][t * w + c] = 0.0f;
    }
    if (m != 2) return;
    float* mean = rows.f[mean_f];
    float* rot = rows.f[rot_f];
    float* ls = rows.f[ls_f];
    float* op = rows.f[op_f];
    float qx = rot[i * 4 + 0], qy = rot[i * 4 + 1], qz = rot[i * 4 + 2], qw = rot[i * 4 + 3];
    const float sx = gsx_expf(ls[i * 3 + 0]), sy = gsx_expf(ls[i * 3 + 1]), sz = gsx_expf(ls[i * 3 + 2]);
    float so = adc_sigmoid(op[i]);
    const float nsx = sx / 1.6f, nsy = sy / 1.6f, nsz = sz / 1.6f;
    gsx_amd_pcg32 rng;
    rng.state = rng_state;
    rng.inc = rng_inc;
    gsx_pcg32_advance(&rng, 12ull * (uint64_t)split_rank[i]);
    const float r1x = adc_next_normal(&rng), r1y = adc_next_normal(&rng), r1z = adc_next_normal(&rng);
    const float r2x = adc_next_normal(&rng), r2y = adc_next_normal(&rng), r2z = adc_next_normal(&rng);
    const float t1x = r1x * (sx + 1e-5f), t1y = r1y * (sy + 1e-5f), t1z = r1z * (sz + 1e-5f);
    const float t2x = r2x * (sx + 1e-5f), t2y = r2y * (sy + 1e-5f), t2z = r2z * (sz + 1e-5f);
    // gsx/src/gsx-cpu/adc.c:290-330
    const float qn = sqrtf(qx * qx + qy * qy + qz * qz + qw * qw);
    if (qn > 1e-8f) {
        const float iq = 1.0f / qn;
        qx *= iq;
        qy *= iq;
        qz *= iq;
        qw *= iq;
    }
    const float m00 = 1.0f - 2.0f * (qy * qy + qz * qz), m01 = 2.0f * (qx * qy - qw * qz),
                m02 = 2.0f * (qx * qz + qw * qy);
    const float m10 = 2.0f * (qx * qy + qw * qz), m11 = 1.0f - 2.0f * (qx * qx + qz * qz),
                m12 = 2.0f * (qy * qz - qw * qx);
    const float m20 = 2.0f * (qx * qz - qw * qy), m21 = 2.0f * (qy * qz + qw * qx),
                m22 = 1.0f - 2.0f * (qx * qx + qy * qy);
    if (so < 0.0f) so = 0.0f;
    if (so > 1.0f - 1e-6f) so = 1.0f - 1e-6f;
    const float sop = 1.0f - sqrtf(1.0f - so);
    const float lx = adc_logf(nsx), ly = adc_logf(nsy), lz = adc_logf(nsz);
    const float lo = adc_prob_to_logit(sop);
    const float mx = mean[i * 3 + 0], my = mean[i * 3 + 1], mz = mean[i * 3 + 2];
    mean[t * 3 + 0] = mx + (m00 * t1x + m01 * t1y + m02 * t1z);
    mean[t * 3 + 1] = my + (m10 * t1x + m11 * t1y + m12 * t1z);
    mean[t * 3 + 2] = mz + (m20 * t1x + m21 * t1y + m22 * t1z);
    ls[t * 3 + 0] = lx;
    ls[t * 3 + 1] = ly;
    ls[t * 3 + 2] = lz;
    op[t] = lo;
    mean[i * 3 + 0] = mx + (m00 * t2x + m01 * t2y + m02 * t2z);
    mean[i * 3 + 1] = my + (m10 * t2x + m11 * t2y + m12 * t2z);
    mean[i * 3 + 2] = mz + (m20 * t2x + m21 * t2y + m22 * t2z);
    ls[i * 3 + 0] = lx;
    ls[i * 3 + 1] = ly;
    ls[i * 3 + 2] = lz;
    op[i] = lo;
}

// default.c:221-273
__global__ __launch_bounds__(kAdcThreads) void adc_keep_kernel(int64_t count, gsx_hip_adc_params p, int prune_large,
                                                               const float* __restrict__ opacity,
                                                               const float* __restrict__ logscale,
                                                               const float* __restrict__ rotation,
                                                               uint32_t* __restrict__ keep) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float o = adc_sigmoid(opacity[i]);
    const bool not_transparent = o > p.pruning_opacity_threshold;
    const float sx = gsx_expf(logscale[i * 3 + 0]), sy = gsx_expf(logscale[i * 3 + 1]),
                sz = gsx_expf(logscale[i * 3 + 2]);
    float mx = sx;
    if (sy > mx) mx = sy;
    if (sz > mx) mx = sz;
    bool not_large_ws = true;
    if (p.max_world_scale > 0.0f) not_large_ws = mx < (p.max_world_scale * p.scene_scale);
    const float rn = fabsf(rotation[i * 4 + 0]) + fabsf(rotation[i * 4 + 1]) + fabsf(rotation[i * 4 + 2]) +
                     fabsf(rotation[i * 4 + 3]);
    const bool not_degenerate = rn > 1.1920928955078125e-07f;  // FLT_EPSILON
    keep[i] = (not_transparent && (not_large_ws || !prune_large) && not_degenerate) ? 1u : 0u;
}

// out row rank[i] = row i for every kept row (stable compaction of all fields and moments)
__global__ __launch_bounds__(kAdcThreads) void adc_compact_kernel(int64_t count, const uint32_t* __restrict__ keep,
                                                                  const uint32_t* __restrict__ rank, RowSet src,
                                                                  RowSet dst, int force_first) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    int64_t t;
    if (force_first) {
        if (i != 0) return;
        t = 0;
    } else {
        if (!keep[i]) return;
        t = rank[i];
    }
    for (int f = 0; f < src.count; ++f) {
        const int w = src.w[f];
        for (int c = 0; c < w; ++c) dst.f[f][t * w + c] = src.f[f][i * w + c];
    }
}

__global__ __launch_bounds__(kAdcThreads) void adc_reset_opacity_kernel(int64_t count, float max_logit,
                                                                        float* __restrict__ opacity,
                                                                        float* __restrict__ m, float* __restrict__ v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    // gsx_tensor_clamp_inplace(opacity, -FLT_MAX, logit(c)) then the optimizer group reset
    float o = opacity[i];
    if (o < -3.4028234663852886e+38f) o = -3.4028234663852886e+38f;
    if (o > max_logit) o = max_logit;
    opacity[i] = o;
    if (m != nullptr) m[i] = 0.0f;
    if (v != nullptr) v[i] = 0.0f;
}

// ---- MCMC (gsx/src/gsx-cpu/adc/mcmc.c) ---------------------------------------------------------

// mcmc.c:13-18: logistic gate that lets only nearly transparent Gaussians move
__device__ inline float mcmc_noise_gate(float opacity) {
    const float shifted = (1.0f - opacity) - 0.995f;
    return 1.0f / (1.0f + gsx_expf(-100.0f * shifted));
}

// mcmc.c:345-451 for Gaussian i: three normals from draws 6i..6i+5 of the step's stream, shaped
// by R diag(s^2) R^T, scaled by the gate and noise_strength * lr, added to mean3d.
__global__ __launch_bounds__(kAdcThreads) void mcmc_noise_kernel(int64_t n, float noise_lr,
                                                                 float* __restrict__ mean3d,
                                                                 const float* __restrict__ rotation,
                                                                 const float* __restrict__ logscale,
                                                                 const float* __restrict__ opacity,
                                                                 uint64_t rng_state, uint64_t rng_inc) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float op = adc_sigmoid(opacity[i]);
    const float gate = mcmc_noise_gate(op);
    const float sx = gsx_expf(logscale[i * 3 + 0]), sy = gsx_expf(logscale[i * 3 + 1]),
                sz = gsx_expf(logscale[i * 3 + 2]);
    float qx = rotation[i * 4 + 0], qy = rotation[i * 4 + 1], qz = rotation[i * 4 + 2], qw = rotation[i * 4 + 3];
    gsx_amd_pcg32 rng;
    rng.state = rng_state;
    rng.inc = rng_inc;
    gsx_pcg32_advance(&rng, 6ull * (uint64_t)i);
    const float nx = adc_next_normal(&rng), ny = adc_next_normal(&rng), nz = adc_next_normal(&rng);
    const float qn = sqrtf(qx * qx + qy * qy + qz * qz + qw * qw);
    if (qn > 1e-8f) {
        const float iq = 1.0f / qn;
        qx *= iq;
        qy *= iq;
        qz *= iq;
        qw *= iq;
    }
    const float m00 = 1.0f - 2.0f * (qy * qy + qz * qz), m01 = 2.0f * (qx * qy - qw * qz),
                m02 = 2.0f * (qx * qz + qw * qy);
    const float m10 = 2.0f * (qx * qy + qw * qz), m11 = 1.0f - 2.0f * (qx * qx + qz * qz),
                m12 = 2.0f * (qy * qz - qw * qx);
    const float m20 = 2.0f * (qx * qz - qw * qy), m21 = 2.0f * (qy * qz + qw * qx),
                m22 = 1.0f - 2.0f * (qx * qx + qy * qy);
    const float c00 = m00 * m00 * sx * sx + m01 * m01 * sy * sy + m02 * m02 * sz * sz;
    const float c01 = m00 * m10 * sx * sx + m01 * m11 * sy * sy + m02 * m12 * sz * sz;
    const float c02 = m00 * m20 * sx * sx + m01 * m21 * sy * sy + m02 * m22 * sz * sz;
    const float c11 = m10 * m10 * sx * sx + m11 * m11 * sy * sy + m12 * m12 * sz * sz;
    const float c12 = m10 * m20 * sx * sx + m11 * m21 * sy * sy + m12 * m22 * sz * sz;
    const float c22 = m20 * m20 * sx * sx + m21 * m21 * sy * sy + m22 * m22 * sz * sz;
    const float snx = nx * gate * noise_lr, sny = ny * gate * noise_lr, snz = nz * gate * noise_lr;
    mean3d[i * 3 + 0] = mean3d[i * 3 + 0] + (c00 * snx + c01 * sny + c02 * snz);
    mean3d[i * 3 + 1] = mean3d[i * 3 + 1] + (c01 * snx + c11 * sny + c12 * snz);
    mean3d[i * 3 + 2] = mean3d[i * 3 + 2] + (c02 * snx + c12 * sny + c22 * snz);
}

// draw weight sigmoid(opacity) of every row and whether it is dead (mcmc.c:502-511)
__global__ __launch_bounds__(kAdcThreads) void mcmc_weight_kernel(int64_t n, float threshold,
                                                                  const float* __restrict__ opacity,
                                                                  float* __restrict__ weight,
                                                                  uint32_t* __restrict__ dead) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float w = adc_sigmoid(opacity[i]);
    weight[i] = w;
    if (dead != nullptr) dead[i] = w <= threshold ? 1u : 0u;
}

// dead rows in index order to dead_idx, live rows (and their weights) to live_idx / live_w
__global__ __launch_bounds__(kAdcThreads) void mcmc_split_kernel(int64_t n, const uint32_t* __restrict__ dead,
                                                                 const uint32_t* __restrict__ dead_rank,
                                                                 const float* __restrict__ weight,
                                                                 uint32_t* __restrict__ dead_idx,
                                                                 uint32_t* __restrict__ live_idx,
                                                                 float* __restrict__ live_w) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t r = dead_rank[i];
    if (dead[i]) {
        dead_idx[r] = (uint32_t)i;
    } else {
        live_idx[i - r] = (uint32_t)i;
        live_w[i - r] = weight[i];
    }
}

// source row of draw j (through the live list when given) and the per-row draw counts
__global__ __launch_bounds__(kAdcThreads) void mcmc_count_kernel(int64_t draws, const int32_t* __restrict__ sample,
                                                                 const uint32_t* __restrict__ live_idx,
                                                                 uint32_t* __restrict__ src,
                                                                 uint32_t* __restrict__ counts) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= draws) return;
    const uint32_t s = live_idx != nullptr ? live_idx[sample[j]] : (uint32_t)sample[j];
    src[j] = s;
    atomicAdd(&counts[s], 1u);
}

// C(n, k) in double, then float (mcmc.c:20-38)
__device__ inline float mcmc_binom(uint32_t n, uint32_t k) {
    if (k > n) return 0.0f;
    if (k == 0 || k == n) return 1.0f;
    if (k > n - k) k = n - k;
    double v = 1.0;
    for (uint32_t j = 1; j <= k; ++j) v = v * (double)(n - (k - j)) / (double)j;
    return (float)v;
}

// mcmc.c:283-343 for a source row drawn c > 0 times (ratio c + 1, at most 51): the opacity that
// c + 1 copies share, and the scale factor that keeps their summed footprint
__global__ __launch_bounds__(kAdcThreads) void mcmc_relocate_kernel(int64_t n, float min_opacity,
                                                                    const uint32_t* __restrict__ counts,
                                                                    float* __restrict__ opacity,
                                                                    float* __restrict__ logscale) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t c = counts[i];
    if (c == 0u) return;
    const float so = adc_sigmoid(opacity[i]);
    const float sx = gsx_expf(logscale[i * 3 + 0]), sy = gsx_expf(logscale[i * 3 + 1]),
                sz = gsx_expf(logscale[i * 3 + 2]);
    uint32_t ratio = c + 1u;
    if (ratio > 51u) ratio = 51u;
    float clamped = so;
    if (clamped < 0.0f) clamped = 0.0f;
    if (clamped > 1.0f - 1e-6f) clamped = 1.0f - 1e-6f;
    float new_op = 1.0f - gsx_powf(1.0f - clamped, 1.0f / (float)ratio);
    float denom = 0.0f;
    for (uint32_t a = 1; a <= ratio; ++a) {
        for (uint32_t k = 0; k < a; ++k) {
            const float sign = (k % 2u) == 0u ? 1.0f : -1.0f;
            const float coeff = mcmc_binom(a - 1u, k);
            const float power = gsx_powf(new_op, (float)(k + 1u));
            denom += coeff * sign * power / sqrtf((float)(k + 1u));
        }
    }
    const float scale_coeff = fabsf(denom) <= 1e-8f ? 1.0f : so / denom;
    if (new_op < min_opacity) new_op = min_opacity;
    if (new_op > 1.0f - 1e-6f) new_op = 1.0f - 1e-6f;
    opacity[i] = adc_prob_to_logit(new_op);
    logscale[i * 3 + 0] = adc_logf(sx * scale_coeff);
    logscale[i * 3 + 1] = adc_logf(sy * scale_coeff);
    logscale[i * 3 + 2] = adc_logf(sz * scale_coeff);
}

// row dst[j] = row src[j] over the parameter fields (dst = dead_idx for a relocation, or the
// appended rows n + j when dst is null), and the optimizer moments of row zero[j] (the source of
// a relocation, the appended row of a growth) cleared
__global__ __launch_bounds__(kAdcThreads) void mcmc_copy_kernel(int64_t draws, int64_t n,
                                                                const uint32_t* __restrict__ dst,
                                                                const uint32_t* __restrict__ src, RowSet rows,
                                                                RowSet moments, int zero_source_moments) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= draws) return;
    const int64_t s = src[j];
    const int64_t t = dst != nullptr ? (int64_t)dst[j] : n + j;
    for (int f = 0; f < rows.count; ++f) {
        const int w = rows.w[f];
        for (int c = 0; c < w; ++c) rows.f[f][t * w + c] = rows.f[f][s * w + c];
    }
    const int64_t z = zero_source_moments ? s : t;
    for (int f = 0; f < moments.count; ++f) {
        const int w = moments.w[f];
        for (int c = 0; c < w; ++c) moments.f[f][z * w + c] = 0.0f;
    }
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                          int64_t row_bytes, int64_t row_count,
                                                          const int32_t* __restrict__ index, int64_t src_rows,
                                                          int* __restrict__ out_of_range, int word_rows) {
    // word_rows: row_bytes and both base addresses are multiples of 4 (checked by the host)
    const int64_t words_per_row = row_bytes / 4;
    const int64_t total = word_rows ? row_count * words_per_row : row_count * row_bytes;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = word_rows ? e / words_per_row : e / row_bytes;
        const int64_t k = word_rows ? e % words_per_row : e % row_bytes;
        const int32_t s = index[r];
        if (s < 0 || (int64_t)s >= src_rows) {
            if (out_of_range != nullptr) *out_of_range = 1;
            continue;
        }
        if (word_rows) {
            reinterpret_cast<uint32_t*>(dst)[r * words_per_row + k] =
                reinterpret_cast<const uint32_t*>(src)[(int64_t)s * words_per_row + k];
        } else {
            dst[r * row_bytes + k] = src[(int64_t)s * row_bytes + k];
        }
    }
}

}  // namespace gsx_amd

using namespace gsx_amd;

namespace {

unsigned adc_blocks(int64_t n) {
    int64_t b = (n + kAdcThreads - 1) / kAdcThreads;
    return (unsigned)(b < 1 ? 1 : b);
}

gsx_hip_status adc_fail(gsx_hip_status code, const char* what) {
    set_last_error(what);
    return code;
}

#define ADC_HIP_TRY(expr)                                                        \
    do {                                                                         \
        hipError_t e_ = (expr);                                                  \
        if (e_ != hipSuccess) return adc_fail((gsx_hip_status)e_, #expr);        \
    } while (0)

#define ADC_TRY(expr)                          \
    do {                                       \
        gsx_hip_status s_ = (expr);            \
        if (s_ != GSX_HIP_SUCCESS) return s_;  \
    } while (0)

// Grow-only scratch from the stream-ordered pool (pool.hip); an outgrown or released block returns
// to the pool behind the queued work of the stream of the call that last reserved it.
struct Scratch {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipStream_t stream = nullptr;
    gsx_hip_status reserve(size_t need, hipStream_t s) {
        stream = s;
        if (need <= bytes) return GSX_HIP_SUCCESS;
        if (ptr != nullptr) (void)gsx_hip_pool_free(ptr, s);
        ptr = nullptr;
        bytes = 0;
        const size_t grow = need + need / 4 + 4096;
        gsx_hip_status st = gsx_hip_pool_malloc(&ptr, grow, s);
        if (st != GSX_HIP_SUCCESS) return st;
        bytes = grow;
        return GSX_HIP_SUCCESS;
    }
    void release() {
        if (ptr != nullptr) (void)gsx_hip_pool_free(ptr, stream);
        ptr = nullptr;
        bytes = 0;
    }
};

__global__ void adc_count_granted_splits_kernel(int64_t n, uint64_t budget, const uint8_t* __restrict__ mode,
                                                const uint32_t* __restrict__ grow_rank, uint32_t* __restrict__ count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (mode[i] == 2 && (uint64_t)grow_rank[i] < budget) atomicAdd(count, 1u);
}

__global__ void adc_fill_kernel(float* __restrict__ p, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.0f;
}

// not_large_ss of default.c:252-254 for rows that existed before growth
__global__ void adc_screen_scale_kernel(int64_t n_before, float max_screen_scale,
                                        const float* __restrict__ max_screen_radius, uint32_t* __restrict__ keep) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_before) return;
    if (!(max_screen_radius[i] < max_screen_scale)) keep[i] = 0u;
}

bool in_refine_window(const gsx_hip_adc_params& p, uint64_t step) {
    const uint64_t s0 = p.start_refine > 0 ? (uint64_t)p.start_refine : 0;
    const uint64_t s1 = p.end_refine > 0 ? (uint64_t)p.end_refine : 0;
    if (p.refine_every == 0) return false;
    if (step % (uint64_t)p.refine_every != 0) return false;
    return !(step < s0 || step > s1);
}

bool in_reset_window(const gsx_hip_adc_params& p, uint64_t step) {
    const uint64_t s0 = p.start_refine > 0 ? (uint64_t)p.start_refine : 0;
    const uint64_t s1 = p.end_refine > 0 ? (uint64_t)p.end_refine : 0;
    if (p.reset_every == 0) return false;
    if (step % (uint64_t)p.reset_every != 0) return false;
    return !(step < s0 || step >= s1);
}

RowSet param_rows(const gsx_hip_gs_rows& r, int* mean_f, int* rot_f, int* ls_f, int* op_f, bool with_aux) {
    RowSet s{};
    s.count = 0;
    auto add = [&](float* p, int w) {
        if (p != nullptr) {
            s.f[s.count] = p;
            s.w[s.count] = w;
            s.count += 1;
        }
    };
    *mean_f = s.count;
    add(r.mean3d, 3);
    *rot_f = s.count;
    add(r.rotation, 4);
    *ls_f = s.count;
    add(r.logscale, 3);
    *op_f = s.count;
    add(r.opacity, 1);
    add(r.sh0, 3);
    if (r.sh_degree >= 1) add(r.sh1, 9);
    if (r.sh_degree >= 2) add(r.sh2, 15);
    if (r.sh_degree >= 3) add(r.sh3, 21);
    if (with_aux) {
        add(r.grad_acc, 1);
        add(r.absgrad_acc, 1);
        add(r.visible_counter, 1);
        add(r.max_screen_radius, 1);
    }
    return s;
}

RowSet moment_rows(const gsx_hip_gs_rows& r) {
    static const int widths[8] = {3, 4, 3, 1, 3, 9, 15, 21};
    RowSet s{};
    s.count = 0;
    for (int k = 0; k < 8; ++k) {
        if (k >= 5 && r.sh_degree < k - 4) continue;
        if (r.first_moment[k] != nullptr) {
            s.f[s.count] = r.first_moment[k];
            s.w[s.count] = widths[k];
            s.count += 1;
        }
        if (r.second_moment[k] != nullptr) {
            s.f[s.count] = r.second_moment[k];
            s.w[s.count] = widths[k];
            s.count += 1;
        }
    }
    return s;
}

}  // namespace

struct gsx_hip_adc_context {
    gsx_amd_pcg32 rng;
    Scratch scratch;
    uint32_t* host = nullptr;  // pinned readback slots
    float* host_cdf = nullptr;  // pinned draw weights / cumulative sums of the MCMC draws
    size_t host_cdf_floats = 0;
};

namespace {

// MCMC position noise (gsx/src/gsx-cpu/adc/mcmc.c:345-451): none past end_refine or without
// noise strength; otherwise 6 draws per Gaussian from the context's stream.
gsx_hip_status mcmc_noise(gsx_hip_adc_context* ctx, const gsx_hip_adc_params& p, uint64_t global_step,
                          gsx_hip_gs_rows* rows, hipStream_t stream) {
    const int64_t n = rows->count;
    if (!(p.noise_strength > 0.0f) || n <= 0) return GSX_HIP_SUCCESS;
    if (p.end_refine > 0 && global_step >= (uint64_t)p.end_refine) return GSX_HIP_SUCCESS;
    const float noise_lr = p.noise_strength * p.mean3d_learning_rate;
    hipLaunchKernelGGL(mcmc_noise_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n, noise_lr, rows->mean3d,
                       rows->rotation, rows->logscale, rows->opacity, ctx->rng.state, ctx->rng.inc);
    ADC_HIP_TRY(hipGetLastError());
    gsx_pcg32_advance(&ctx->rng, 6ull * (uint64_t)n);
    return GSX_HIP_SUCCESS;
}

// cdf[0..count) = running float sum of max(w, 0) in index order, the exact sums of the CPU
// backend's sampler (mcmc.c:137-140); the weights come from the device, the sums go back.
gsx_hip_status mcmc_cdf(gsx_hip_adc_context* ctx, const float* weight, int64_t count, float* cdf, hipStream_t stream) {
    if ((size_t)count > ctx->host_cdf_floats) {
        if (ctx->host_cdf != nullptr) {
            ADC_HIP_TRY(hipStreamSynchronize(stream));
            (void)hipHostFree(ctx->host_cdf);
            ctx->host_cdf = nullptr;
            ctx->host_cdf_floats = 0;
        }
        const size_t grow = (size_t)count + (size_t)count / 4 + 1024;
        ADC_HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&ctx->host_cdf), grow * sizeof(float), hipHostMallocDefault));
        ctx->host_cdf_floats = grow;
    }
    float* h = ctx->host_cdf;
    ADC_HIP_TRY(hipMemcpyAsync(h, weight, (size_t)count * sizeof(float), hipMemcpyDeviceToHost, stream));
    ADC_HIP_TRY(hipStreamSynchronize(stream));
    float total = 0.0f;
    for (int64_t j = 0; j < count; ++j) {
        total += h[j] > 0.0f ? h[j] : 0.0f;
        h[j] = total;
    }
    if (!(total > 0.0f)) {
        return adc_fail(GSX_HIP_ERROR_INVALID_STATE, "mcmc weighted sampling requires positive opacity mass");
    }
    ADC_HIP_TRY(hipMemcpyAsync(cdf, h, (size_t)count * sizeof(float), hipMemcpyHostToDevice, stream));
    return GSX_HIP_SUCCESS;
}

// MCMC refine (mcmc.c:453-766): relocate the dead rows, then grow; rows are appended in place.
gsx_hip_status mcmc_refine(gsx_hip_adc_context* ctx, const gsx_hip_adc_params& p, gsx_hip_gs_rows* rows,
                           int64_t capacity, int64_t* result_count, int64_t* out_counts, hipStream_t stream) {
    const int64_t n = rows->count;
    // the growth target: floor(n (1 + grow_ratio)) in double, capped at max_num_gaussians
    int64_t target = n;
    if (p.max_num_gaussians > 0 && p.grow_ratio > 0.0f) {
        double t = floor((double)n * (1.0 + (double)p.grow_ratio));
        if (t > (double)p.max_num_gaussians) t = (double)p.max_num_gaussians;
        if (t > (double)n) target = (int64_t)t;
    }
    if (capacity < target) return adc_fail(GSX_HIP_ERROR_OUT_OF_RANGE, "row capacity below the mcmc growth target");
    const int64_t draws_max = n > target - n ? n : target - n;
    // scratch: weight[n] | dead[n] | dead_rank[n+1] | dead_idx[n] | live_idx[n] | live_w[n] |
    //          cdf[n] | sample[draws] | src[draws] | counts[n] | scan temp
    const size_t a = 256;
    auto up = [&](size_t x) { return (x + a - 1) / a * a; };
    size_t off = 0;
    const size_t o_w = off;
    off += up((size_t)n * 4);
    const size_t o_dead = off;
    off += up((size_t)n * 4);
    const size_t o_drank = off;
    off += up((size_t)(n + 1) * 4);
    const size_t o_didx = off;
    off += up((size_t)n * 4);
    const size_t o_lidx = off;
    off += up((size_t)n * 4);
    const size_t o_lw = off;
    off += up((size_t)n * 4);
    const size_t o_cdf = off;
    off += up((size_t)n * 4);
    const size_t o_samp = off;
    off += up((size_t)draws_max * 4);
    const size_t o_src = off;
    off += up((size_t)draws_max * 4);
    const size_t o_cnt = off;
    off += up((size_t)n * 4);
    const size_t o_temp = off;
    off += up(gsx_hip_scan_temp_bytes(n));
    ADC_TRY(ctx->scratch.reserve(off, stream));
    uint8_t* base = static_cast<uint8_t*>(ctx->scratch.ptr);
    float* weight = reinterpret_cast<float*>(base + o_w);
    uint32_t* dead = reinterpret_cast<uint32_t*>(base + o_dead);
    uint32_t* drank = reinterpret_cast<uint32_t*>(base + o_drank);
    uint32_t* didx = reinterpret_cast<uint32_t*>(base + o_didx);
    uint32_t* lidx = reinterpret_cast<uint32_t*>(base + o_lidx);
    float* lw = reinterpret_cast<float*>(base + o_lw);
    float* cdf = reinterpret_cast<float*>(base + o_cdf);
    int32_t* sample = reinterpret_cast<int32_t*>(base + o_samp);
    uint32_t* src = reinterpret_cast<uint32_t*>(base + o_src);
    uint32_t* counts = reinterpret_cast<uint32_t*>(base + o_cnt);
    void* temp = base + o_temp;
    int d0, d1, d2, d3;
    const RowSet prow = param_rows(*rows, &d0, &d1, &d2, &d3, false);
    const RowSet mrow = moment_rows(*rows);

    hipLaunchKernelGGL(mcmc_weight_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n,
                       p.pruning_opacity_threshold, rows->opacity, weight, dead);
    ADC_HIP_TRY(hipGetLastError());
    ADC_TRY(gsx_hip_scan_exclusive_u32(dead, drank, n, temp, stream));
    ADC_HIP_TRY(hipMemcpyAsync(ctx->host, drank + n, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
    ADC_HIP_TRY(hipStreamSynchronize(stream));
    const int64_t dead_count = ctx->host[0];
    out_counts[0] = dead_count;
    if (dead_count == n) {
        return adc_fail(GSX_HIP_ERROR_INVALID_STATE, "mcmc relocate requires at least one live gaussian");
    }
    if (dead_count > 0) {
        const int64_t live = n - dead_count;
        hipLaunchKernelGGL(mcmc_split_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n, dead, drank,
                           weight, didx, lidx, lw);
        ADC_HIP_TRY(hipGetLastError());
        ADC_TRY(mcmc_cdf(ctx, lw, live, cdf, stream));
        ADC_TRY(gsx_hip_multinomial_i32(sample, dead_count, cdf, live, ctx->rng.state, ctx->rng.inc, stream));
        gsx_pcg32_advance(&ctx->rng, (uint64_t)dead_count);
        hipLaunchKernelGGL(adc_fill_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream,
                           reinterpret_cast<float*>(counts), n);
        hipLaunchKernelGGL(mcmc_count_kernel, dim3(adc_blocks(dead_count)), dim3(kAdcThreads), 0, stream, dead_count,
                           sample, lidx, src, counts);
        hipLaunchKernelGGL(mcmc_relocate_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n,
                           p.pruning_opacity_threshold, counts, rows->opacity, rows->logscale);
        hipLaunchKernelGGL(mcmc_copy_kernel, dim3(adc_blocks(dead_count)), dim3(kAdcThreads), 0, stream, dead_count,
                           n, didx, src, prow, mrow, 1);
        ADC_HIP_TRY(hipGetLastError());
        out_counts[2] += dead_count;
    }
    if (target > n) {
        const int64_t growth = target - n;
        hipLaunchKernelGGL(mcmc_weight_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n,
                           p.pruning_opacity_threshold, rows->opacity, weight, nullptr);
        ADC_HIP_TRY(hipGetLastError());
        ADC_TRY(mcmc_cdf(ctx, weight, n, cdf, stream));
        ADC_TRY(gsx_hip_multinomial_i32(sample, growth, cdf, n, ctx->rng.state, ctx->rng.inc, stream));
        gsx_pcg32_advance(&ctx->rng, (uint64_t)growth);
        hipLaunchKernelGGL(adc_fill_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream,
                           reinterpret_cast<float*>(counts), n);
        hipLaunchKernelGGL(mcmc_count_kernel, dim3(adc_blocks(growth)), dim3(kAdcThreads), 0, stream, growth, sample,
                           nullptr, src, counts);
        hipLaunchKernelGGL(mcmc_relocate_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n,
                           p.pruning_opacity_threshold, counts, rows->opacity, rows->logscale);
        hipLaunchKernelGGL(mcmc_copy_kernel, dim3(adc_blocks(growth)), dim3(kAdcThreads), 0, stream, growth, n,
                           nullptr, src, prow, mrow, 0);
        ADC_HIP_TRY(hipGetLastError());
        out_counts[2] += growth;
    }
    *result_count = target;
    // gsx/src/gsx-cpu/adc.c:430-436: the auxiliary statistics restart after a refine
    float* aux[4] = {rows->grad_acc, rows->absgrad_acc, rows->visible_counter, rows->max_screen_radius};
    for (float* a2 : aux) {
        if (a2 != nullptr) {
            hipLaunchKernelGGL(adc_fill_kernel, dim3(adc_blocks(target)), dim3(kAdcThreads), 0, stream, a2, target);
        }
    }
    ADC_HIP_TRY(hipGetLastError());
    return GSX_HIP_SUCCESS;
}

}  // namespace

extern "C" {

gsx_hip_status gsx_hip_adc_context_create(gsx_hip_adc_context** out, uint64_t seed) {
    if (out == nullptr) return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out must be non-null");
    gsx_hip_adc_context* ctx = new (std::nothrow) gsx_hip_adc_context();
    if (ctx == nullptr) return adc_fail(GSX_HIP_ERROR_OUT_OF_MEMORY, "adc context allocation");
    // gsx_pcg32_init(seed) -> pcg32_init(seed, seed) (gsx/src/gsx-random.c:25, gsx-cpu/adc.c:466)
    gsx_pcg32_seed2(&ctx->rng, seed, seed);
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&ctx->host), 4 * sizeof(uint32_t), hipHostMallocDefault);
    if (e != hipSuccess) {
        delete ctx;
        return adc_fail((gsx_hip_status)e, "hipHostMalloc");
    }
    *out = ctx;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_adc_context_destroy(gsx_hip_adc_context* ctx) {
    if (ctx == nullptr) return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context must be non-null");
    ctx->scratch.release();
    if (ctx->host != nullptr) (void)hipHostFree(ctx->host);
    if (ctx->host_cdf != nullptr) (void)hipHostFree(ctx->host_cdf);
    delete ctx;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_adc_step(gsx_hip_adc_context* ctx, const gsx_hip_adc_params* params, uint64_t global_step,
                                gsx_hip_gs_rows* rows, int64_t capacity, gsx_hip_gs_rows* out, int32_t* out_result_in_out,
                                int64_t* out_counts, hipStream_t stream) {
    if (ctx == nullptr || params == nullptr || rows == nullptr || out == nullptr || out_result_in_out == nullptr ||
        out_counts == nullptr) {
        return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "adc arguments must be non-null");
    }
    const gsx_hip_adc_params& p = *params;
    if (p.algorithm != 0 && p.algorithm != 1 && p.algorithm != 2) {
        return adc_fail(GSX_HIP_ERROR_NOT_SUPPORTED, "adc algorithm");
    }
    if (p.algorithm != 2 && !(p.scene_scale > 0.0f)) {
        return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "scene_scale must be positive");
    }
    const int64_t n = rows->count;
    if (rows->mean3d == nullptr || rows->rotation == nullptr || rows->logscale == nullptr || rows->opacity == nullptr ||
        rows->sh0 == nullptr) {
        return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "mean3d, rotation, logscale, opacity, sh0 are required");
    }
    out_counts[0] = out_counts[1] = out_counts[2] = out_counts[3] = 0;
    *out_result_in_out = 0;
    out->count = n;
    gsx_hip_gs_rows* result = rows;
    int64_t result_count = n;
    const bool refine = in_refine_window(p, global_step);
    const bool reset = in_reset_window(p, global_step);
    if (p.algorithm == 2) {
        // gsx/src/gsx-cpu/adc.c:515-547: noise every step, then the refine
        ADC_TRY(mcmc_noise(ctx, p, global_step, rows, stream));
        if (refine && n > 0) ADC_TRY(mcmc_refine(ctx, p, rows, capacity, &result_count, out_counts, stream));
    } else if (refine && n > 0) {
        const float* acc = p.algorithm == 1 ? rows->absgrad_acc : rows->grad_acc;
        if (acc == nullptr) return adc_fail(GSX_HIP_ERROR_NOT_SUPPORTED, "refine requires the grad accumulator");
        const uint64_t cap = p.max_num_gaussians > 0 ? (uint64_t)p.max_num_gaussians : 0;
        const uint64_t budget = cap > (uint64_t)n ? cap - (uint64_t)n : 0;
        const int64_t max_rows = n + (int64_t)budget;
        if (capacity < max_rows) return adc_fail(GSX_HIP_ERROR_OUT_OF_RANGE, "row capacity below count + budget");
        // scratch: mode[n] | grow[n] | grow_rank[n+1] | split[n] | split_rank[n+1] | keep[max] |
        //          keep_rank[max+1] | counter | scan temp
        const size_t a = 256;
        auto up = [&](size_t x) { return (x + a - 1) / a * a; };
        size_t off = 0;
        const size_t o_mode = off;
        off += up((size_t)n);
        const size_t o_grow = off;
        off += up((size_t)n * 4);
        const size_t o_grank = off;
        off += up((size_t)(n + 1) * 4);
        const size_t o_split = off;
        off += up((size_t)n * 4);
        const size_t o_srank = off;
        off += up((size_t)(n + 1) * 4);
        const size_t o_keep = off;
        off += up((size_t)max_rows * 4);
        const size_t o_krank = off;
        off += up((size_t)(max_rows + 1) * 4);
        const size_t o_cnt = off;
        off += a;
        const size_t o_temp = off;
        off += up(gsx_hip_scan_temp_bytes(max_rows > n ? max_rows : n));
        ADC_TRY(ctx->scratch.reserve(off, stream));
        uint8_t* base = static_cast<uint8_t*>(ctx->scratch.ptr);
        uint8_t* mode = base + o_mode;
        uint32_t* grow = reinterpret_cast<uint32_t*>(base + o_grow);
        uint32_t* grank = reinterpret_cast<uint32_t*>(base + o_grank);
        uint32_t* split = reinterpret_cast<uint32_t*>(base + o_split);
        uint32_t* srank = reinterpret_cast<uint32_t*>(base + o_srank);
        uint32_t* keep = reinterpret_cast<uint32_t*>(base + o_keep);
        uint32_t* krank = reinterpret_cast<uint32_t*>(base + o_krank);
        uint32_t* cnt = reinterpret_cast<uint32_t*>(base + o_cnt);
        void* temp = base + o_temp;

        hipLaunchKernelGGL(adc_classify_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n, p,
                           rows->logscale, acc, rows->visible_counter, mode, grow, split);
        ADC_HIP_TRY(hipGetLastError());
        ADC_TRY(gsx_hip_scan_exclusive_u32(grow, grank, n, temp, stream));
        ADC_TRY(gsx_hip_scan_exclusive_u32(split, srank, n, temp, stream));
        hipLaunchKernelGGL(adc_fill_kernel, dim3(1), dim3(64), 0, stream, reinterpret_cast<float*>(cnt), (int64_t)1);
        hipLaunchKernelGGL(adc_count_granted_splits_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n,
                           budget, mode, grank, cnt);
        ADC_HIP_TRY(hipMemcpyAsync(ctx->host, grank + n, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
        ADC_HIP_TRY(hipMemcpyAsync(ctx->host + 1, cnt, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
        ADC_HIP_TRY(hipStreamSynchronize(stream));
        const uint64_t candidates = ctx->host[0];
        const uint64_t grown = candidates < budget ? candidates : budget;
        const uint64_t splits = ctx->host[1];
        int mean_f, rot_f, ls_f, op_f;
        const RowSet prow = param_rows(*rows, &mean_f, &rot_f, &ls_f, &op_f, true);
        const RowSet mrow = moment_rows(*rows);
        if (grown > 0) {
            hipLaunchKernelGGL(adc_grow_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n, budget, p, mode,
                               grank, srank, prow, mrow, ctx->rng.state, ctx->rng.inc, mean_f, rot_f, ls_f, op_f);
            ADC_HIP_TRY(hipGetLastError());
            gsx_pcg32_advance(&ctx->rng, 12ull * splits);
            out_counts[1] = (int64_t)(grown - splits);
            out_counts[2] = (int64_t)splits;
        }
        const int64_t grown_count = n + (int64_t)grown;
        const int prune_large = global_step > (uint64_t)(p.reset_every > 0 ? p.reset_every : 0);
        hipLaunchKernelGGL(adc_keep_kernel, dim3(adc_blocks(grown_count)), dim3(kAdcThreads), 0, stream, grown_count, p,
                           prune_large, rows->opacity, rows->logscale, rows->rotation, keep);
        ADC_HIP_TRY(hipGetLastError());
        if (p.max_screen_scale > 0.0f && rows->max_screen_radius != nullptr && prune_large) {
            hipLaunchKernelGGL(adc_screen_scale_kernel, dim3(adc_blocks(n)), dim3(kAdcThreads), 0, stream, n,
                               p.max_screen_scale, rows->max_screen_radius, keep);
        }
        ADC_TRY(gsx_hip_scan_exclusive_u32(keep, krank, grown_count, temp, stream));
        ADC_HIP_TRY(hipMemcpyAsync(ctx->host + 2, krank + grown_count, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
        ADC_HIP_TRY(hipStreamSynchronize(stream));
        int64_t kept = ctx->host[2];
        const int force_first = kept == 0;
        if (force_first) kept = 1;
        if (kept < grown_count) {
            if (out->mean3d == nullptr || out->rotation == nullptr || out->logscale == nullptr ||
                out->opacity == nullptr || out->sh0 == nullptr) {
                return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out rows are required when rows are pruned");
            }
            out->sh_degree = rows->sh_degree;
            int d0, d1, d2, d3;
            const RowSet orow = param_rows(*out, &d0, &d1, &d2, &d3, true);
            const RowSet omrow = moment_rows(*out);
            if (orow.count != prow.count || omrow.count != mrow.count) {
                return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out rows must bind the same fields as rows");
            }
            hipLaunchKernelGGL(adc_compact_kernel, dim3(adc_blocks(grown_count)), dim3(kAdcThreads), 0, stream,
                               grown_count, keep, krank, prow, orow, force_first);
            hipLaunchKernelGGL(adc_compact_kernel, dim3(adc_blocks(grown_count)), dim3(kAdcThreads), 0, stream,
                               grown_count, keep, krank, mrow, omrow, force_first);
            ADC_HIP_TRY(hipGetLastError());
            out_counts[0] = grown_count - kept;
            result = out;
            *out_result_in_out = 1;
        }
        result_count = kept;
        // gsx/src/gsx-cpu/adc.c:446-452: auxiliary statistics restart after a refine
        float* aux[4] = {result->grad_acc, result->absgrad_acc, result->visible_counter, result->max_screen_radius};
        for (float* a2 : aux) {
            if (a2 != nullptr) {
                hipLaunchKernelGGL(adc_fill_kernel, dim3(adc_blocks(result_count)), dim3(kAdcThreads), 0, stream, a2,
                                   result_count);
            }
        }
        ADC_HIP_TRY(hipGetLastError());
    }
    if (reset && result_count > 0) {
        // default.c:275-314
        float c = p.opacity_clamp_value;
        if (c > 1.0f) c = 1.0f;
        if (c < 1e-6f) c = 1e-6f;
        float cc = c;
        if (cc <= 1e-6f) cc = 1e-6f;
        if (cc >= 1.0f - 1e-6f) cc = 1.0f - 1e-6f;
        const float max_logit = logf(cc / (1.0f - cc));
        hipLaunchKernelGGL(adc_reset_opacity_kernel, dim3(adc_blocks(result_count)), dim3(kAdcThreads), 0, stream,
                           result_count, max_logit, result->opacity, result->first_moment[3], result->second_moment[3]);
        ADC_HIP_TRY(hipGetLastError());
        out_counts[3] = 1;
    }
    result->count = result_count;
    return GSX_HIP_SUCCESS;
}

// Replaces gsx_cuda_gather_rows_kernel_launch (gsx/src/gsx-cuda/internal.h:396-405): out row r =
// src row index[r]. An index outside [0, src_row_count) sets *out_has_out_of_range (device int,
// may be null) and leaves that row unwritten; the host decides when to read the flag, so no
// synchronisation happens here (the CUDA backend syncs per gather, gsx-cuda/buffer.c:1179-1207).
gsx_hip_status gsx_hip_gather_rows_kernel_launch(const void* src, void* dst, int64_t row_bytes, int64_t row_count,
                                                 const int32_t* src_indices, int64_t src_row_count,
                                                 int* out_has_out_of_range, hipStream_t stream) {
    if (row_count <= 0) return GSX_HIP_SUCCESS;
    if (src == nullptr || dst == nullptr || src_indices == nullptr || row_bytes <= 0) {
        return adc_fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "gather arguments must be non-null and sized");
    }
    const bool word_rows = (row_bytes & 3) == 0 && ((reinterpret_cast<uintptr_t>(src) |
                                                      reinterpret_cast<uintptr_t>(dst)) & 3) == 0;
    const int64_t total = word_rows ? row_count * (row_bytes / 4) : row_count * row_bytes;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst),
                       row_bytes, row_count, src_indices, src_row_count, out_has_out_of_range, word_rows ? 1 : 0);
    ADC_HIP_TRY(hipGetLastError());
    return GSX_HIP_SUCCESS;
}

}  // extern "C"
