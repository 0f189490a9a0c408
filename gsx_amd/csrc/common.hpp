// common.hpp - device-side building blocks shared by the gfx950 kernels.
//
// All float arithmetic that decides visibility, footprints or blend contributions follows the
// gsx CPU backend operation by operation (gsx/src/gsx-cpu/render.c:397-1088). The library is
// compiled with -ffp-contract=off, correctly rounded f32 division/sqrt and no denormal flush, so
// each expression below rounds exactly as its CPU counterpart does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gsx_math.h"
#include "tile_cull.h"
#include "../../include/gsx_hip.h"

namespace gsx_amd {

constexpr int kWave = 64;
constexpr int kTile = 16;                    // screen tile edge in pixels
constexpr int kTilePixels = kTile * kTile;   // one workgroup (4 waves) per tile

// Constants of the CPU renderer: render.c:85-111.
constexpr float kShC0 = 0.28209479177387814f;
constexpr float kShC1 = 0.4886025119029199f;
constexpr float kMinAbsZ = 1.0e-8f;
constexpr float kMinQuatNormSq = 1.0e-20f;
constexpr float kCov2dDilation = 0.3f;
constexpr float kPowerThreshold = -4.5f;
constexpr float kMinAlpha = 1.0f / 255.0f;
constexpr float kOpacityLogitCull = -5.537334267018537f;
constexpr float kMaxFragmentAlpha = 0.999f;
constexpr float kTransmittanceThreshold = 1.0e-4f;

__device__ __constant__ const float kShC2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                                                -1.0925484305920792f, 0.5462742152960396f};
__device__ __constant__ const float kShC3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                                                0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                                                -0.5900435899266435f};

// Camera block shared by every render kernel (passed by value as a kernel argument).
struct CameraParams {
    float w[3][3];      // world-to-camera rotation (render.c:561-581 of the pose quaternion)
    float t[3];         // world-to-camera translation
    float centre[3];    // camera centre in world space, -W^T t (render.c:603-609)
    float fx, fy, cx, cy;
    float near_plane, far_plane;
    float bg[3];
    int32_t width, height;
    int32_t tiles_x, tiles_y;
};

struct Mat3 {
    float m[3][3];
};

// exp_table (optional): an LDS copy of the 32-entry exp table (gsx_exp2_table_entry), in place
// of the global one, for this and the helpers below.
__device__ inline float sigmoid_render(float x, const uint64_t* exp_table = nullptr) {
    // render.c:397-407
    if (x >= 0.0f) {
        float z = gsx_expf_table(-x, exp_table);
        return 1.0f / (1.0f + z);
    }
    float z = gsx_expf_table(x, exp_table);
    return z / (1.0f + z);
}

__device__ inline bool quat_normalize(float qx, float qy, float qz, float qw, float& nx, float& ny, float& nz,
                                      float& nw) {
    // render.c:421-451
    float norm_sq = qx * qx + qy * qy + qz * qz + qw * qw;
    if (norm_sq <= kMinQuatNormSq) {
        nx = 0.0f;
        ny = 0.0f;
        nz = 0.0f;
        nw = 1.0f;
        return false;
    }
    float inv_norm = 1.0f / sqrtf(norm_sq);
    nx = qx * inv_norm;
    ny = qy * inv_norm;
    nz = qz * inv_norm;
    nw = qw * inv_norm;
    return true;
}

__device__ inline Mat3 rotation_from_xyzw(float qx_raw, float qy_raw, float qz_raw, float qw_raw) {
    // render.c:561-581
    float qx, qy, qz, qw;
    (void)quat_normalize(qx_raw, qy_raw, qz_raw, qw_raw, qx, qy, qz, qw);
    Mat3 r;
    r.m[0][0] = 1.0f - 2.0f * (qy * qy + qz * qz);
    r.m[0][1] = 2.0f * (qx * qy - qw * qz);
    r.m[0][2] = 2.0f * (qx * qz + qw * qy);
    r.m[1][0] = 2.0f * (qx * qy + qw * qz);
    r.m[1][1] = 1.0f - 2.0f * (qx * qx + qz * qz);
    r.m[1][2] = 2.0f * (qy * qz - qw * qx);
    r.m[2][0] = 2.0f * (qx * qz - qw * qy);
    r.m[2][1] = 2.0f * (qy * qz + qw * qx);
    r.m[2][2] = 1.0f - 2.0f * (qx * qx + qy * qy);
    return r;
}

// Zero-initialised triple loop product (render.c:543-559): r = ((0 + a0 b0) + a1 b1) + a2 b2.
__device__ inline Mat3 mat3_mul(const Mat3& a, const Mat3& b) {
    Mat3 r;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) acc += a.m[i][k] * b.m[k][j];
            r.m[i][j] = acc;
        }
    }
    return r;
}

// a * b^T with the same accumulation order as mat3_mul(a, transpose(b)).
__device__ inline Mat3 mat3_mul_t(const Mat3& a, const Mat3& b) {
    Mat3 r;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 3; ++k) acc += a.m[i][k] * b.m[j][k];
            r.m[i][j] = acc;
        }
    }
    return r;
}

__device__ inline Mat3 camera_rotation(const CameraParams& cam) {
    Mat3 w;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) w.m[i][j] = cam.w[i][j];
    return w;
}

// Result of the per-Gaussian preprocess: the CPU's gsx_cpu_render_visible record
// (render.c:19-39) plus the visibility verdict.
struct Projected {
    bool visible;
    int32_t x_min, x_max, y_min, y_max;
    float mx, my, a, b, c, inv_det, depth, xc, yc, zc;
    float color[3];
    float opacity;
    float dir[3];
};

// Covariance of a Gaussian: Sigma = (R S)(R S)^T with S = diag(exp(logscale)) (render.c:583-601).
__device__ inline Mat3 cov3d_from(const float4 q, const float ls[3], const uint64_t* exp_table = nullptr) {
    Mat3 rs = rotation_from_xyzw(q.x, q.y, q.z, q.w);
    float sx = gsx_expf_table(ls[0], exp_table);
    float sy = gsx_expf_table(ls[1], exp_table);
    float sz = gsx_expf_table(ls[2], exp_table);
#pragma unroll
    for (int row = 0; row < 3; ++row) {
        rs.m[row][0] *= sx;
        rs.m[row][1] *= sy;
        rs.m[row][2] *= sz;
    }
    return mat3_mul_t(rs, rs);
}

// SH colour with the CPU clamp max(c + 0.5, 0) (render.c:730-828). sh1..sh3 are [N,k,3].
__device__ inline void eval_sh(int64_t g, int deg, const float d[3], const float* __restrict__ sh0,
                               const float* __restrict__ sh1, const float* __restrict__ sh2,
                               const float* __restrict__ sh3, float out[3]) {
    float r0 = kShC0 * sh0[g * 3 + 0];
    float r1 = kShC0 * sh0[g * 3 + 1];
    float r2 = kShC0 * sh0[g * 3 + 2];
    if (deg >= 1) {
        const float x = d[0], y = d[1], z = d[2];
        const float* c1 = sh1 + g * 9;
        float s0 = -kShC1 * y, s1 = kShC1 * z, s2 = -kShC1 * x;
        r0 = r0 + c1[0] * s0;
        r1 = r1 + c1[1] * s0;
        r2 = r2 + c1[2] * s0;
        r0 = r0 + c1[3] * s1;
        r1 = r1 + c1[4] * s1;
        r2 = r2 + c1[5] * s1;
        r0 = r0 + c1[6] * s2;
        r1 = r1 + c1[7] * s2;
        r2 = r2 + c1[8] * s2;
        if (deg >= 2) {
            float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
            float basis[5];
            basis[0] = kShC2[0] * xy;
            basis[1] = kShC2[1] * yz;
            basis[2] = kShC2[2] * (2.0f * zz - xx - yy);
            basis[3] = kShC2[3] * xz;
            basis[4] = kShC2[4] * (xx - yy);
            const float* c2 = sh2 + g * 15;
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                r0 = r0 + c2[i * 3 + 0] * basis[i];
                r1 = r1 + c2[i * 3 + 1] * basis[i];
                r2 = r2 + c2[i * 3 + 2] * basis[i];
            }
            if (deg >= 3) {
                float b3[7];
                b3[0] = kShC3[0] * y * (3.0f * xx - yy);
                b3[1] = kShC3[1] * xy * z;
                b3[2] = kShC3[2] * y * (4.0f * zz - xx - yy);
                b3[3] = kShC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
                b3[4] = kShC3[4] * x * (4.0f * zz - xx - yy);
                b3[5] = kShC3[5] * z * (xx - yy);
                b3[6] = kShC3[6] * x * (xx - 3.0f * yy);
                const float* c3 = sh3 + g * 21;
#pragma unroll
                for (int i = 0; i < 7; ++i) {
                    r0 = r0 + c3[i * 3 + 0] * b3[i];
                    r1 = r1 + c3[i * 3 + 1] * b3[i];
                    r2 = r2 + c3[i * 3 + 2] * b3[i];
                }
            }
        }
    }
    out[0] = fmaxf(r0 + 0.5f, 0.0f);
    out[1] = fmaxf(r1 + 0.5f, 0.0f);
    out[2] = fmaxf(r2 + 0.5f, 0.0f);
}

// mean_cam = W mean + t (render.c:611-620), the one sequence of operations that every kernel
// uses for it (so a pre-test and the full projection see the same camera-space mean).
__device__ inline void camera_space_mean(float mx, float my, float mz, const CameraParams& cam, float& xc, float& yc,
                                         float& zc) {
    const Mat3 w = camera_rotation(cam);
    xc = w.m[0][0] * mx + w.m[0][1] * my + w.m[0][2] * mz;
    yc = w.m[1][0] * mx + w.m[1][1] * my + w.m[1][2] * mz;
    zc = w.m[2][0] * mx + w.m[2][1] * my + w.m[2][2] * mz;
    xc = xc + cam.t[0];
    yc = yc + cam.t[1];
    zc = zc + cam.t[2];
}

// One Gaussian through the CPU's visibility culls, EWA projection, pixel box and colour
// (render.c:850-1016 per entry; projection :611-668, box :670-694).
__device__ inline Projected preprocess_one(int64_t g, const float* __restrict__ mean3d,
                                           const float* __restrict__ rotation, const float* __restrict__ logscale,
                                           const float* __restrict__ opacity, const float* __restrict__ sh0,
                                           const float* __restrict__ sh1, const float* __restrict__ sh2,
                                           const float* __restrict__ sh3, int sh_degree, const CameraParams& cam,
                                           bool want_color, const uint64_t* exp_table = nullptr) {
    Projected p;
    p.visible = false;
    const float raw_op = opacity[g];
    if (raw_op <= kOpacityLogitCull) return p;
    const float mx = mean3d[g * 3 + 0], my = mean3d[g * 3 + 1], mz = mean3d[g * 3 + 2];
    const float4 q = reinterpret_cast<const float4*>(rotation)[g];
    const float ls[3] = {logscale[g * 3 + 0], logscale[g * 3 + 1], logscale[g * 3 + 2]};
    const Mat3 cov3d = cov3d_from(q, ls, exp_table);
    const Mat3 w = camera_rotation(cam);
    float xc, yc, zc;
    camera_space_mean(mx, my, mz, cam, xc, yc, zc);
    const Mat3 cov_cam = mat3_mul_t(mat3_mul(w, cov3d), w);
    if (fabsf(zc) < kMinAbsZ) return p;
    const float inv_z = 1.0f / zc;
    const float inv_z2 = inv_z * inv_z;
    const float j00 = cam.fx * inv_z;
    const float j02 = -cam.fx * xc * inv_z2;
    const float j11 = cam.fy * inv_z;
    const float j12 = -cam.fy * yc * inv_z2;
    const float jc00 = j00 * cov_cam.m[0][0] + j02 * cov_cam.m[2][0];
    const float jc01 = j00 * cov_cam.m[0][1] + j02 * cov_cam.m[2][1];
    const float jc02 = j00 * cov_cam.m[0][2] + j02 * cov_cam.m[2][2];
    const float jc11 = j11 * cov_cam.m[1][1] + j12 * cov_cam.m[2][1];
    const float jc12 = j11 * cov_cam.m[1][2] + j12 * cov_cam.m[2][2];
    p.mx = cam.fx * xc * inv_z + cam.cx;
    p.my = cam.fy * yc * inv_z + cam.cy;
    p.a = jc00 * j00 + jc02 * j02 + kCov2dDilation;
    p.b = jc01 * j11 + jc02 * j12;
    p.c = jc11 * j11 + jc12 * j12 + kCov2dDilation;
    p.depth = zc;
    p.xc = xc;
    p.yc = yc;
    p.zc = zc;
    const float det = p.a * p.c - p.b * p.b;
    if (p.depth < cam.near_plane || p.depth > cam.far_plane || det <= 0.0f) return p;
    {
        const float trace = p.a + p.c;
        const float det2 = p.a * p.c - p.b * p.b;
        const float disc = sqrtf(fmaxf(0.0f, trace * trace * 0.25f - det2));
        const float l1 = trace * 0.5f + disc;
        const float l2 = trace * 0.5f - disc;
        const float radius = 3.0f * sqrtf(fmaxf(l1, l2));
        p.x_min = (int32_t)fmaxf(0.0f, floorf(p.mx - radius));
        p.x_max = (int32_t)fminf((float)(cam.width - 1), ceilf(p.mx + radius));
        p.y_min = (int32_t)fmaxf(0.0f, floorf(p.my - radius));
        p.y_max = (int32_t)fminf((float)(cam.height - 1), ceilf(p.my + radius));
    }
    if (p.x_min > p.x_max || p.y_min > p.y_max) return p;
    p.visible = true;
    p.inv_det = 1.0f / det;
    p.opacity = sigmoid_render(raw_op, exp_table);
    if (want_color) {
        // render.c:487-496 normalise(mean - centre)
        float dx = mx - cam.centre[0], dy = my - cam.centre[1], dz = mz - cam.centre[2];
        float len = sqrtf(dx * dx + dy * dy + dz * dz);
        if (len <= 0.0f) {
            p.dir[0] = 0.0f;
            p.dir[1] = 0.0f;
            p.dir[2] = 0.0f;
        } else {
            float s = 1.0f / len;
            p.dir[0] = dx * s;
            p.dir[1] = dy * s;
            p.dir[2] = dz * s;
        }
        eval_sh(g, sh_degree, p.dir, sh0, sh1, sh2, sh3, p.color);
    }
    return p;
}

// The part of preprocess_one's projection that the projection backward uses for a Gaussian
// already known visible: the camera-space mean, the view direction and the clamped SH colour,
// by the same operations in the same order (so the same values).
struct ProjectedView {
    bool visible;
    float xc, yc, zc;
    float color[3];
    float dir[3];
};

__device__ inline ProjectedView project_view(int64_t g, const float* __restrict__ mean3d,
                                             const float* __restrict__ sh0, const float* __restrict__ sh1,
                                             const float* __restrict__ sh2, const float* __restrict__ sh3,
                                             int sh_degree, const CameraParams& cam) {
    ProjectedView p;
    p.visible = true;
    const float mx = mean3d[g * 3 + 0], my = mean3d[g * 3 + 1], mz = mean3d[g * 3 + 2];
    camera_space_mean(mx, my, mz, cam, p.xc, p.yc, p.zc);
    const float dx = mx - cam.centre[0], dy = my - cam.centre[1], dz = mz - cam.centre[2];
    const float len = sqrtf(dx * dx + dy * dy + dz * dz);
    if (len <= 0.0f) {
        p.dir[0] = 0.0f;
        p.dir[1] = 0.0f;
        p.dir[2] = 0.0f;
    } else {
        const float s = 1.0f / len;
        p.dir[0] = dx * s;
        p.dir[1] = dy * s;
        p.dir[2] = dz * s;
    }
    eval_sh(g, sh_degree, p.dir, sh0, sh1, sh2, sh3, p.color);
    return p;
}

// ---- wave64 helpers ------------------------------------------------------------------------

// Mask of the active lanes whose p is true. A bool that the compiler already holds as a lane
// mask is copied with scalar instructions (HIP's __ballot compares an integer and spends two
// vector instructions on it).
__device__ inline uint64_t wave_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// True when no active lane has p: the mask is pinned in scalar registers first, so the test is a
// scalar compare (a branch on `ballot == 0` is otherwise selected as a vector select + compare).
__device__ inline bool wave_none(bool p) {
    uint64_t m = __builtin_amdgcn_ballot_w64(p);
    asm volatile("" : "+s"(m));
    return m == 0ull;
}

// True when mask (a ballot) has no lane set; the mask is pinned to scalar registers so the test
// is one scalar compare.
__device__ inline bool mask_none(uint64_t m) {
    asm volatile("" : "+s"(m));
    return m == 0ull;
}

__device__ inline uint64_t lanemask_lt() {
    const uint32_t lane = __lane_id();
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Slot of each lane with `take` in a list whose length is *count: one atomic add per wave (by
// the lowest taking lane, a vector atomic) instead of one per lane; every lane of the wave must
// call it. Lanes without `take` get an unspecified value.
__device__ inline uint32_t wave_append_slot(uint32_t* count, bool take) {
    const uint64_t mask = __ballot(take);
    if (mask == 0ull) return 0u;
    const uint32_t leader = (uint32_t)__builtin_ctzll(mask);
    uint32_t base = 0u;
    if (__lane_id() == leader) base = atomicAdd(count, (uint32_t)__popcll(mask));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, (int)leader);
    return base + (uint32_t)__popcll(mask & lanemask_lt());
}

// Inclusive prefix sum over the 64 lanes of a wave (DPP row shifts, then the two row broadcasts);
// every lane must be active.
__device__ inline uint32_t wave_inclusive_sum_u32(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

__device__ inline uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, off, kWave);
        v = o < v ? o : v;
    }
    return v;
}

// Orders the LDS accesses of one wave around this point (the lanes of a wave exchange data
// through LDS without a workgroup barrier).
__device__ inline void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Sum over the 64 lanes of a wave with DPP lane moves only (no LDS traffic): quad swaps, the
// half-row and row mirrors leave each 16-lane row's sum in all its lanes, then two row
// broadcasts carry rows 0-2 into row 3. Every lane must be active. The total is returned as a
// wave-uniform value (read from lane 63).
template <int kCtrl, int kRowMask>
__device__ inline float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, kRowMask, 0xf,
                                                                 false));
}

__device__ inline float wave_reduce_sum(float v) {
    v += dpp_move<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_move<0x140, 0xf>(v);  // row_mirror
    v += dpp_move<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_move<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// wave_reduce_sum for unsigned integers (wraps modulo 2^32; every lane must be active).
template <int kCtrl, int kRowMask>
__device__ inline uint32_t dpp_move_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, kRowMask, 0xf, false);
}

__device__ inline uint32_t wave_reduce_sum_u32(uint32_t v) {
    v += dpp_move_u32<0xb1, 0xf>(v);
    v += dpp_move_u32<0x4e, 0xf>(v);
    v += dpp_move_u32<0x141, 0xf>(v);
    v += dpp_move_u32<0x140, 0xf>(v);
    v += dpp_move_u32<0x142, 0xa>(v);
    v += dpp_move_u32<0x143, 0xc>(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Row totals (over the 16 lanes of each DPP row) of v[0..8], scattered over the row: the returned
// value of lane l (l = lane index within its row) is the row total of v[(l >> 1) & 7], and
// total8 receives the row total of v[8] in every lane. Each step pairs every lane with a partner
// whose lane-group bit differs and halves the values a lane carries: the lane keeps one half and
// sends its partner the other (two lane-constant selects), and adds what the partner sent (one
// fused DPP add). Partners: row rotate by 8 (l ^ 8, group bit 3), row half mirror (l ^ 7 within
// each 8-lane half, group bit 2), quad permute l ^ 2 (bit 1), then l ^ 1 adds the last value:
// 22 lane operations for the 8 values instead of 32, plus 4 for v[8], and 8 lanes of a row hold
// the 8 totals, so one store writes them all.
__device__ inline float row_reduce_scatter9(const float (&v)[9], float& total8) {
    // lane-constant predicates from constant lane masks (scalar moves; (l & 8) != 0 etc. would be
    // recomputed with vector instructions wherever scalar registers run short)
    const bool b3 = __builtin_amdgcn_inverse_ballot_w64(0xff00ff00ff00ff00ull);  // lane bit 3
    const bool b2 = __builtin_amdgcn_inverse_ballot_w64(0xf0f0f0f0f0f0f0f0ull);  // lane bit 2
    const bool b1 = __builtin_amdgcn_inverse_ballot_w64(0xccccccccccccccccull);  // lane bit 1
    float b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // lanes 0-7 of the row keep v[i], lanes 8-15 keep v[4 + i]
        const float keep = b3 ? v[4 + i] : v[i];
        const float send = b3 ? v[i] : v[4 + i];
        b[i] = keep + dpp_move<0x128, 0xf>(send);  // row_ror:8
    }
    float c[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        // lanes with bit 2 clear keep b[i], the others b[2 + i]
        const float keep = b2 ? b[2 + i] : b[i];
        const float send = b2 ? b[i] : b[2 + i];
        c[i] = keep + dpp_move<0x141, 0xf>(send);  // row_half_mirror
    }
    const float keep = b1 ? c[1] : c[0];
    const float send = b1 ? c[0] : c[1];
    float d = keep + dpp_move<0x4e, 0xf>(send);  // quad_perm [2,3,0,1]
    d += dpp_move<0xb1, 0xf>(d);                 // quad_perm [1,0,3,2]
    float t = v[8];
    t += dpp_move<0xb1, 0xf>(t);
    t += dpp_move<0x4e, 0xf>(t);
    t += dpp_move<0x141, 0xf>(t);  // row_half_mirror
    t += dpp_move<0x140, 0xf>(t);  // row_mirror
    total8 = t;
    return d;
}

// n / d rounded to nearest for normal, finite operands whose quotient is normal (no scaling
// steps): a hardware reciprocal refined once, a quotient and one residual correction, all with
// fused multiply-adds (Markstein's sequence).
__device__ inline float div_rn_normal(float n, float d) {
    float y = __builtin_amdgcn_rcpf(d);
    const float e = __builtin_fmaf(-d, y, 1.0f);
    y = __builtin_fmaf(e, y, y);
    const float q = n * y;
    const float r = __builtin_fmaf(-d, q, n);
    return __builtin_fmaf(r, y, q);
}

// Exclusive scan of the 256 per-thread values of a 256-thread workgroup (a wave scan with
// shuffles, then the 4 wave totals through LDS); returns this thread's prefix and the workgroup
// total through `total`. s_wave holds 4 words of LDS. Contains two workgroup barriers.
__device__ inline uint32_t block_exclusive_scan_256(uint32_t v, uint32_t* s_wave, uint32_t& total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        uint32_t o = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += o;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    uint32_t wave_base = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < 256 / kWave; ++w) {
        uint32_t sw = s_wave[w];
        if (w < wave) wave_base += sw;
        total += sw;
    }
    __syncthreads();
    return wave_base + incl - v;
}

// ---- radix sort building blocks shared with render.hip (sort.hip holds the passes) ----------
constexpr int kSortThreads = 256;
constexpr int kChunkWaves = kSortThreads / kWave;  // 4 (upsweep)
// The depth order sorts about a million keys: 2048-key chunks give ~500 workgroups per launch
// (with 4096 a launch has fewer workgroups than the GPU has CUs, one wave per SIMD; 1024 doubles
// the histogram and row-scan work for no gain in the passes)
constexpr int kCompactingChunk = 2048;
constexpr uint64_t kSentinelKey = ~0ull;  // dropped by a pass with drop_sentinel set

// Workgroup -> sort chunk. Consecutive workgroups go round-robin to the 8 XCDs, so workgroup b
// takes chunk (b % 8) * per + b / 8 (per = ceil(chunks / 8)): each XCD holds a contiguous band of
// chunks, and what neighbouring chunks write next to each other (their counts in one histogram
// row, their runs of one digit in the output) meets in the same L2 and leaves it as whole lines.
// The grid has sort_chunk_grid(chunks) workgroups; those past the last chunk exit.
__device__ inline int64_t sort_chunk_of(uint32_t block, int64_t chunks) {
    const int64_t per = (chunks + 7) / 8;
    return (int64_t)(block & 7u) * per + (int64_t)(block >> 3);
}
inline unsigned sort_chunk_grid(int64_t chunks) { return (unsigned)(8 * ((chunks + 7) / 8)); }

template <int kBits, typename KeyT>
__device__ inline uint32_t digit_of(KeyT key, int shift) {
    return (uint32_t)(key >> shift) & ((1u << kBits) - 1u);
}

// Upsweep of one kChunk-key chunk (workgroup `blk` of kSortThreads threads): its digit counts,
// counted in wave-private LDS counters, to hist[digit][blk]. n_dev (may be null): live key
// count, n = min(n, *n_dev); drop_sentinel: keys equal to kSentinelKey are not counted.
// dmask keeps the digit's bits below the sort's end bit (a last pass narrower than kBits). KeyT:
// uint64_t (the depth order and the public sorts) or uint32_t (tile indices).
// Digit histograms of an upsweep workgroup: per wave, kUpsweepCopies<kBits> copies (one per
// group of 64 / copies lanes), so that lanes of one wave that count the same digit in the same
// round mostly add to different words; each copy kBins + 64 / copies words long, so that a digit's
// copies lie on different banks. (Up to 8-bit digits; the depth sort's 512 digits keep one copy.)
template <int kBits>
constexpr int kUpsweepCopies = kBits <= 8 ? 8 : 1;
template <int kBits>
constexpr int kUpsweepCopyWords = (1 << kBits) + (kUpsweepCopies<kBits> > 1 ? 64 / kUpsweepCopies<kBits> : 0);
template <int kBits>
constexpr int kUpsweepHistWords = kChunkWaves * kUpsweepCopies<kBits> * kUpsweepCopyWords<kBits>;

template <int kBits, int kChunk, typename KeyT>
__device__ inline void radix_upsweep_block(uint32_t blk, const KeyT* __restrict__ keys, int64_t n,
                                           const uint32_t* __restrict__ n_dev, bool drop_sentinel, int shift,
                                           int64_t num_chunks, uint32_t* __restrict__ hist,
                                           uint32_t* s_hist, uint32_t dmask = (1u << kBits) - 1u) {
    constexpr int kBins = 1 << kBits;
    constexpr int kCopies = kUpsweepCopies<kBits>;
    constexpr int kCopyWords = kUpsweepCopyWords<kBits>;
    if (n_dev != nullptr) n = min(n, (int64_t)*n_dev);
    const int wave = threadIdx.x / kWave;
    for (int i = threadIdx.x; i < kUpsweepHistWords<kBits>; i += kSortThreads) s_hist[i] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blk * kChunk;
    if (base < n) {  // uniform; a chunk past the live count counts nothing
        // every key of the chunk is loaded before the first count waits on one (no load sits
        // under a branch: lanes past n re-read key n - 1 and count nothing)
        constexpr int kRounds = kChunk / kSortThreads;
        KeyT k[kRounds];
#pragma unroll
        for (int r = 0; r < kRounds; ++r) k[r] = keys[min(base + (int64_t)r * kSortThreads + threadIdx.x, n - 1)];
        uint32_t* my_hist = s_hist + (wave * kCopies + (int)(__lane_id() / (kWave / kCopies))) * kCopyWords;
#pragma unroll
        for (int r = 0; r < kRounds; ++r) {
            const int64_t i = base + (int64_t)r * kSortThreads + threadIdx.x;
            if (i < n && (!drop_sentinel || (uint64_t)k[r] != kSentinelKey))
                atomicAdd(&my_hist[digit_of<kBits>(k[r], shift) & dmask], 1u);
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kBins; d += kSortThreads) {
        uint32_t c = 0;
#pragma unroll
        for (int h = 0; h < kChunkWaves * kCopies; ++h) c += s_hist[h * kCopyWords + d];
        hist[(int64_t)d * num_chunks + blk] = c;
    }
}

// Keys-only stable radix sort (sort.hip) that also drops every key equal to ~0: the first pass
// reads all n keys and moves the others, in input order within each digit, to the front, and
// stores their number in *n_live (overwritten; no initial value needed); the later passes sort that
// many (grids are sized for n, so no host round trip is needed). Output positions >= *n_live
// are not written.
// Its digits are kCompactingRadixBits wide (passes = ceil((end_bit - begin_bit) / 9)), and temp
// holds radix_sort_keys_u64_compacting_temp_bytes(n) bytes.
constexpr int kCompactingRadixBits = 9;
gsx_hip_status radix_sort_keys_u64_compacting(uint64_t* keys, uint64_t* keys_alt, int64_t n, uint32_t* n_live,
                                              int begin_bit, int end_bit, void* temp, int* out_in_alt,
                                              hipStream_t stream);
size_t radix_sort_keys_u64_compacting_temp_bytes(int64_t n);

// Stable LSD radix sort of n u32 tile indices (bits [0, tile_bits)) with their input positions
// as values, in `passes` passes of digit_bits (6, 7 or 8) bits: a tile field of b bits sorts in
// ceil(b / 8) passes of ceil(b / passes) bits, fewer ballots and bins than 8-bit digits (13-bit
// tiles: 2 passes of 7). The first pass reads `tiles` (left unchanged) and no values; the result
// lands in tiles_sorted / vals_sorted (the alternates hold a middle pass). temp holds
// tile_sort_u32_temp_bytes(n) bytes (the 8-bit need, the largest).
gsx_hip_status tile_sort_u32(const uint32_t* tiles, uint32_t* tiles_alt, uint32_t* tiles_sorted, uint32_t* vals_alt,
                             uint32_t* vals_sorted, int64_t n, int tile_bits, int passes, int digit_bits, void* temp,
                             hipStream_t stream);
size_t tile_sort_u32_temp_bytes(int64_t n);

// Exclusive scan of partials[0..count) in place, the total stored at [count], by one workgroup;
// with arrays > 1, the arrays of count + 1 entries that follow it too (one workgroup each).
gsx_hip_status scan_partials_in_place(uint32_t* partials, int64_t count, hipStream_t stream, int arrays = 1);

}  // namespace gsx_amd
