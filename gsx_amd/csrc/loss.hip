// loss.hip - L1 / MSE pointwise losses and the 11x11 Gaussian-window SSIM, forward and backward.
//
// Semantics follow the gsx CPU backend (gsx/src/gsx-cpu/loss.c:316-709):
//   - the loss map and the prediction gradient are accumulators (+=);
//   - SSIM uses an 11-tap Gaussian window (sigma 1.5), zero padding, C1 = 0.01^2, C2 = 0.03^2;
//   - SSIM forward *sets* the 5-pixel boundary of the loss map to 0 (loss.c:471-481);
//   - the SSIM gradient convolves dm/dmu1, dm/dsigma1^2, dm/dsigma12 (0 at the boundary) and
//     adds -(conv_mu + 2 p conv_s1 + t conv_s12) * grad_scale.
// The CPU evaluates SSIM as a direct 2D sum in float64; here the window is applied as two
// separable 11-tap passes in float32 through LDS (16x16 output tile, 26x26 halo), which is
// within 1e-5 of the float64 value on [0,1] images.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"
#include "../../include/gsx_hip.h"

namespace gsx_amd {

// loss.c:120-132, rounded to float
__device__ __constant__ const float kSsimW[11] = {
    0.001028380123898387f, 0.0075987582094967365f, 0.036000773310661316f, 0.10936068743467331f,
    0.21300552785396576f,  0.26601171493530273f,   0.21300552785396576f,  0.10936068743467331f,
    0.036000773310661316f, 0.0075987582094967365f, 0.001028380123898387f};

constexpr int kSsimTile = 16;
constexpr int kSsimHalo = kSsimTile + 10;  // 26

__global__ __launch_bounds__(256) void l1_forward_kernel(float* __restrict__ map, const float* __restrict__ pred,
                                                         const float* __restrict__ target, int64_t n, float scale) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float d = pred[i] - target[i];
        map[i] += scale * fabsf(d);
    }
}

__global__ __launch_bounds__(256) void l1_backward_kernel(float* __restrict__ grad, const float* __restrict__ pred,
                                                          const float* __restrict__ target, int64_t n,
                                                          float grad_scale) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float d = pred[i] - target[i];
        const float s = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
        grad[i] += s * grad_scale;
    }
}

__global__ __launch_bounds__(256) void mse_forward_kernel(float* __restrict__ map, const float* __restrict__ pred,
                                                          const float* __restrict__ target, int64_t n, float scale) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float d = pred[i] - target[i];
        map[i] += scale * (d * d);
    }
}

__global__ __launch_bounds__(256) void mse_backward_kernel(float* __restrict__ grad, const float* __restrict__ pred,
                                                           const float* __restrict__ target, int64_t n,
                                                           float grad_scale) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float d = pred[i] - target[i];
        grad[i] += 2.0f * d * grad_scale;
    }
}

// One 16x16 output tile of one image plane per workgroup (256 threads).
// Forward: 5 moments (mu_p, mu_t, E[p^2], E[t^2], E[pt]) by a horizontal pass over 26 halo rows
// then a vertical pass; writes the loss map (optionally fused with a preceding L1 term) and the
// three dm maps [3][planes][H][W] consumed by the backward.
__global__ __launch_bounds__(256) void ssim_forward_kernel(float* __restrict__ map, const float* __restrict__ pred,
                                                           const float* __restrict__ target, int32_t height,
                                                           int32_t width, int64_t planes, float scale, float l1_scale,
                                                           int fuse_l1, float* __restrict__ dm) {
    __shared__ float s_p[kSsimHalo][kSsimHalo + 1];
    __shared__ float s_t[kSsimHalo][kSsimHalo + 1];
    __shared__ float s_h[5][kSsimHalo][kSsimTile + 1];
    const int tiles_x = (width + kSsimTile - 1) / kSsimTile;
    const int tile = blockIdx.x;
    const int64_t plane = blockIdx.y;
    const int ox = (tile % tiles_x) * kSsimTile;
    const int oy = (tile / tiles_x) * kSsimTile;
    const float* pp = pred + plane * (int64_t)height * width;
    const float* tp = target + plane * (int64_t)height * width;
    for (int i = threadIdx.x; i < kSsimHalo * kSsimHalo; i += 256) {
        const int hy = i / kSsimHalo, hx = i % kSsimHalo;
        const int y = oy + hy - 5, x = ox + hx - 5;
        float pv = 0.0f, tv = 0.0f;
        if (y >= 0 && y < height && x >= 0 && x < width) {
            pv = pp[(int64_t)y * width + x];
            tv = tp[(int64_t)y * width + x];
        }
        s_p[hy][hx] = pv;
        s_t[hy][hx] = tv;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < kSsimHalo * kSsimTile; i += 256) {
        const int hy = i / kSsimTile, cx = i % kSsimTile;
        float a = 0.0f, b = 0.0f, c = 0.0f, d = 0.0f, e = 0.0f;
#pragma unroll
        for (int k = 0; k < 11; ++k) {
            const float w = kSsimW[k];
            const float pv = s_p[hy][cx + k];
            const float tv = s_t[hy][cx + k];
            a += w * pv;
            b += w * tv;
            c += w * (pv * pv);
            d += w * (tv * tv);
            e += w * (pv * tv);
        }
        s_h[0][hy][cx] = a;
        s_h[1][hy][cx] = b;
        s_h[2][hy][cx] = c;
        s_h[3][hy][cx] = d;
        s_h[4][hy][cx] = e;
    }
    __syncthreads();
    const int lx = threadIdx.x % kSsimTile, ly = threadIdx.x / kSsimTile;
    const int x = ox + lx, y = oy + ly;
    if (x >= width || y >= height) return;
    float mu1 = 0.0f, mu2 = 0.0f, ex2 = 0.0f, ey2 = 0.0f, exy = 0.0f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
        const float w = kSsimW[k];
        mu1 += w * s_h[0][ly + k][lx];
        mu2 += w * s_h[1][ly + k][lx];
        ex2 += w * s_h[2][ly + k][lx];
        ey2 += w * s_h[3][ly + k][lx];
        exy += w * s_h[4][ly + k][lx];
    }
    const float c1 = 0.01f * 0.01f, c2 = 0.03f * 0.03f;
    const float m1s = mu1 * mu1, m2s = mu2 * mu2;
    const float s1 = ex2 - m1s, s2 = ey2 - m2s, s12 = exy - mu1 * mu2;
    const float a = m1s + m2s + c1;
    const float b = s1 + s2 + c2;
    const float ct = 2.0f * mu1 * mu2 + c1;
    const float dt = 2.0f * s12 + c2;
    const float ab = a * b;
    const float ssim = ab == 0.0f ? 1.0f : (ct * dt) / ab;
    const bool boundary = y < 5 || y >= height - 5 || x < 5 || x >= width - 5;
    const int64_t idx = plane * (int64_t)height * width + (int64_t)y * width + x;
    if (map != nullptr) {
        float m = map[idx];
        if (fuse_l1) m += l1_scale * fabsf(s_p[ly + 5][lx + 5] - s_t[ly + 5][lx + 5]);
        map[idx] = boundary ? 0.0f : m + (1.0f - ssim) * scale;
    }
    if (dm != nullptr) {
        const int64_t total = planes * (int64_t)height * width;
        float g_mu = 0.0f, g_s1 = 0.0f, g_s12 = 0.0f;
        if (!(boundary || a == 0.0f || b == 0.0f)) {
            const float aab = a * ab, abb = ab * b;
            g_mu = (2.0f * mu2 * dt) / ab - (2.0f * mu2 * ct) / ab - (2.0f * mu1 * ct * dt) / aab +
                   (2.0f * mu1 * ct * dt) / abb;
            g_s1 = -(ct * dt) / abb;
            g_s12 = (2.0f * ct) / ab;
        }
        dm[idx] = g_mu;
        dm[total + idx] = g_s1;
        dm[2 * total + idx] = g_s12;
    }
}

__global__ __launch_bounds__(256) void ssim_backward_kernel(float* __restrict__ grad, const float* __restrict__ pred,
                                                            const float* __restrict__ target, int32_t height,
                                                            int32_t width, int64_t planes, float grad_scale,
                                                            float l1_grad_scale, int fuse_l1,
                                                            const float* __restrict__ dm) {
    __shared__ float s_m[3][kSsimHalo][kSsimHalo + 1];
    __shared__ float s_h[3][kSsimHalo][kSsimTile + 1];
    const int tiles_x = (width + kSsimTile - 1) / kSsimTile;
    const int tile = blockIdx.x;
    const int64_t plane = blockIdx.y;
    const int ox = (tile % tiles_x) * kSsimTile;
    const int oy = (tile / tiles_x) * kSsimTile;
    const int64_t total = planes * (int64_t)height * width;
    const int64_t pbase = plane * (int64_t)height * width;
    for (int i = threadIdx.x; i < kSsimHalo * kSsimHalo; i += 256) {
        const int hy = i / kSsimHalo, hx = i % kSsimHalo;
        const int y = oy + hy - 5, x = ox + hx - 5;
        float v0 = 0.0f, v1 = 0.0f, v2 = 0.0f;
        if (y >= 0 && y < height && x >= 0 && x < width) {
            const int64_t j = pbase + (int64_t)y * width + x;
            v0 = dm[j];
            v1 = dm[total + j];
            v2 = dm[2 * total + j];
        }
        s_m[0][hy][hx] = v0;
        s_m[1][hy][hx] = v1;
        s_m[2][hy][hx] = v2;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < kSsimHalo * kSsimTile; i += 256) {
        const int hy = i / kSsimTile, cx = i % kSsimTile;
        float a = 0.0f, b = 0.0f, c = 0.0f;
#pragma unroll
        for (int k = 0; k < 11; ++k) {
            const float w = kSsimW[k];
            a += w * s_m[0][hy][cx + k];
            b += w * s_m[1][hy][cx + k];
            c += w * s_m[2][hy][cx + k];
        }
        s_h[0][hy][cx] = a;
        s_h[1][hy][cx] = b;
        s_h[2][hy][cx] = c;
    }
    __syncthreads();
    const int lx = threadIdx.x % kSsimTile, ly = threadIdx.x / kSsimTile;
    const int x = ox + lx, y = oy + ly;
    if (x >= width || y >= height) return;
    float cm = 0.0f, c1 = 0.0f, c12 = 0.0f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
        const float w = kSsimW[k];
        cm += w * s_h[0][ly + k][lx];
        c1 += w * s_h[1][ly + k][lx];
        c12 += w * s_h[2][ly + k][lx];
    }
    const int64_t idx = pbase + (int64_t)y * width + x;
    const float pv = pred[idx], tv = target[idx];
    float g = grad[idx];
    if (fuse_l1) {
        const float d = pv - tv;
        const float s = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
        g += s * l1_grad_scale;
    }
    grad[idx] = g + (-(cm + 2.0f * pv * c1 + tv * c12) * grad_scale);
}

}  // namespace gsx_amd

using namespace gsx_amd;

static unsigned pointwise_blocks(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b > 65536) b = 65536;
    if (b < 1) b = 1;
    return (unsigned)b;
}

extern "C" {

// Replace gsx_cuda_loss_{l1,mse}_f32_{forward,backward}_kernel_launch (gsx-cuda/internal.h:312-343).
gsx_hip_status gsx_hip_loss_l1_f32_forward_kernel_launch(float* loss_map, const float* prediction, const float* target,
                                                     int64_t total_elements, float scale, hipStream_t stream) {
    hipLaunchKernelGGL(l1_forward_kernel, dim3(pointwise_blocks(total_elements)), dim3(256), 0, stream, loss_map,
                       prediction, target, total_elements, scale);
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status gsx_hip_loss_l1_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                      const float* target, int64_t total_elements, float grad_scale,
                                                      hipStream_t stream) {
    hipLaunchKernelGGL(l1_backward_kernel, dim3(pointwise_blocks(total_elements)), dim3(256), 0, stream,
                       grad_prediction, prediction, target, total_elements, grad_scale);
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status gsx_hip_loss_mse_f32_forward_kernel_launch(float* loss_map, const float* prediction, const float* target,
                                                      int64_t total_elements, float scale, hipStream_t stream) {
    hipLaunchKernelGGL(mse_forward_kernel, dim3(pointwise_blocks(total_elements)), dim3(256), 0, stream, loss_map,
                       prediction, target, total_elements, scale);
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status gsx_hip_loss_mse_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                       const float* target, int64_t total_elements, float grad_scale,
                                                       hipStream_t stream) {
    hipLaunchKernelGGL(mse_backward_kernel, dim3(pointwise_blocks(total_elements)), dim3(256), 0, stream,
                       grad_prediction, prediction, target, total_elements, grad_scale);
    return (gsx_hip_status)hipGetLastError();
}

// Replace gsx_cuda_loss_ssim_chw_f32_{forward,backward}_kernel_launch (gsx-cuda/internal.h:344-369).
// ssim_workspace holds the three dm maps: 3 * outer_count * channels * height * width floats.
// l1_scale/l1_grad_scale fuse a preceding L1 term in the same pass (0 disables the fusion);
// the result is bit-identical to running the L1 launcher first.
gsx_hip_status gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(float* loss_map, const float* prediction,
                                                           const float* target, int64_t outer_count, int32_t channels,
                                                           int32_t height, int32_t width, float scale,
                                                           float* ssim_workspace, float l1_scale, int fuse_l1,
                                                           hipStream_t stream) {
    const int64_t planes = outer_count * channels;
    if (planes <= 0 || height <= 0 || width <= 0) return GSX_HIP_ERROR_INVALID_ARGUMENT;
    if (planes > 65535) return GSX_HIP_ERROR_OUT_OF_RANGE;
    const int tiles = ((width + kSsimTile - 1) / kSsimTile) * ((height + kSsimTile - 1) / kSsimTile);
    hipLaunchKernelGGL(ssim_forward_kernel, dim3((unsigned)tiles, (unsigned)planes), dim3(256), 0, stream, loss_map,
                       prediction, target, height, width, planes, scale, l1_scale, fuse_l1, ssim_workspace);
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                            const float* target, int64_t outer_count,
                                                            int32_t channels, int32_t height, int32_t width,
                                                            float grad_scale, const float* ssim_workspace,
                                                            float l1_grad_scale, int fuse_l1, hipStream_t stream) {
    const int64_t planes = outer_count * channels;
    if (planes <= 0 || height <= 0 || width <= 0) return GSX_HIP_ERROR_INVALID_ARGUMENT;
    if (planes > 65535) return GSX_HIP_ERROR_OUT_OF_RANGE;
    const int tiles = ((width + kSsimTile - 1) / kSsimTile) * ((height + kSsimTile - 1) / kSsimTile);
    hipLaunchKernelGGL(ssim_backward_kernel, dim3((unsigned)tiles, (unsigned)planes), dim3(256), 0, stream,
                       grad_prediction, prediction, target, height, width, planes, grad_scale, l1_grad_scale, fuse_l1,
                       ssim_workspace);
    return (gsx_hip_status)hipGetLastError();
}

}  // extern "C"
