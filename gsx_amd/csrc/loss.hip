// loss.hip - L1 / MSE pointwise losses and the 11x11 Gaussian-window SSIM, forward and backward.
//
// Semantics follow the gsx CPU backend (gsx/src/gsx-cpu/loss.c:316-709):
//   - the loss map and the prediction gradient are accumulators (+=);
//   - SSIM uses an 11-tap Gaussian window (sigma 1.5), zero padding, C1 = 0.01^2, C2 = 0.03^2;
//   - SSIM forward *sets* the 5-pixel boundary of the loss map to 0 (loss.c:471-481);
//   - the SSIM gradient convolves dm/dmu1, dm/dsigma1^2, dm/dsigma12 (0 at the boundary) and
//     adds -(conv_mu + 2 p conv_s1 + t conv_s12) * grad_scale.
// The CPU evaluates SSIM as a direct 2D sum in float64; here the window is applied as two
// separable 11-tap passes of fused multiply-adds in float32 through LDS (32x16 output tile,
// 42x26 halo) over inputs shifted by a per-tile value (against the cancellation in
// E[x^2] - mu^2 on smooth images), which is within 1e-5 of the float64 value on [0,1] images.
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

// One 32-column output tile of one image plane per workgroup, two output rows per thread: 16
// rows (256 threads) for the forward, 32 rows (512 threads) for the backward, whose three-map
// passes leave room for the taller halo (42 halo rows per 32 output rows instead of 26 per 16).
// The window sums use explicit fused multiply-adds: the SSIM bar is a tolerance (the CPU sums in
// float64), unlike the L1 term fused into the same pass, which keeps the L1 kernel's exact
// operations.
constexpr int kSsimTW = 32;
constexpr int kSsimFwdTH = 16, kSsimBwdTH = 32;

// Workgroup -> tile of the plane: consecutive workgroups go round-robin to the 8 XCDs, so each
// XCD takes a contiguous band of tiles and neighbouring tiles' halos meet in the same L2. The
// grid has 8 * ceil(tiles / 8) workgroups per plane; those past the last tile exit.
__device__ inline int ssim_tile_of(int block, int tiles) {
    const int per = (tiles + 7) / 8;
    return (block & 7) * per + (block >> 3);
}
// The halo of a tile is staged in LDS as rows of 48 columns, column j holding image column
// ox - 8 + j (the window needs ox - 5 .. ox + 36, columns 3 .. 44). Rows start 16-byte aligned,
// so the staging stores and the horizontal work items' window reads are whole 16-byte pieces.
constexpr int kSsimInW = 48;
// The horizontal sums are kept as planes of kHH rows of kSsimTW columns, each plane padded by 4
// floats: an unpadded plane is a multiple of 64 floats long, so a read of two planes at one
// position (which the compiler pairs into one instruction) would put both on one bank.
#define GSX_SSIM_TILE(kTH)                                                     \
    constexpr int kSsimTH = (kTH);                                             \
    constexpr int kSsimThreads = kSsimTW * kSsimTH / 2;                        \
    constexpr int kSsimHH = kSsimTH + 10;                                      \
    constexpr int kSsimHPlane = kSsimHH * kSsimTW + 4;
// Output columns per work item of the horizontal passes: each loaded input pixel (and its
// moments) serves 4 outputs, which the item stores as one 16-byte piece per moment.
constexpr int kHCols = 4;
static_assert(kSsimTW / kHCols == 8, "eight horizontal work items per staged row");
// Work item i of a horizontal pass -> its staged row. Each run of 64 items (one wave) covers 8
// rows; its eight 8-lane groups take rows 0, 2, 4, 6, 1, 3, 5, 7 of them. Sixteen lanes reading
// 16 bytes each are served together, and two rows 2 apart (96 floats) fall on disjoint banks
// where two adjacent rows (48 floats) would share a quarter of them (measured on gfx950: adjacent
// rows take twice as long per read). Rows past kHH (the padding of the last wave) are skipped.
__device__ inline int ssim_item_row(int i) {
    const int k = (i >> 3) & 7;
    return 8 * (i >> 6) + (((k & 3) << 1) | (k >> 2));
}

// Fills the staged rows of kPlanes planes (plane c at s + c * kHH * kSsimInW; kHH rows, image rows
// oy - 5 ..) from the image planes src[c] (each already offset to this plane), each value minus
// shift[c]. A position outside the image reads the nearest pixel inside it (clamped row and
// column); the callers never use such a value where it would matter (see each kernel). kVec:
// 16-byte loads, which needs width % 4 == 0 and 16-byte aligned planes (a 4-aligned run of
// columns is then all inside or all outside the image); otherwise one float per load. Every load
// is issued before the first store. In-plane offsets are 32-bit (the launchers check H * W).
template <bool kVec, int kPlanes, int kHH, int kThreads>
__device__ inline void ssim_stage_halo(float* s, const float* const (&src)[kPlanes], int ox, int oy, int height,
                                       int width, const float (&shift)[kPlanes]) {
    constexpr int kPlane = kHH * kSsimInW;
    if constexpr (kVec) {
        constexpr int kChunks = kSsimInW / 4;
        constexpr int kItems = kHH * kChunks;
        constexpr int kRounds = (kItems + kThreads - 1) / kThreads;
        float4 v[kRounds][kPlanes];
#pragma unroll
        for (int u = 0; u < kRounds; ++u) {
            // items past the halo load its last one again, and are not stored
            const int i = min((int)threadIdx.x + kThreads * u, kItems - 1);
            const int hy = i / kChunks, hc = i % kChunks;
            const int y = min(max(oy + hy - 5, 0), height - 1);
            const int x = min(max(ox - 8 + 4 * hc, 0), width - 4);
            const uint32_t j = (uint32_t)y * (uint32_t)width + (uint32_t)x;
#pragma unroll
            for (int c = 0; c < kPlanes; ++c) v[u][c] = *reinterpret_cast<const float4*>(src[c] + j);
        }
#pragma unroll
        for (int u = 0; u < kRounds; ++u) {
            const int i = (int)threadIdx.x + kThreads * u;
            if (i >= kItems) break;
#pragma unroll
            for (int c = 0; c < kPlanes; ++c)
                *reinterpret_cast<float4*>(s + c * kPlane + 4 * i) =
                    make_float4(v[u][c].x - shift[c], v[u][c].y - shift[c], v[u][c].z - shift[c], v[u][c].w - shift[c]);
        }
    } else {
        constexpr int kItems = kHH * kSsimInW;
        constexpr int kRounds = (kItems + kThreads - 1) / kThreads;
        float v[kRounds][kPlanes];
#pragma unroll
        for (int u = 0; u < kRounds; ++u) {
            const int i = min((int)threadIdx.x + kThreads * u, kItems - 1);
            const int hy = i / kSsimInW, hx = i % kSsimInW;
            const int y = min(max(oy + hy - 5, 0), height - 1);
            const int x = min(max(ox - 8 + hx, 0), width - 1);
            const uint32_t j = (uint32_t)y * (uint32_t)width + (uint32_t)x;
#pragma unroll
            for (int c = 0; c < kPlanes; ++c) v[u][c] = src[c][j];
        }
#pragma unroll
        for (int u = 0; u < kRounds; ++u) {
            const int i = (int)threadIdx.x + kThreads * u;
            if (i >= kItems) break;
#pragma unroll
            for (int c = 0; c < kPlanes; ++c) s[c * kPlane + i] = v[u][c] - shift[c];
        }
    }
}

// The 14 staged values of one horizontal work item: its four output columns cx .. cx + 3 (cx a
// multiple of 4) take image columns ox + cx - 5 .. ox + cx + 8, staged columns cx + 3 .. cx + 16,
// read as the five 16-byte pieces at cx .. cx + 19. The reads are volatile so that they stay
// whole 16-byte reads: narrowed to the 14 used values they become pairs of single floats at odd
// offsets, whose lanes share banks (measured: 0.5 to 0.9 bank conflicts per access).
__device__ inline void ssim_row_window(const float* row, int cx, float (&w)[10 + kHCols]) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) const volatile v4f lds_v4f;
    float r[20];
#pragma unroll
    for (int q = 0; q < 5; ++q) {
        const v4f v = *(lds_v4f*)(row + cx + 4 * q);
        r[4 * q] = v.x;
        r[4 * q + 1] = v.y;
        r[4 * q + 2] = v.z;
        r[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int k = 0; k < 10 + kHCols; ++k) w[k] = r[3 + k];
}

// Forward: p and t of the halo in LDS; a horizontal 11-tap pass where each thread forms the
// five moments (p, t, p^2, t^2, p t) of four adjacent output columns from 14 loads per plane;
// then a vertical pass where each thread produces two adjacent output rows from 12 loads per
// moment plane. Writes the loss map (optionally after a fused L1 term) and the three dm maps
// [3][planes][H][W] that the backward convolves.
// The halo is staged one float per load and the shift applied per work item. The backward's
// 16-byte staging, used here, cut this kernel's instructions by a quarter and ran it at 52.7 us
// instead of 62 with a cached target, but a training target comes from HBM (one of many images),
// and with its loads' latency exposed it ran at 65.6 us against this version's 60.0 (metric
// training step, one box): here the larger arithmetic share covers that latency.
__global__ __launch_bounds__(kSsimTW * kSsimFwdTH / 2) void ssim_forward_kernel(float* __restrict__ map, const float* __restrict__ pred,
                                                           const float* __restrict__ target, int32_t height,
                                                           int32_t width, int64_t planes, float scale, float l1_scale,
                                                           int fuse_l1, float* __restrict__ dm) {
    constexpr int kSsimTH = kSsimFwdTH;
    constexpr int kSsimThreads = kSsimTW * kSsimTH / 2;
    constexpr int kSsimHH = kSsimTH + 10;
    constexpr int kSsimHW = kSsimTW + 10;  // halo columns
    constexpr int kHaloItems = kSsimHH * kSsimHW;
    constexpr int kHaloRounds = (kHaloItems + kSsimThreads - 1) / kSsimThreads;
    __shared__ float s_in[2][kSsimHH][kSsimHW + 1];
    __shared__ float s_h[5][kSsimHH][kSsimTW + 1];
    const int tiles_x = (width + kSsimTW - 1) / kSsimTW;
    const int tiles = tiles_x * ((height + kSsimTH - 1) / kSsimTH);
    const int tile = ssim_tile_of((int)blockIdx.x, tiles);
    if (tile >= tiles) return;
    const int ox = (tile % tiles_x) * kSsimTW;
    const int oy = (tile / tiles_x) * kSsimTH;
    const int64_t plane = blockIdx.y;
    const int64_t pbase = plane * (int64_t)height * width;
    const int lx = threadIdx.x % kSsimTW;
    const int ly0 = 2 * (threadIdx.x / kSsimTW);
    // the loss map values this thread adds to, loaded up front with the halo (clamped positions
    // outside the image are never stored; without a map the prediction stands in)
    float map_in[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int64_t j = pbase + (int64_t)min(oy + ly0 + r, height - 1) * width + min(ox + lx, width - 1);
        map_in[r] = (map != nullptr ? map : pred)[j];
    }
    {
        // the whole halo is loaded before the first store waits (no load under a branch: a
        // position outside the image reads a clamped one and keeps 0; threads past the halo
        // repeat its last item, same value to the same slot)
        float pv[kHaloRounds], tv[kHaloRounds];
#pragma unroll
        for (int u = 0; u < kHaloRounds; ++u) {
            const int i = min((int)threadIdx.x + kSsimThreads * u, kHaloItems - 1);
            const int hy = i / kSsimHW, hx = i % kSsimHW;
            const int y = oy + hy - 5, x = ox + hx - 5;
            const bool in = y >= 0 && y < height && x >= 0 && x < width;
            const int64_t j = pbase + (int64_t)min(max(y, 0), height - 1) * width + min(max(x, 0), width - 1);
            const float p = pred[j], t = target[j];
            pv[u] = in ? p : 0.0f;
            tv[u] = in ? t : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kHaloRounds; ++u) {
            const int i = min((int)threadIdx.x + kSsimThreads * u, kHaloItems - 1);
            const int hy = i / kSsimHW, hx = i % kSsimHW;
            s_in[0][hy][hx] = pv[u];
            s_in[1][hy][hx] = tv[u];
        }
    }
    __syncthreads();
    // The moments are formed from inputs shifted by one value per image and tile (the tile's
    // centre pixel): sigma^2 = E[x^2] - mu^2 loses the bits of E[x^2] to cancellation when mu is
    // large and the window nearly flat, and variances and covariances do not change under a
    // shift. The windows of the outputs that are kept (5 or more pixels from the edge) hold no
    // padding, so shifting the padding's zeros changes only outputs the map and dm overwrite
    // with 0. The means are the shifted means plus the shift. The shift pixel is the tile's
    // centre clamped into the image (a partial last tile's centre can lie in the padding).
    const int shift_hy = min(oy + kSsimTH / 2, height - 1) - oy + 5;
    const int shift_hx = min(ox + kSsimTW / 2, width - 1) - ox + 5;
    const float shift_p = s_in[0][shift_hy][shift_hx], shift_t = s_in[1][shift_hy][shift_hx];
    for (int i = threadIdx.x; i < kSsimHH * (kSsimTW / kHCols); i += kSsimThreads) {
        const int hy = i / (kSsimTW / kHCols), cx = kHCols * (i % (kSsimTW / kHCols));
        float a[kHCols][5];
#pragma unroll
        for (int j = 0; j < kHCols; ++j)
#pragma unroll
            for (int c = 0; c < 5; ++c) a[j][c] = 0.0f;
#pragma unroll
        for (int k = 0; k < 10 + kHCols; ++k) {
            const float pv = s_in[0][hy][cx + k] - shift_p, tv = s_in[1][hy][cx + k] - shift_t;
            const float m[5] = {pv, tv, pv * pv, tv * tv, pv * tv};
#pragma unroll
            for (int j = 0; j < kHCols; ++j) {
                // input column cx + k is tap k - j of output column cx + j (taps in order 0..10)
                if (k - j >= 0 && k - j < 11) {
#pragma unroll
                    for (int c = 0; c < 5; ++c) a[j][c] = __builtin_fmaf(kSsimW[k - j], m[c], a[j][c]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kHCols; ++j)
#pragma unroll
            for (int c = 0; c < 5; ++c) s_h[c][hy][cx + j] = a[j][c];
    }
    __syncthreads();
    float mom[2][5] = {{0.0f, 0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int k = 0; k < 12; ++k) {
#pragma unroll
        for (int c = 0; c < 5; ++c) {
            const float v = s_h[c][ly0 + k][lx];
            if (k < 11) mom[0][c] = __builtin_fmaf(kSsimW[k], v, mom[0][c]);
            if (k > 0) mom[1][c] = __builtin_fmaf(kSsimW[k - 1], v, mom[1][c]);
        }
    }
    const int64_t total = planes * (int64_t)height * width;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int ly = ly0 + r;
        const int x = ox + lx, y = oy + ly;
        if (x >= width || y >= height) continue;
        // shifted moments: d1 = mu1 - shift_p, d2 = mu2 - shift_t, e.. = E[shifted products]
        const float d1 = mom[r][0], d2 = mom[r][1], ex2 = mom[r][2], ey2 = mom[r][3], exy = mom[r][4];
        const float mu1 = d1 + shift_p, mu2 = d2 + shift_t;
        const float c1 = 0.01f * 0.01f, c2 = 0.03f * 0.03f;
        const float m1s = mu1 * mu1, m2s = mu2 * mu2;
        const float s1 = ex2 - d1 * d1, s2 = ey2 - d2 * d2, s12 = exy - d1 * d2;
        const float a = m1s + m2s + c1;
        const float b = s1 + s2 + c2;
        const float ct = 2.0f * mu1 * mu2 + c1;
        const float dt = 2.0f * s12 + c2;
        const float ab = a * b;
        // one hardware reciprocal serves all quotients (the SSIM bar is a tolerance): 1/ab,
        // 1/(a ab) = r/a and 1/(ab b) = r/b with r = 1/ab
        const float r_ab = __builtin_amdgcn_rcpf(ab);
        const float ssim = ab == 0.0f ? 1.0f : (ct * dt) * r_ab;
        const bool boundary = y < 5 || y >= height - 5 || x < 5 || x >= width - 5;
        const int64_t idx = pbase + (int64_t)y * width + x;
        if (map != nullptr) {
            float m = map_in[r];
            // exactly the L1 kernel's operations (loss.c:354-371)
            if (fuse_l1) m += l1_scale * fabsf(s_in[0][ly + 5][lx + 5] - s_in[1][ly + 5][lx + 5]);
            map[idx] = boundary ? 0.0f : m + (1.0f - ssim) * scale;
        }
        if (dm != nullptr) {
            float g_mu = 0.0f, g_s1 = 0.0f, g_s12 = 0.0f;
            if (!(boundary || a == 0.0f || b == 0.0f)) {
                const float r_aab = r_ab * __builtin_amdgcn_rcpf(a), r_abb = r_ab * __builtin_amdgcn_rcpf(b);
                const float ctdt = ct * dt;
                g_mu = 2.0f * mu2 * (dt - ct) * r_ab + 2.0f * mu1 * ctdt * (r_abb - r_aab);
                g_s1 = -ctdt * r_abb;
                g_s12 = 2.0f * ct * r_ab;
            }
            dm[idx] = g_mu;
            dm[total + idx] = g_s1;
            dm[2 * total + idx] = g_s12;
        }
    }
}

template <bool kVec>
__global__ __launch_bounds__(kSsimTW * kSsimBwdTH / 2) void ssim_backward_kernel(float* __restrict__ grad, const float* __restrict__ pred,
                                                            const float* __restrict__ target, int32_t height,
                                                            int32_t width, int64_t planes, float grad_scale,
                                                            float l1_grad_scale, int fuse_l1,
                                                            const float* __restrict__ dm) {
    GSX_SSIM_TILE(kSsimBwdTH)
    __shared__ __align__(16) float s_m[3 * kSsimHH * kSsimInW];
    __shared__ __align__(16) float s_h[3][kSsimHPlane];
    const int tiles_x = (width + kSsimTW - 1) / kSsimTW;
    const int tiles = tiles_x * ((height + kSsimTH - 1) / kSsimTH);
    const int tile = ssim_tile_of((int)blockIdx.x, tiles);
    if (tile >= tiles) return;
    const int ox = (tile % tiles_x) * kSsimTW;
    const int oy = (tile / tiles_x) * kSsimTH;
    // this plane's arrays (uniform bases; in-plane offsets are 32-bit)
    const int64_t pbase = (int64_t)blockIdx.y * height * width;
    const int64_t total = planes * (int64_t)height * width;
    const float* const pp = pred + pbase;
    const float* const tp = target + pbase;
    float* const gp = grad + pbase;
    const int lx = threadIdx.x % kSsimTW;
    const int ly0 = 2 * (threadIdx.x / kSsimTW);
    // this thread's two output pixels (prediction, target, gradient so far), loaded up front with
    // the halo (clamped positions outside the image are never stored)
    float pv_in[2], tv_in[2], g_in[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t j = (uint32_t)min(oy + ly0 + r, height - 1) * (uint32_t)width + (uint32_t)min(ox + lx, width - 1);
        pv_in[r] = pp[j];
        tv_in[r] = tp[j];
        g_in[r] = gp[j];
    }
    // The convolution's zero padding outside the image comes for free: a position outside reads
    // the nearest pixel inside, which lies in the 5-pixel boundary band, where the forward stored
    // 0 in every dm map.
    const float* const src[3] = {dm + pbase, dm + total + pbase, dm + 2 * total + pbase};
    const float zero[3] = {0.0f, 0.0f, 0.0f};
    ssim_stage_halo<kVec, 3, kSsimHH, kSsimThreads>(s_m, src, ox, oy, height, width, zero);
    __syncthreads();
    for (int i = threadIdx.x; i < (kSsimHH + 7) / 8 * 64; i += kSsimThreads) {
        const int hy = ssim_item_row(i), cx = kHCols * (i & 7);
        if (hy >= kSsimHH) continue;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float w[10 + kHCols];
            ssim_row_window(s_m + (c * kSsimHH + hy) * kSsimInW, cx, w);
            float a[kHCols] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < 10 + kHCols; ++k) {
#pragma unroll
                for (int j = 0; j < kHCols; ++j) {
                    if (k - j >= 0 && k - j < 11) a[j] = __builtin_fmaf(kSsimW[k - j], w[k], a[j]);
                }
            }
            *reinterpret_cast<float4*>(&s_h[c][hy * kSsimTW + cx]) = make_float4(a[0], a[1], a[2], a[3]);
        }
    }
    __syncthreads();
    float cv[2][3] = {{0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int k = 0; k < 12; ++k) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float v = s_h[c][(ly0 + k) * kSsimTW + lx];
            if (k < 11) cv[0][c] = __builtin_fmaf(kSsimW[k], v, cv[0][c]);
            if (k > 0) cv[1][c] = __builtin_fmaf(kSsimW[k - 1], v, cv[1][c]);
        }
    }
    const int x = ox + lx;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int y = oy + ly0 + r;
        if (x >= width || y >= height) continue;
        const float pv = pv_in[r], tv = tv_in[r];
        float g = g_in[r];
        if (fuse_l1) {  // exactly the L1 kernel's operations
            const float d = pv - tv;
            const float s = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
            g += s * l1_grad_scale;
        }
        gp[(uint32_t)y * (uint32_t)width + (uint32_t)x] =
            g + (-(cv[r][0] + 2.0f * pv * cv[r][1] + tv * cv[r][2]) * grad_scale);
    }
}

}  // namespace gsx_amd

using namespace gsx_amd;

// The SSIM halos are staged with 16-byte loads when every image row and plane starts 16-byte
// aligned: width a multiple of 4 and the staged arrays' bases 16-byte aligned.
static bool ssim_vector_halo(int32_t width, const float* a, const float* b) {
    return width % 4 == 0 && (((uintptr_t)a | (uintptr_t)b) & 15u) == 0;
}

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
    if (planes > 65535 || (int64_t)height * width > (int64_t)UINT32_MAX) return GSX_HIP_ERROR_OUT_OF_RANGE;
    const int tiles = ((width + kSsimTW - 1) / kSsimTW) * ((height + kSsimFwdTH - 1) / kSsimFwdTH);
    hipLaunchKernelGGL(ssim_forward_kernel, dim3((unsigned)(8 * ((tiles + 7) / 8)), (unsigned)planes),
                       dim3(kSsimTW * kSsimFwdTH / 2), 0, stream, loss_map, prediction, target, height, width, planes,
                       scale, l1_scale, fuse_l1, ssim_workspace);
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                            const float* target, int64_t outer_count,
                                                            int32_t channels, int32_t height, int32_t width,
                                                            float grad_scale, const float* ssim_workspace,
                                                            float l1_grad_scale, int fuse_l1, hipStream_t stream) {
    const int64_t planes = outer_count * channels;
    if (planes <= 0 || height <= 0 || width <= 0) return GSX_HIP_ERROR_INVALID_ARGUMENT;
    if (planes > 65535 || (int64_t)height * width > (int64_t)UINT32_MAX) return GSX_HIP_ERROR_OUT_OF_RANGE;
    const int tiles = ((width + kSsimTW - 1) / kSsimTW) * ((height + kSsimBwdTH - 1) / kSsimBwdTH);
    const bool vec = ssim_vector_halo(width, ssim_workspace, ssim_workspace);
    hipLaunchKernelGGL(vec ? ssim_backward_kernel<true> : ssim_backward_kernel<false>,
                       dim3((unsigned)(8 * ((tiles + 7) / 8)), (unsigned)planes), dim3(kSsimTW * kSsimBwdTH / 2), 0,
                       stream, grad_prediction, prediction, target, height, width, planes, grad_scale, l1_grad_scale,
                       fuse_l1, ssim_workspace);
    return (gsx_hip_status)hipGetLastError();
}

}  // extern "C"
