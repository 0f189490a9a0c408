// tensor.hip - the element-wise, random, reduce and image-conversion operations of a gsx backend
// buffer (the gsx_backend_buffer_i entries of gsx/src/gsx-impl.h:302-458) as gfx950 kernels.
//
// Semantics follow the CPU backend element by element (gsx/src/gsx-cpu/core.c:874-2019):
//   fills, clamps, gathers, HWC/CHW and u8/f32 conversions, exp / sigmoid / |x|, the pcg32
//   streams of rand / randn / randint / multinomial and the sRGB transfer functions are
//   bit-identical (expf, logf, sinf, cosf and powf are the glibc-exact restatements of
//   gsx_math.h); sums (sum, mean,
//   mse, mae) accumulate in double in a fixed tree order (deterministic, and at least as
//   accurate as the CPU's sequential float sum), max keeps the CPU's first-occurrence and NaN
//   rules exactly.
// Every stream position is explicit: element i of a rand fill is draw i of the (state, inc)
// stream, reached with the O(log i) jump of gsx_pcg32_advance, so the fill is one parallel
// launch instead of the CPU's sequential loop.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/gsx_hip.h"
#include "common.hpp"
#include "gsx_math.h"

namespace gsx_amd {
void set_last_error(const char* what);
}

using namespace gsx_amd;

#define GSX_TRY_STATUS(expr)                  \
    do {                                      \
        const gsx_hip_status s_ = (expr);     \
        if (s_ != GSX_HIP_SUCCESS) return s_; \
    } while (0)

namespace {

constexpr int kThreads = 256;
constexpr int kRandPerThread = 16;  // consecutive draws per lane of the rand-like fills

unsigned grid_for(int64_t n, int64_t per_block) {
    int64_t b = (n + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > 65535LL * 64) b = 65535LL * 64;
    return (unsigned)b;
}

gsx_hip_status launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_last_error(what);
        return (gsx_hip_status)e;
    }
    return GSX_HIP_SUCCESS;
}

gsx_hip_status invalid(const char* what) {
    set_last_error(what);
    return GSX_HIP_ERROR_INVALID_ARGUMENT;
}

struct Pattern {
    uint8_t b[64];
};

// 16-byte stores of a pattern whose length divides 16 (dst 16-byte aligned, n16 vectors).
__global__ __launch_bounds__(kThreads) void fill_vec16_kernel(uint4* __restrict__ dst, int64_t n16, uint4 v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = v;
}

// Any pattern length up to 64 bytes: byte i of the buffer is pattern byte i mod len.
__global__ __launch_bounds__(kThreads) void fill_bytes_kernel(uint8_t* __restrict__ dst, int64_t bytes, Pattern p,
                                                              int len) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = p.b[i % len];
}

// rand: element i = pcg32_next_float of draw i (gsx-cpu/core.c:970-1007).
__global__ __launch_bounds__(kThreads) void fill_rand_kernel(float* __restrict__ dst, int64_t count, uint64_t state,
                                                             uint64_t inc) {
    const int64_t first = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kRandPerThread;
    if (first >= count) return;
    gsx_amd_pcg32 rng{state, inc};
    gsx_pcg32_advance(&rng, (uint64_t)first);
    const int64_t end = first + kRandPerThread < count ? first + kRandPerThread : count;
    for (int64_t i = first; i < end; ++i) dst[i] = gsx_pcg32_next_f32(&rng);
}


// randn: pair k of elements from draws 2k, 2k+1 by Box-Muller (gsx-cpu/core.c:1009-1064).
__global__ __launch_bounds__(kThreads) void fill_randn_kernel(float* __restrict__ dst, int64_t count, uint64_t state,
                                                              uint64_t inc, float sigma) {
    const int64_t pairs = (count + 1) / 2;
    const int64_t first = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * (kRandPerThread / 2);
    if (first >= pairs) return;
    gsx_amd_pcg32 rng{state, inc};
    gsx_pcg32_advance(&rng, (uint64_t)(2 * first));
    const int64_t end = first + kRandPerThread / 2 < pairs ? first + kRandPerThread / 2 : pairs;
    for (int64_t k = first; k < end; ++k) {
        float u1 = gsx_pcg32_next_f32(&rng);
        const float u2 = gsx_pcg32_next_f32(&rng);
        if (u1 < 1e-7f) u1 = 1e-7f;
        const float radius = sqrtf(-2.0f * gsx_logf(u1));
        const float theta = 6.2831853071795864769f * u2;
        dst[2 * k] = radius * gsx_cosf(theta) * sigma;
        if (2 * k + 1 < count) dst[2 * k + 1] = radius * gsx_sinf(theta) * sigma;
    }
}

// randint, step 1: draw j of the stream and whether pcg32_next_uint_bound accepts it
// (r >= (2^32 - bound) mod bound, gsx/src/pcg32.h:75-83).
__global__ __launch_bounds__(kThreads) void randint_draws_kernel(uint32_t* __restrict__ draws,
                                                                 uint32_t* __restrict__ accepted, int64_t m,
                                                                 uint64_t state, uint64_t inc, uint32_t threshold) {
    const int64_t first = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kRandPerThread;
    if (first >= m) return;
    gsx_amd_pcg32 rng{state, inc};
    gsx_pcg32_advance(&rng, (uint64_t)first);
    const int64_t end = first + kRandPerThread < m ? first + kRandPerThread : m;
    for (int64_t j = first; j < end; ++j) {
        const uint32_t r = gsx_pcg32_next_u32(&rng);
        draws[j] = r;
        accepted[j] = r >= threshold ? 1u : 0u;
    }
}

// randint, step 2: element i is the i-th accepted draw mod bound.
__global__ __launch_bounds__(kThreads) void randint_scatter_kernel(const uint32_t* __restrict__ draws,
                                                                   const uint32_t* __restrict__ accepted,
                                                                   const uint32_t* __restrict__ rank, int64_t m,
                                                                   void* __restrict__ dst, int64_t count,
                                                                   int element_bytes, uint32_t bound) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < m; j += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = rank[j];
        if (accepted[j] == 0u || i >= count) continue;
        const uint32_t v = draws[j] % bound;
        if (element_bytes == 1) static_cast<uint8_t*>(dst)[i] = (uint8_t)v;
        else static_cast<int32_t*>(dst)[i] = (int32_t)v;
    }
}

// multinomial: sample i from draw i, u * cdf[last], first category whose cdf exceeds it
// (gsx-cpu/core.c:1118-1206).
__global__ __launch_bounds__(kThreads) void multinomial_kernel(int32_t* __restrict__ out, int64_t samples,
                                                               const float* __restrict__ cdf, int64_t categories,
                                                               uint64_t state, uint64_t inc) {
    const int64_t first = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * kRandPerThread;
    if (first >= samples) return;
    gsx_amd_pcg32 rng{state, inc};
    gsx_pcg32_advance(&rng, (uint64_t)first);
    const float total = cdf[categories - 1];
    const int64_t end = first + kRandPerThread < samples ? first + kRandPerThread : samples;
    for (int64_t i = first; i < end; ++i) {
        const float draw = gsx_pcg32_next_f32(&rng) * total;
        int64_t lo = 0, hi = categories;
        while (lo < hi) {
            const int64_t mid = lo + (hi - lo) / 2;
            if (draw < cdf[mid]) hi = mid;
            else lo = mid + 1;
        }
        out[i] = (int32_t)(lo >= categories ? categories - 1 : lo);
    }
}

// *flag = 1 when an element is inf or NaN (gsx-cpu/core.c:1208-1246).
__global__ __launch_bounds__(kThreads) void check_finite_kernel(const float* __restrict__ x, int64_t count,
                                                                uint32_t* __restrict__ flag) {
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        bad |= (__float_as_uint(x[i]) & 0x7f800000u) == 0x7f800000u;
    if (wave_ballot(bad) != 0ull && __lane_id() == 0) *flag = 1u;
}

// exp, sigmoid, sigmoid', |x| with the CPU's expressions (gsx-cpu/core.c:1335-1412); x may
// equal out. The op is a template parameter: one straight-line kernel per op (hipcc's lowering of
// this chain as a run-time uniform branch stored an unset register for op 3).
template <int OP>
__global__ __launch_bounds__(kThreads) void unary_kernel(const float* x, float* out, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = x[i];
        float r;
        if constexpr (OP == GSX_HIP_UNARY_EXP) {
            r = gsx_expf(v);
        } else if constexpr (OP == GSX_HIP_UNARY_SIGMOID) {
            r = 1.0f / (1.0f + gsx_expf(-v));
        } else if constexpr (OP == GSX_HIP_UNARY_SIGMOID_DERIVATIVE) {
            const float s = 1.0f / (1.0f + gsx_expf(-v));
            r = s * (1.0f - s);
        } else {
            r = fabsf(v);
        }
        out[i] = r;
    }
}

// Clamp in place with the CPU's compares (a NaN stays NaN; gsx-cpu/core.c:1717-1798).
template <typename T>
__global__ __launch_bounds__(kThreads) void clamp_kernel(T* __restrict__ x, int64_t count, T lo, T hi) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const T v = x[i];
        if (v < lo) x[i] = lo;
        else if (v > hi) x[i] = hi;
    }
}

// ---- reductions over rows of `reduce` elements (out[outer]) --------------------------------
// Stage 1 cuts every row into `chunks` ranges; each workgroup reduces one range to a partial
// (double sum, or a max record), stage 2 combines a row's partials in range order. The max
// record keeps the CPU's rule (gsx-cpu/core.c:1566-1583: accum = x[0], then x > accum): the
// first of equal maxima wins, NaN entries are skipped, and a NaN x[0] makes the row NaN.
struct MaxRec {
    float v;
    uint32_t has;  // a non-NaN value was seen
};

__device__ inline MaxRec max_combine(MaxRec a, MaxRec b) {  // a covers the earlier range
    if (!b.has) return a;
    if (!a.has) return b;
    return b.v > a.v ? b : a;
}

constexpr int kReduceChunk = 8192;  // elements per stage-1 workgroup

__device__ inline double block_sum_double(double v, double* s_wave) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_down(v, off, kWave);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) s_wave[wave] = v;
    __syncthreads();
    double total = 0.0;
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / kWave; ++w) total += s_wave[w];
    return total;  // valid in thread 0
}

__device__ inline MaxRec block_max(MaxRec r, MaxRec* s_wave) {
    // lanes hold consecutive sub-ranges in lane order: combine neighbours, earlier first
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        MaxRec o;
        o.v = __shfl_down(r.v, off, kWave);
        o.has = (uint32_t)__shfl_down((int)r.has, off, kWave);
        if (((threadIdx.x & (kWave - 1)) & ((off << 1) - 1)) == 0 && (threadIdx.x & (kWave - 1)) + off < kWave)
            r = max_combine(r, o);
    }
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) s_wave[wave] = r;
    __syncthreads();
    MaxRec total{0.0f, 0u};
    if (threadIdx.x == 0)
        for (int w = 0; w < kThreads / kWave; ++w) total = max_combine(total, s_wave[w]);
    return total;
}

// op: 0 sum, 1 mean, 2 max, 3 mse (lhs, rhs), 4 mae (lhs, rhs)
__global__ __launch_bounds__(kThreads) void reduce_stage1_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ y, int64_t reduce,
                                                                 int64_t chunks, int op, double* __restrict__ psum,
                                                                 MaxRec* __restrict__ pmax) {
    __shared__ double s_sum[kThreads / kWave];
    __shared__ MaxRec s_max[kThreads / kWave];
    const int64_t row = blockIdx.x / chunks, c = blockIdx.x % chunks;
    const int64_t b = c * kReduceChunk;
    const int64_t e = b + kReduceChunk < reduce ? b + kReduceChunk : reduce;
    const float* xr = x + row * reduce;
    if (op == 2) {
        // each lane takes a contiguous sub-range, so lane order is element order
        const int64_t per = (kReduceChunk + kThreads - 1) / kThreads;
        const int64_t lb = b + (int64_t)threadIdx.x * per;
        const int64_t le = lb + per < e ? lb + per : e;
        MaxRec r{0.0f, 0u};
        for (int64_t i = lb; i < le; ++i) {
            const float v = xr[i];
            if (v != v) continue;
            if (!r.has || v > r.v) {
                r.v = v;
                r.has = 1u;
            }
        }
        const MaxRec t = block_max(r, s_max);
        if (threadIdx.x == 0) pmax[blockIdx.x] = t;
        return;
    }
    const float* yr = y != nullptr ? y + row * reduce : nullptr;
    double acc = 0.0;
    for (int64_t i = b + threadIdx.x; i < e; i += kThreads) {
        float t = xr[i];
        if (op >= 3) {
            const float d = t - yr[i];
            t = op == 3 ? d * d : fabsf(d);
        }
        acc += (double)t;
    }
    const double total = block_sum_double(acc, s_sum);
    if (threadIdx.x == 0) psum[blockIdx.x] = total;
}

__global__ __launch_bounds__(kThreads) void reduce_stage2_kernel(const float* __restrict__ x, int64_t outer,
                                                                 int64_t reduce, int64_t chunks, int op,
                                                                 const double* __restrict__ psum,
                                                                 const MaxRec* __restrict__ pmax,
                                                                 float* __restrict__ out) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= outer) return;
    if (op == 2) {
        const float first = x[row * reduce];
        MaxRec r{0.0f, 0u};
        for (int64_t c = 0; c < chunks; ++c) r = max_combine(r, pmax[row * chunks + c]);
        out[row] = first != first ? first : r.v;
        return;
    }
    double s = 0.0;
    for (int64_t c = 0; c < chunks; ++c) s += psum[row * chunks + c];
    const float sf = (float)s;
    out[row] = op == 0 ? sf : sf / (float)reduce;  // mean, mse, mae divide as the CPU does
}

__device__ inline float clamp_unit(float v) {
    // gsx/src/extra/gsx-image-impl.h:9-21
    if ((__float_as_uint(v) & 0x7f800000u) == 0x7f800000u) return v > 0.0f ? 1.0f : 0.0f;
    if (v < 0.0f) return 0.0f;
    if (v > 1.0f) return 1.0f;
    return v;
}


// gsx-image-impl.h:34-50; DIR 1 linear -> sRGB, 2 sRGB -> linear, 0 copy (a template parameter,
// as for the unary ops)
template <int DIR>
__global__ __launch_bounds__(kThreads) void colorspace_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                              int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        float v = src[i];
        if constexpr (DIR == 1) {
            v = clamp_unit(v);
            v = v <= 0.0031308f ? 12.92f * v : 1.055f * gsx_powf(v, 1.0f / 2.4f) - 0.055f;
        } else if constexpr (DIR == 2) {
            v = clamp_unit(v);
            v = v <= 0.04045f ? v / 12.92f : gsx_powf((v + 0.055f) / 1.055f, 2.4f);
        }
        dst[i] = v;
    }
}

// One element per thread: its (c, y, x) from the destination index, the source index in the
// other layout (gsx-image-impl.h:128-170).
template <typename T>
__global__ __launch_bounds__(kThreads) void storage_kernel(const T* __restrict__ src, int src_hwc, T* __restrict__ dst,
                                                           int dst_hwc, int64_t c, int64_t h, int64_t w) {
    const int64_t total = c * h * w;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t ch, y, x;
        if (dst_hwc) {
            ch = i % c;
            x = (i / c) % w;
            y = i / (c * w);
        } else {
            x = i % w;
            y = (i / w) % h;
            ch = i / (w * h);
        }
        const int64_t s = src_hwc ? (y * w + x) * c + ch : (ch * h + y) * w + x;
        dst[i] = src[s];
    }
}

// f32 -> u8 quantise, u8 -> f32 dequantise (gsx-image-impl.h:23-32).
__global__ __launch_bounds__(kThreads) void quantize_kernel(const float* __restrict__ src, uint8_t* __restrict__ dst,
                                                            int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = (uint8_t)(clamp_unit(src[i]) * 255.0f + 0.5f);
}

__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                              int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = (float)src[i] / 255.0f;
}

// Dataloader layout: element (c, y, x) of a CHW float tensor from a tightly packed HWC (channels 3)
// or HW (channels 1) host payload of u8 or f32, value-preserving (u8 v becomes v.0f), as
// gsx/src/gsx-data-impl.h:173-268 packs it on the CPU.
template <typename T>
__global__ __launch_bounds__(kThreads) void to_chw_f32_kernel(const T* __restrict__ src, float* __restrict__ dst,
                                                              int64_t channels, int64_t pixels) {
    const int64_t total = channels * pixels;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t c = i / pixels, px = i - c * pixels;
        dst[i] = (float)src[px * channels + c];
    }
}

int64_t reduce_chunks(int64_t reduce) {
    const int64_t c = (reduce + kReduceChunk - 1) / kReduceChunk;
    return c < 1 ? 1 : c;
}

}  // namespace

extern "C" {

gsx_hip_status gsx_hip_fill_pattern(void* dst, size_t bytes, const void* pattern, size_t pattern_bytes,
                                    hipStream_t stream) {
    if (bytes == 0) return GSX_HIP_SUCCESS;
    if (dst == nullptr || pattern == nullptr || pattern_bytes == 0 || pattern_bytes > 64 || bytes % pattern_bytes != 0)
        return invalid("fill: pattern of 1..64 bytes dividing the byte count required");
    Pattern p{};
    for (size_t i = 0; i < pattern_bytes; ++i) p.b[i] = static_cast<const uint8_t*>(pattern)[i];
    if (16 % pattern_bytes == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 && bytes % 16 == 0) {
        uint8_t v16[16];
        for (int i = 0; i < 16; ++i) v16[i] = p.b[i % pattern_bytes];
        uint4 v;
        memcpy(&v, v16, 16);
        const int64_t n16 = (int64_t)(bytes / 16);
        hipLaunchKernelGGL(fill_vec16_kernel, dim3(grid_for(n16, kThreads * 4)), dim3(kThreads), 0, stream,
                           static_cast<uint4*>(dst), n16, v);
    } else {
        hipLaunchKernelGGL(fill_bytes_kernel, dim3(grid_for((int64_t)bytes, kThreads * 4)), dim3(kThreads), 0, stream,
                           static_cast<uint8_t*>(dst), (int64_t)bytes, p, (int)pattern_bytes);
    }
    return launch_status("fill kernel");
}

gsx_hip_status gsx_hip_fill_rand_f32(float* dst, int64_t count, uint64_t state, uint64_t inc, hipStream_t stream) {
    if (count < 0 || (count > 0 && dst == nullptr)) return invalid("rand fill: bad destination");
    if (count == 0) return GSX_HIP_SUCCESS;
    hipLaunchKernelGGL(fill_rand_kernel, dim3(grid_for(count, (int64_t)kThreads * kRandPerThread)), dim3(kThreads), 0,
                       stream, dst, count, state, inc);
    return launch_status("fill_rand_kernel");
}

gsx_hip_status gsx_hip_fill_randn_f32(float* dst, int64_t count, uint64_t state, uint64_t inc, float sigma,
                                      hipStream_t stream) {
    if (count < 0 || (count > 0 && dst == nullptr)) return invalid("randn fill: bad destination");
    if (count == 0) return GSX_HIP_SUCCESS;
    const int64_t pairs = (count + 1) / 2;
    hipLaunchKernelGGL(fill_randn_kernel, dim3(grid_for(pairs, (int64_t)kThreads * (kRandPerThread / 2))),
                       dim3(kThreads), 0, stream, dst, count, state, inc, sigma);
    return launch_status("fill_randn_kernel");
}

size_t gsx_hip_fill_randint_temp_bytes(int64_t draws) {
    const int64_t m = draws < 1 ? 1 : draws;
    return (size_t)m * 3 * sizeof(uint32_t) + gsx_hip_scan_temp_bytes(m) + 256;
}

gsx_hip_status gsx_hip_fill_randint(void* dst, int64_t count, int32_t element_bytes, uint64_t state, uint64_t inc,
                                    uint32_t bound, int64_t draws, void* temp, int64_t* out_accepted,
                                    hipStream_t stream) {
    if (count < 0 || draws < count || bound == 0 || (element_bytes != 1 && element_bytes != 4) ||
        (count > 0 && (dst == nullptr || temp == nullptr)))
        return invalid("randint fill: bad arguments");
    if (out_accepted) *out_accepted = 0;
    if (count == 0) return GSX_HIP_SUCCESS;
    const uint32_t threshold = (~bound + 1u) % bound;
    const int64_t m = draws;
    uint32_t* d = static_cast<uint32_t*>(temp);
    uint32_t* acc = d + m;
    uint32_t* rank = acc + m;  // m + 1 words (scan total at [m])
    void* scan_temp = reinterpret_cast<void*>(((reinterpret_cast<uintptr_t>(rank + m + 1)) + 255u) & ~(uintptr_t)255u);
    hipLaunchKernelGGL(randint_draws_kernel, dim3(grid_for(m, (int64_t)kThreads * kRandPerThread)), dim3(kThreads), 0,
                       stream, d, acc, m, state, inc, threshold);
    GSX_TRY_STATUS(launch_status("randint_draws_kernel"));
    GSX_TRY_STATUS(gsx_hip_scan_exclusive_u32(acc, rank, m, scan_temp, stream));
    hipLaunchKernelGGL(randint_scatter_kernel, dim3(grid_for(m, kThreads * 4)), dim3(kThreads), 0, stream, d, acc, rank,
                       m, dst, count, element_bytes, bound);
    GSX_TRY_STATUS(launch_status("randint_scatter_kernel"));
    if (out_accepted != nullptr) {
        uint32_t total = 0;
        hipError_t e = hipMemcpyAsync(&total, rank + m, sizeof(total), hipMemcpyDeviceToHost, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) {
            set_last_error("randint fill: reading the accepted count");
            return (gsx_hip_status)e;
        }
        *out_accepted = total;
    }
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_multinomial_i32(int32_t* out, int64_t samples, const float* cdf, int64_t categories,
                                       uint64_t state, uint64_t inc, hipStream_t stream) {
    if (samples < 0 || categories < 0 || (samples > 0 && categories > 0 && (out == nullptr || cdf == nullptr)))
        return invalid("multinomial: bad arguments");
    if (samples == 0 || categories == 0) return GSX_HIP_SUCCESS;
    hipLaunchKernelGGL(multinomial_kernel, dim3(grid_for(samples, (int64_t)kThreads * kRandPerThread)), dim3(kThreads),
                       0, stream, out, samples, cdf, categories, state, inc);
    return launch_status("multinomial_kernel");
}

gsx_hip_status gsx_hip_check_finite_f32(const float* x, int64_t count, uint32_t* flag, hipStream_t stream) {
    if (count < 0 || flag == nullptr || (count > 0 && x == nullptr)) return invalid("check_finite: bad arguments");
    if (count == 0) return GSX_HIP_SUCCESS;
    hipLaunchKernelGGL(check_finite_kernel, dim3(grid_for(count, kThreads * 16)), dim3(kThreads), 0, stream, x, count,
                       flag);
    return launch_status("check_finite_kernel");
}

gsx_hip_status gsx_hip_unary_f32(const float* x, float* out, int64_t count, int32_t op, hipStream_t stream) {
    if (count < 0 || op < GSX_HIP_UNARY_EXP || op > GSX_HIP_UNARY_ABS || (count > 0 && (x == nullptr || out == nullptr)))
        return invalid("unary: bad arguments");
    if (count == 0) return GSX_HIP_SUCCESS;
    const dim3 grid(grid_for(count, kThreads * 4));
    switch (op) {
        case GSX_HIP_UNARY_EXP:
            hipLaunchKernelGGL(unary_kernel<GSX_HIP_UNARY_EXP>, grid, dim3(kThreads), 0, stream, x, out, count);
            break;
        case GSX_HIP_UNARY_SIGMOID:
            hipLaunchKernelGGL(unary_kernel<GSX_HIP_UNARY_SIGMOID>, grid, dim3(kThreads), 0, stream, x, out, count);
            break;
        case GSX_HIP_UNARY_SIGMOID_DERIVATIVE:
            hipLaunchKernelGGL(unary_kernel<GSX_HIP_UNARY_SIGMOID_DERIVATIVE>, grid, dim3(kThreads), 0, stream, x, out,
                               count);
            break;
        default:
            hipLaunchKernelGGL(unary_kernel<GSX_HIP_UNARY_ABS>, grid, dim3(kThreads), 0, stream, x, out, count);
            break;
    }
    return launch_status("unary_kernel");
}

gsx_hip_status gsx_hip_clamp_inplace(void* x, int64_t count, int32_t data_type, const void* lo, const void* hi,
                                     hipStream_t stream) {
    if (count < 0 || lo == nullptr || hi == nullptr || (count > 0 && x == nullptr)) return invalid("clamp: bad arguments");
    if (count == 0) return GSX_HIP_SUCCESS;
    const unsigned g = grid_for(count, kThreads * 4);
    switch (data_type) {
        case GSX_HIP_DTYPE_F32:
            hipLaunchKernelGGL(clamp_kernel<float>, dim3(g), dim3(kThreads), 0, stream, static_cast<float*>(x), count,
                               *static_cast<const float*>(lo), *static_cast<const float*>(hi));
            break;
        case GSX_HIP_DTYPE_U8:
            hipLaunchKernelGGL(clamp_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, stream, static_cast<uint8_t*>(x),
                               count, *static_cast<const uint8_t*>(lo), *static_cast<const uint8_t*>(hi));
            break;
        case GSX_HIP_DTYPE_I32:
            hipLaunchKernelGGL(clamp_kernel<int32_t>, dim3(g), dim3(kThreads), 0, stream, static_cast<int32_t*>(x),
                               count, *static_cast<const int32_t*>(lo), *static_cast<const int32_t*>(hi));
            break;
        default:
            set_last_error("clamp: only f32, u8 and i32 tensors");
            return GSX_HIP_ERROR_NOT_SUPPORTED;
    }
    return launch_status("clamp_kernel");
}

size_t gsx_hip_reduce_temp_bytes(int64_t outer, int64_t reduce) {
    const int64_t parts = (outer < 1 ? 1 : outer) * reduce_chunks(reduce);
    return (size_t)parts * sizeof(double) + 256;
}

gsx_hip_status gsx_hip_reduce_f32(const float* x, const float* y, int64_t outer, int64_t reduce, int32_t op,
                                  float* out, void* temp, hipStream_t stream) {
    if (outer < 1 || reduce < 1 || op < GSX_HIP_REDUCE_SUM || op > GSX_HIP_REDUCE_MAE || x == nullptr ||
        out == nullptr || temp == nullptr || (op >= GSX_HIP_REDUCE_MSE && y == nullptr))
        return invalid("reduce: bad arguments");
    const int64_t chunks = reduce_chunks(reduce);
    if (outer * chunks > 0x7fffffffLL) {
        set_last_error("reduce: too many rows");
        return GSX_HIP_ERROR_OUT_OF_RANGE;
    }
    double* psum = static_cast<double*>(temp);
    MaxRec* pmax = static_cast<MaxRec*>(temp);
    hipLaunchKernelGGL(reduce_stage1_kernel, dim3((unsigned)(outer * chunks)), dim3(kThreads), 0, stream, x,
                       op >= GSX_HIP_REDUCE_MSE ? y : nullptr, reduce, chunks, (int)op, psum, pmax);
    GSX_TRY_STATUS(launch_status("reduce_stage1_kernel"));
    hipLaunchKernelGGL(reduce_stage2_kernel, dim3(grid_for(outer, kThreads)), dim3(kThreads), 0, stream, x, outer,
                       reduce, chunks, (int)op, psum, pmax, out);
    return launch_status("reduce_stage2_kernel");
}

gsx_hip_status gsx_hip_image_colorspace_f32(const float* src, float* dst, int64_t count, int32_t src_srgb,
                                            int32_t dst_srgb, hipStream_t stream) {
    if (count < 0 || (count > 0 && (src == nullptr || dst == nullptr))) return invalid("colorspace: bad arguments");
    if (count == 0) return GSX_HIP_SUCCESS;
    const int direction = (!src_srgb && dst_srgb) ? 1 : ((src_srgb && !dst_srgb) ? 2 : 0);
    const dim3 grid(grid_for(count, kThreads * 4));
    if (direction == 1)
        hipLaunchKernelGGL(colorspace_kernel<1>, grid, dim3(kThreads), 0, stream, src, dst, count);
    else if (direction == 2)
        hipLaunchKernelGGL(colorspace_kernel<2>, grid, dim3(kThreads), 0, stream, src, dst, count);
    else
        hipLaunchKernelGGL(colorspace_kernel<0>, grid, dim3(kThreads), 0, stream, src, dst, count);
    return launch_status("colorspace_kernel");
}

gsx_hip_status gsx_hip_image_storage_convert(const void* src, int32_t src_hwc, void* dst, int32_t dst_hwc,
                                             int64_t channels, int64_t height, int64_t width, int32_t element_bytes,
                                             hipStream_t stream) {
    const int64_t total = channels * height * width;
    if (channels < 0 || height < 0 || width < 0 || (total > 0 && (src == nullptr || dst == nullptr)))
        return invalid("storage convert: bad arguments");
    if (total == 0) return GSX_HIP_SUCCESS;
    const unsigned g = grid_for(total, kThreads * 4);
    switch (element_bytes) {
        case 1:
            hipLaunchKernelGGL(storage_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, stream,
                               static_cast<const uint8_t*>(src), (int)src_hwc, static_cast<uint8_t*>(dst), (int)dst_hwc,
                               channels, height, width);
            break;
        case 2:
            hipLaunchKernelGGL(storage_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, stream,
                               static_cast<const uint16_t*>(src), (int)src_hwc, static_cast<uint16_t*>(dst),
                               (int)dst_hwc, channels, height, width);
            break;
        case 4:
            hipLaunchKernelGGL(storage_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, stream,
                               static_cast<const uint32_t*>(src), (int)src_hwc, static_cast<uint32_t*>(dst),
                               (int)dst_hwc, channels, height, width);
            break;
        default:
            return invalid("storage convert: element size must be 1, 2 or 4 bytes");
    }
    return launch_status("storage_kernel");
}

gsx_hip_status gsx_hip_dataloader_to_chw_f32(const void* src, int32_t src_is_u8, int64_t channels, int64_t height,
                                            int64_t width, float* dst, hipStream_t stream) {
    const int64_t pixels = height * width;
    if (channels < 1 || height < 0 || width < 0 || (pixels > 0 && (src == nullptr || dst == nullptr)))
        return invalid("dataloader layout: bad arguments");
    if (pixels == 0) return GSX_HIP_SUCCESS;
    const unsigned g = grid_for(channels * pixels, kThreads * 4);
    if (src_is_u8)
        hipLaunchKernelGGL(to_chw_f32_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, stream,
                           static_cast<const uint8_t*>(src), dst, channels, pixels);
    else
        hipLaunchKernelGGL(to_chw_f32_kernel<float>, dim3(g), dim3(kThreads), 0, stream,
                           static_cast<const float*>(src), dst, channels, pixels);
    return launch_status("to_chw_f32_kernel");
}

gsx_hip_status gsx_hip_image_quantize_u8(const float* src, uint8_t* dst, int64_t count, hipStream_t stream) {
    if (count < 0 || (count > 0 && (src == nullptr || dst == nullptr))) return invalid("quantize: bad arguments");
    if (count == 0) return GSX_HIP_SUCCESS;
    hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(count, kThreads * 4)), dim3(kThreads), 0, stream, src, dst, count);
    return launch_status("quantize_kernel");
}

gsx_hip_status gsx_hip_image_dequantize_u8(const uint8_t* src, float* dst, int64_t count, hipStream_t stream) {
    if (count < 0 || (count > 0 && (src == nullptr || dst == nullptr))) return invalid("dequantize: bad arguments");
    if (count == 0) return GSX_HIP_SUCCESS;
    hipLaunchKernelGGL(dequantize_kernel, dim3(grid_for(count, kThreads * 4)), dim3(kThreads), 0, stream, src, dst,
                       count);
    return launch_status("dequantize_kernel");
}

}  // extern "C"
