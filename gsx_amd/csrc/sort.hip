// sort.hip - device-wide exclusive scan and stable LSD radix sort of (u64 key, u32 value) pairs.
//
// Replaces cub::DeviceScan::ExclusiveSum (gsx/src/gsx-cuda/fastgs/forward.cu:180-185) and
// cub::DeviceRadixSort::SortPairs (forward.cu:155-161, 214-220).
//
// Radix sort: 8-bit digits, one "reduce then scan" pass per digit:
//   1. digit histogram per 4096-key block (LDS counters)                 -> hist[digit][block]
//   2. exclusive scan of hist in digit-major order                       -> global bases
//   3. scatter: every 256-key round is ranked with wave64 ballots (8 ballots give each lane
//      the mask of lanes holding the same digit); waves are ordered through LDS counters, so
//      the rank of a key is its position among equal digits in input order: the sort is
//      stable, which the tile lists rely on (equal (tile, depth) keys keep Gaussian order).
// No kernel waits on another workgroup, so every wave always runs to completion.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"
#include "../../include/gsx_hip.h"

namespace gsx_amd {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanChunk = kScanThreads * kScanItems;  // 4096 elements per block

constexpr int kSortThreads = 256;
constexpr int kSortRounds = 16;
constexpr int kSortChunk = kSortThreads * kSortRounds;  // 4096 keys per block
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;

// Exclusive scan of the 256 per-thread values of a block; returns this thread's prefix and
// the block total through `total`.
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
    for (int w = 0; w < kScanThreads / kWave; ++w) {
        uint32_t s = s_wave[w];
        if (w < wave) wave_base += s;
        total += s;
    }
    __syncthreads();
    return wave_base + incl - v;
}

__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(const uint32_t* __restrict__ in, int64_t n,
                                                                   uint32_t* __restrict__ partials) {
    __shared__ uint32_t s_wave[kScanThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kScanChunk;
    uint32_t sum = 0;
#pragma unroll
    for (int r = 0; r < kScanItems; ++r) {
        int64_t i = base + (int64_t)r * kScanThreads + threadIdx.x;
        if (i < n) sum += in[i];
    }
    uint32_t total;
    (void)block_exclusive_scan_256(sum, s_wave, total);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Single workgroup: exclusive scan of `count` partial sums in place; grand total at [count].
__global__ __launch_bounds__(kScanThreads) void scan_partials_kernel(uint32_t* __restrict__ partials, int64_t count) {
    __shared__ uint32_t s_wave[kScanThreads / kWave];
    uint32_t carry = 0;
    for (int64_t base = 0; base < count; base += kScanChunk) {
        uint32_t vals[kScanItems];
        uint32_t sum = 0;
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            int64_t i = base + (int64_t)threadIdx.x * kScanItems + k;
            vals[k] = i < count ? partials[i] : 0u;
            sum += vals[k];
        }
        uint32_t total;
        uint32_t prefix = block_exclusive_scan_256(sum, s_wave, total) + carry;
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            int64_t i = base + (int64_t)threadIdx.x * kScanItems + k;
            if (i < count) partials[i] = prefix;
            prefix += vals[k];
        }
        carry += total;
    }
    if (threadIdx.x == 0) partials[count] = carry;
}

__global__ __launch_bounds__(kScanThreads) void scan_downsweep_kernel(const uint32_t* __restrict__ in, int64_t n,
                                                                      const uint32_t* __restrict__ partials,
                                                                      uint32_t* __restrict__ out) {
    __shared__ uint32_t s_wave[kScanThreads / kWave];
    const int64_t base = (int64_t)blockIdx.x * kScanChunk + (int64_t)threadIdx.x * kScanItems;
    uint32_t vals[kScanItems];
    uint32_t sum = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        int64_t i = base + k;
        vals[k] = i < n ? in[i] : 0u;
        sum += vals[k];
    }
    uint32_t total;
    uint32_t prefix = block_exclusive_scan_256(sum, s_wave, total) + partials[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        int64_t i = base + k;
        if (i < n) out[i] = prefix;
        prefix += vals[k];
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) {
        out[n] = partials[gridDim.x];  // grand total after the last element
    }
}

__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(const uint64_t* __restrict__ keys, int64_t n,
                                                                  int shift, int64_t num_blocks,
                                                                  uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_hist[kRadix];
    s_hist[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortChunk;
#pragma unroll 4
    for (int r = 0; r < kSortRounds; ++r) {
        int64_t i = base + (int64_t)r * kSortThreads + threadIdx.x;
        if (i < n) {
            uint32_t d = (uint32_t)(keys[i] >> shift) & (kRadix - 1);
            atomicAdd(&s_hist[d], 1u);
        }
    }
    __syncthreads();
    hist[(int64_t)threadIdx.x * num_blocks + blockIdx.x] = s_hist[threadIdx.x];
}

__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const uint64_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n, int shift,
    int64_t num_blocks, const uint32_t* __restrict__ offsets, uint64_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out) {
    __shared__ uint32_t s_base[kRadix];                       // global base of each digit for this block
    __shared__ uint32_t s_wave_cnt[kSortThreads / kWave][kRadix];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    s_base[threadIdx.x] = offsets[(int64_t)threadIdx.x * num_blocks + blockIdx.x];
    const int64_t base = (int64_t)blockIdx.x * kSortChunk;
    const uint64_t lt = lanemask_lt();
    for (int r = 0; r < kSortRounds; ++r) {
        const int64_t i = base + (int64_t)r * kSortThreads + threadIdx.x;
        const bool valid = i < n;
        uint64_t key = 0;
        uint32_t val = 0;
        uint32_t d = 0;
        if (valid) {
            key = keys_in[i];
            val = vals_in[i];
            d = (uint32_t)(key >> shift) & (kRadix - 1);
        }
#pragma unroll
        for (int w = 0; w < kSortThreads / kWave; ++w) s_wave_cnt[w][threadIdx.x] = 0;
        __syncthreads();
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < kRadixBits; ++b) {
            const bool bit = ((d >> b) & 1u) != 0;
            const uint64_t m = __ballot(valid && bit);
            peers &= bit ? m : ~m;
        }
        const uint32_t rank = (uint32_t)__popcll(peers & lt);
        if (valid && rank == 0) s_wave_cnt[wave][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        {
            // thread t owns digit t: turn per-wave counts into per-wave bases, advance s_base
            const uint32_t c0 = s_wave_cnt[0][threadIdx.x];
            const uint32_t c1 = s_wave_cnt[1][threadIdx.x];
            const uint32_t c2 = s_wave_cnt[2][threadIdx.x];
            const uint32_t c3 = s_wave_cnt[3][threadIdx.x];
            const uint32_t b0 = s_base[threadIdx.x];
            s_wave_cnt[0][threadIdx.x] = b0;
            s_wave_cnt[1][threadIdx.x] = b0 + c0;
            s_wave_cnt[2][threadIdx.x] = b0 + c0 + c1;
            s_wave_cnt[3][threadIdx.x] = b0 + c0 + c1 + c2;
            s_base[threadIdx.x] = b0 + c0 + c1 + c2 + c3;
        }
        __syncthreads();
        if (valid) {
            const uint32_t pos = s_wave_cnt[wave][d] + rank;
            keys_out[pos] = key;
            vals_out[pos] = val;
        }
        __syncthreads();
    }
    (void)lane;
}

}  // namespace gsx_amd

using namespace gsx_amd;

extern "C" {

size_t gsx_hip_scan_temp_bytes(int64_t n) {
    int64_t blocks = (n + kScanChunk - 1) / kScanChunk;
    if (blocks < 1) blocks = 1;
    return (size_t)(blocks + 1) * sizeof(uint32_t);
}

// out[0..n) = exclusive prefix sums of in[0..n), out[n] = total. out may not alias in.
gsx_hip_status gsx_hip_scan_exclusive_u32(const uint32_t* in, uint32_t* out, int64_t n, void* temp, hipStream_t stream) {
    int64_t blocks = (n + kScanChunk - 1) / kScanChunk;
    if (blocks < 1) blocks = 1;
    uint32_t* partials = static_cast<uint32_t*>(temp);
    hipLaunchKernelGGL(scan_reduce_kernel, dim3((unsigned)blocks), dim3(kScanThreads), 0, stream, in, n, partials);
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanThreads), 0, stream, partials, blocks);
    hipLaunchKernelGGL(scan_downsweep_kernel, dim3((unsigned)blocks), dim3(kScanThreads), 0, stream, in, n, partials,
                       out);
    return (gsx_hip_status)hipGetLastError();
}

size_t gsx_hip_radix_sort_temp_bytes(int64_t n) {
    int64_t blocks = (n + kSortChunk - 1) / kSortChunk;
    if (blocks < 1) blocks = 1;
    const int64_t hist_count = blocks * kRadix;
    // hist + scanned offsets (hist_count + 1) + scan partials
    return (size_t)(hist_count + hist_count + 1) * sizeof(uint32_t) + gsx_hip_scan_temp_bytes(hist_count) + 256;
}

// Stable LSD sort of n pairs on key bits [begin_bit, end_bit). The result ends in (keys, vals)
// when *out_in_alt == 0, else in (keys_alt, vals_alt).
gsx_hip_status gsx_hip_radix_sort_pairs_u64(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt,
                                        int64_t n, int begin_bit, int end_bit, void* temp, int* out_in_alt,
                                        hipStream_t stream) {
    int64_t blocks = (n + kSortChunk - 1) / kSortChunk;
    if (blocks < 1) blocks = 1;
    const int64_t hist_count = blocks * kRadix;
    uint32_t* hist = static_cast<uint32_t*>(temp);
    uint32_t* offsets = hist + hist_count;
    void* scan_temp = offsets + hist_count + 1;
    int in_alt = 0;
    if (n > 0) {
        for (int shift = begin_bit; shift < end_bit; shift += kRadixBits) {
            uint64_t* kin = in_alt ? keys_alt : keys;
            uint32_t* vin = in_alt ? vals_alt : vals;
            uint64_t* kout = in_alt ? keys : keys_alt;
            uint32_t* vout = in_alt ? vals : vals_alt;
            hipLaunchKernelGGL(radix_hist_kernel, dim3((unsigned)blocks), dim3(kSortThreads), 0, stream, kin, n,
                               shift, blocks, hist);
            gsx_hip_status e = gsx_hip_scan_exclusive_u32(hist, offsets, hist_count, scan_temp, stream);
            if (e != GSX_HIP_SUCCESS) return e;
            hipLaunchKernelGGL(radix_scatter_kernel, dim3((unsigned)blocks), dim3(kSortThreads), 0, stream, kin, vin,
                               n, shift, blocks, offsets, kout, vout);
            in_alt ^= 1;
        }
    }
    if (out_in_alt) *out_in_alt = in_alt;
    return (gsx_hip_status)hipGetLastError();
}

}  // extern "C"
