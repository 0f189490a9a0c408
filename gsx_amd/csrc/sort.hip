// sort.hip - device-wide exclusive scan and stable LSD radix sort of (u64 key, u32 value) pairs.
//
// Replaces cub::DeviceScan::ExclusiveSum (gsx/src/gsx-cuda/fastgs/forward.cu:180-185) and
// cub::DeviceRadixSort::SortPairs (forward.cu:155-161, 214-220).
//
// Radix sort: 8-bit digits, LSD, stable (the tile lists rely on it: equal (tile, depth) keys keep
// Gaussian order); see the pass description above radix_upsweep_kernel.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "../../include/gsx_hip.h"

namespace gsx_amd {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 4;
constexpr int kScanChunk = kScanThreads * kScanItems;  // 1024 elements per block

constexpr int kSortChunk = 4096;  // keys per chunk (one upsweep / downsweep workgroup), public sorts
constexpr int kRadixBits = 8;     // digit width of the public sorts
// Chunks of the tile sort's passes (tile_sort_u32): 4096 keys below kLargeTileSort keys, 8192
// from there on (runs of a digit twice as long per workgroup: each workgroup's writes meet half as
// many distinct places of the output per byte, and the histograms and row scans halve; below it
// the larger chunk leaves too few workgroups to fill the GPU). The downsweep runs chunk / 8
// threads, 8 keys per thread.
constexpr int kDigitsChunk = 4096;
constexpr int kDigitsChunkLarge = 8192;
constexpr int64_t kLargeTileSort = (int64_t)1 << 24;
constexpr int kRowItems = 16;  // row scan: 16 chunk counts per thread and step
constexpr int kRowChunk = kSortThreads * kRowItems;

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
// A step covers 16 values per thread (4096: the block sums of 1M ranks in one step); wave w
// takes the step's w-th run of 1024 as 16 coalesced groups of 64, each scanned with DPP, and the
// next step's values are loaded before the current step's are written.
constexpr int kPartialItems = 16;
// Workgroup b scans the b-th of gridDim.x arrays of count + 1 entries laid out back to back.
__global__ __launch_bounds__(kScanThreads) void scan_partials_kernel(uint32_t* __restrict__ partials, int64_t count) {
    constexpr int kWaves = kScanThreads / kWave;
    constexpr int64_t kStep = (int64_t)kScanThreads * kPartialItems;
    __shared__ uint32_t s_wave[kWaves];
    partials += (int64_t)blockIdx.x * (count + 1);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int64_t first = (int64_t)wave * kWave * kPartialItems + lane;
    uint32_t carry = 0;
    uint32_t next[kPartialItems];
#pragma unroll
    for (int j = 0; j < kPartialItems; ++j) {
        const int64_t i = first + j * kWave;
        next[j] = i < count ? partials[i] : 0u;
    }
    for (int64_t base = 0; base < count; base += kStep) {
        uint32_t excl[kPartialItems];
        uint32_t run = 0;
#pragma unroll
        for (int j = 0; j < kPartialItems; ++j) {
            const uint32_t v = next[j];
            const uint32_t incl = wave_inclusive_sum_u32(v);
            excl[j] = run + incl - v;
            run += (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
        }
#pragma unroll
        for (int j = 0; j < kPartialItems; ++j) {
            const int64_t i = base + kStep + first + j * kWave;
            next[j] = i < count ? partials[i] : 0u;
        }
        if (lane == 0) s_wave[wave] = run;
        __syncthreads();
        uint32_t wave_base = carry, total = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t sw = s_wave[w];
            if (w < wave) wave_base += sw;
            total += sw;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kPartialItems; ++j) {
            const int64_t i = base + first + j * kWave;
            if (i < count) partials[i] = wave_base + excl[j];
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

// ---------------------------------------------------------------------------------------------
// One LSD pass on the kBits-bit digit at `shift` (8, or 9 for the compacting sort: 512 bins,
// three passes for 27 depth bits), reduce-then-scan, three launches:
//   upsweep: digit counts of each chunk (4096 keys, 2048 in the depth order) -> hist[digit][chunk]
//   rowscan: one workgroup per digit scans its row over the chunks    -> offsets, totals[digit]
//   downsweep: 8 waves each rank an eighth of the chunk (rounds of 64 keys) stably with kBits
//      ballots per round and wave-private digit counters; the chunk is then reordered by digit
//      in LDS and written out in order, so consecutive lanes store consecutive addresses of one
//      digit's run.
// Stability: a chunk's keys keep input order within a digit (waves own consecutive eighths,
// rounds and lanes follow input order), and chunks are laid out in order inside each digit.
// No workgroup waits on another, so every wave runs to completion.
// ---------------------------------------------------------------------------------------------
// n_dev (may be null): live key count, n = min(n, *n_dev); chunks past it count nothing.
// drop_sentinel: keys equal to kSentinelKey are left out (they vanish from the output).
template <int kBits, int kChunk, typename KeyT = uint64_t>
__global__ __launch_bounds__(kSortThreads) void radix_upsweep_kernel(const KeyT* __restrict__ keys, int64_t n,
                                                                     const uint32_t* __restrict__ n_dev,
                                                                     bool drop_sentinel, int shift,
                                                                     uint32_t dmask, int64_t num_chunks,
                                                                     uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_hist[kUpsweepHistWords<kBits>];
    const int64_t chunk = sort_chunk_of(blockIdx.x, num_chunks);
    if (chunk >= num_chunks) return;  // uniform
    radix_upsweep_block<kBits, kChunk, KeyT>((uint32_t)chunk, keys, n, n_dev, drop_sentinel, shift, num_chunks, hist,
                                             s_hist, dmask);
}

// Workgroup d: exclusive scan of hist[d][0..num_chunks) into offsets[d][..], row total into
// totals[d]. A step covers kThreads * kRowItems counts; wave w takes the step's w-th run of
// 64 * kRowItems, as kRowItems coalesced groups of 64 (one count per lane), each scanned with DPP
// and carried into the next. The next step's counts are loaded before the current step's scan,
// so the row's serial steps overlap their loads. Long rows (config 4's tile sort: 82k chunks) run
// 1024 threads, short ones 256.
template <int kThreads>
__global__ __launch_bounds__(kThreads) void radix_rowscan_kernel(const uint32_t* __restrict__ hist,
                                                                 int64_t num_chunks,
                                                                 uint32_t* __restrict__ offsets,
                                                                 uint32_t* __restrict__ totals) {
    constexpr int kWaveRun = kWave * kRowItems;
    constexpr int kStep = kThreads * kRowItems;
    constexpr int kWaves = kThreads / kWave;
    __shared__ uint32_t s_wave[kWaves];
    const uint32_t* row = hist + (int64_t)blockIdx.x * num_chunks;
    uint32_t* out = offsets + (int64_t)blockIdx.x * num_chunks;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int64_t first = (int64_t)wave * kWaveRun + lane;  // this lane's first count of a step
    uint32_t carry = 0;
    uint32_t next[kRowItems];
#pragma unroll
    for (int j = 0; j < kRowItems; ++j) {
        const int64_t i = first + j * kWave;
        next[j] = i < num_chunks ? row[i] : 0u;
    }
    for (int64_t base = 0; base < num_chunks; base += kStep) {
        uint32_t excl[kRowItems];
        uint32_t run = 0;
#pragma unroll
        for (int j = 0; j < kRowItems; ++j) {
            const uint32_t v = next[j];
            const uint32_t incl = wave_inclusive_sum_u32(v);
            excl[j] = run + incl - v;
            run += (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
        }
#pragma unroll
        for (int j = 0; j < kRowItems; ++j) {
            const int64_t i = base + kStep + first + j * kWave;
            next[j] = i < num_chunks ? row[i] : 0u;
        }
        if (lane == 0) s_wave[wave] = run;
        __syncthreads();
        uint32_t wave_base = carry, total = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t sw = s_wave[w];
            if (w < wave) wave_base += sw;
            total += sw;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kRowItems; ++j) {
            const int64_t i = base + first + j * kWave;
            if (i < num_chunks) out[i] = wave_base + excl[j];
        }
        carry += total;
    }
    if (threadIdx.x == 0) totals[blockIdx.x] = carry;
}

// Row scan launch for `bins` rows of num_chunks counts.
inline void launch_rowscan(int bins, const uint32_t* hist, int64_t num_chunks, uint32_t* offsets, uint32_t* totals,
                           hipStream_t stream) {
    if (num_chunks > 4 * kRowChunk) {
        hipLaunchKernelGGL(radix_rowscan_kernel<1024>, dim3(bins), dim3(1024), 0, stream, hist, num_chunks, offsets,
                           totals);
    } else {
        hipLaunchKernelGGL(radix_rowscan_kernel<kSortThreads>, dim3(bins), dim3(kSortThreads), 0, stream, hist,
                           num_chunks, offsets, totals);
    }
}

// The downsweep runs 512 threads (8 waves of 512 keys, 8 rounds each): the serial ranking chain
// of a chunk is half as long as with 4 waves.
constexpr int kDownThreads = 512;

// Exclusive scan over the kBins digits held by threads 0..kBins-1 of the workgroup
// (threads past kBins pass 0 and get garbage); `total` receives the sum over the digits.
template <int kBins>
__device__ inline uint32_t digit_exclusive_scan(uint32_t v, uint32_t* s_wave, uint32_t& total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += o;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    uint32_t wave_base = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < kBins / kWave; ++w) {
        const uint32_t sw = s_wave[w];
        if (w < wave) wave_base += sw;
        total += sw;
    }
    __syncthreads();
    return wave_base + incl - v;
}

// KeyT: uint64_t or uint32_t keys. kPairs with vals_in == nullptr: each key's value is its input
// position (the first pass of the tile sort, whose values are the emission positions). kNarrow:
// n * sizeof(KeyT) <= 2^32, so every output byte offset fits in 32 bits. kThreads: workgroup size
// (kChunk / kThreads keys per thread). Register target: 8 waves per SIMD, except for 64-bit keys
// with values, whose 54 KB of LDS admits two workgroups (4 waves per SIMD) per CU anyway.
template <bool kPairs, int kBits, int kChunk, typename KeyT = uint64_t, bool kNarrow = false,
          int kThreads = kDownThreads>
__global__ __launch_bounds__(kThreads, (kPairs && sizeof(KeyT) == 8) ? 4 : 8) void radix_downsweep_kernel(
    const KeyT* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n,
    const uint32_t* __restrict__ n_dev, bool drop_sentinel, int shift, uint32_t dmask, int64_t num_chunks,
    const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ totals, KeyT* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, uint32_t* __restrict__ kept_total) {
    constexpr int kWaves = kThreads / kWave;
    constexpr int kDownWaveKeys = kChunk / kWaves;  // keys ranked by one wave
    constexpr int kDownRounds = kDownWaveKeys / kWave;
    static_assert(kDownRounds >= 1 && kDownWaveKeys % kWave == 0, "whole rounds per wave");
    // the reordered chunk: 32-bit keys with values as one 64-bit entry per key (one scatter
    // store instead of two), otherwise keys (and values) in arrays of their own
    constexpr bool kPack = kPairs && sizeof(KeyT) == 4;
    __shared__ uint64_t s_kv[kPack ? kChunk : 1];
    __shared__ KeyT s_keys[kPack ? 1 : kChunk];
    __shared__ uint32_t s_vals[(kPairs && !kPack) ? kChunk : 1];
    constexpr int kBins = 1 << kBits;
    static_assert(kBins <= kThreads, "one thread per digit");
    // wave-private digit counters, then wave starts. Up to 256 digits they are 16-bit halves
    // (values stay below kChunk <= 2^16): digit d sits in half d / kHalf of dword d % kHalf, so
    // the two digits of a dword share one bank and lanes reading either are served by one access
    // of it (as full dwords, digits d and d + 64 fall on one bank at different addresses; tile
    // sort downsweep 25.3 -> 21.5 us on the metric scene). The 512 digits of the depth sort keep
    // full dwords: their extra address arithmetic cost more than the fewer conflicts saved.
    constexpr bool kCnt16 = kBits <= 8;
    constexpr int kHalf = kCnt16 ? kBins / 2 : kBins;
    static_assert(!kCnt16 || kChunk <= 65536, "16-bit counters");
    __shared__ uint32_t s_cnt32[kWaves][kHalf];
    using CntT = std::conditional_t<kCnt16, uint16_t, uint32_t>;
    auto cnt = [&](int w, uint32_t d) -> CntT& {
        if constexpr (kCnt16) return reinterpret_cast<uint16_t*>(&s_cnt32[w][0])[2 * (d % kHalf) + d / kHalf];
        else return s_cnt32[w][d];
    };
    // output position of the reordered chunk's position 0 as counted in each digit: the digit's
    // run starts at s_out[d] + (its start in the reordered chunk) (modulo 2^32)
    __shared__ uint32_t s_out[kBins];
    __shared__ uint32_t s_wave[kWaves];
    __shared__ uint32_t s_kept;                     // keys of the chunk that are moved
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t chunk = sort_chunk_of(blockIdx.x, num_chunks);
    if (chunk >= num_chunks) return;  // uniform
    const int64_t base = chunk * kChunk;
    if (n_dev != nullptr) n = min(n, (int64_t)*n_dev);
    if (base >= n) return;  // uniform: a chunk past the live count has nothing to move
    const int chunk_count = (int)min((int64_t)kChunk, n - base);
    // this chunk's digit offsets and the digit totals, loaded with the keys (threads past kBins
    // re-read digit kBins - 1 and ignore it)
    const int td = min((int)threadIdx.x, kBins - 1);
    const uint32_t my_total = totals[td];
    const uint32_t my_offset = offsets[(int64_t)td * num_chunks + chunk];
    for (int i = threadIdx.x; i < kWaves * kHalf; i += kThreads) (&s_cnt32[0][0])[i] = 0;
    __syncthreads();
    // 1. per wave: stable ranks among equal digits (rank = keys of the digit before it in this
    //    wave's eighth of the chunk), packed as digit << 16 | rank
    const uint64_t lt = lanemask_lt();
    KeyT key[kDownRounds];
    uint32_t val[kDownRounds];
    uint32_t dr[kDownRounds];
#pragma unroll
    for (int r = 0; r < kDownRounds; ++r) {
        const int local = wave * kDownWaveKeys + r * kWave + lane;
        const bool valid = local < chunk_count;
        key[r] = valid ? keys_in[base + local] : (KeyT)0;
        if (kPairs) val[r] = vals_in == nullptr ? (uint32_t)(base + local) : (valid ? vals_in[base + local] : 0u);
        else val[r] = 0u;
    }
#pragma unroll
    for (int r = 0; r < kDownRounds; ++r) {
        const int local = wave * kDownWaveKeys + r * kWave + lane;
        const bool valid = local < chunk_count && !(drop_sentinel && (uint64_t)key[r] == kSentinelKey);
        const uint32_t d = digit_of<kBits>(key[r], shift) & dmask;
        const uint64_t vm = wave_ballot(valid);
        // per digit bit: the bit as 0 / all ones (a signed bit-field extract) and the wave's ballot
        // of it; the lanes that agree with this lane in bit b are ~(ballot ^ ext), folded into the
        // peer mask with one three-input bitwise operation per half (truth table 0x90:
        // p & ~(m ^ e))
        uint32_t ext[kBits];
        uint64_t m[kBits];
#pragma unroll
        for (int b = 0; b < kBits; ++b) {
            ext[b] = (uint32_t)((int32_t)(d << (31 - b)) >> 31);
            asm volatile("" : "+v"(ext[b]));  // the ballot compares the extracted bit itself
        }
#pragma unroll
        for (int b = 0; b < kBits; ++b) m[b] = wave_ballot(ext[b] != 0u);
        uint32_t plo = (uint32_t)vm, phi = (uint32_t)(vm >> 32);
#pragma unroll
        for (int b = 0; b < kBits; ++b) {
            plo = __builtin_amdgcn_bitop3_b32(plo, (uint32_t)m[b], ext[b], 0x90);
            phi = __builtin_amdgcn_bitop3_b32(phi, (uint32_t)(m[b] >> 32), ext[b], 0x90);
        }
        const uint64_t peers = (uint64_t)plo | ((uint64_t)phi << 32);
        const uint32_t before = cnt(wave, d);  // read by all lanes before the leader updates
        const uint32_t rank = (uint32_t)__popcll(peers & lt);
        if (valid && rank == 0) cnt(wave, d) = (CntT)(before + (uint32_t)__popcll(peers));
        __builtin_amdgcn_wave_barrier();
        dr[r] = valid ? (d << 16) | (before + rank) : 0xffffffffu;
        // formed here, so that the peer masks die with the round (not kept alive for the reorder)
        asm volatile("" : "+v"(dr[r]));
    }
    __syncthreads();
    // 2. threads 0..255 = digits: wave starts inside the digit, digit starts inside the chunk,
    //    and the digit's output position for this chunk
    {
        const int t = threadIdx.x;
        uint32_t total_cnt = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) total_cnt += t < kBins ? (uint32_t)cnt(w, t) : 0u;
        uint32_t kept, all_kept;
        const uint32_t start = digit_exclusive_scan<kBins>(total_cnt, s_wave, kept);
        const uint32_t digit_base = digit_exclusive_scan<kBins>(t < kBins ? my_total : 0u, s_wave, all_kept);
        if (t == 0) s_kept = kept;
        // the number of keys this pass keeps, for the later passes (a plain store: one writer)
        if (kept_total != nullptr && chunk == 0 && t == 0) *kept_total = all_kept;
        if (t < kBins) {
            s_out[t] = digit_base + my_offset - start;
            uint32_t run = start;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const uint32_t c = cnt(w, t);
                cnt(w, t) = (CntT)run;
                run += c;
            }
        }
    }
    __syncthreads();
    // 3. reorder the chunk by digit in LDS
#pragma unroll
    for (int r = 0; r < kDownRounds; ++r) {
        if (dr[r] != 0xffffffffu) {
            const uint32_t pos = (uint32_t)cnt(wave, dr[r] >> 16) + (dr[r] & 0xffffu);
            if (kPack) {
                s_kv[pos] = (uint64_t)key[r] | ((uint64_t)val[r] << 32);
            } else {
                s_keys[pos] = key[r];
                if (kPairs) s_vals[pos] = val[r];
            }
        }
    }
    __syncthreads();
    // 4. write out in order: runs of one digit go to consecutive addresses. Every LDS read of the
    //    thread's keys is issued before the first store; kNarrow: byte offsets of the output fit
    //    in 32 bits (stores address a scalar base plus a 32-bit offset).
    constexpr int kOutRounds = kChunk / kThreads;
    const int kept_count = (int)s_kept;
    KeyT ok[kOutRounds];
    uint32_t ov[kOutRounds];
    uint32_t opos[kOutRounds];
#pragma unroll
    for (int j = 0; j < kOutRounds; ++j) {
        const int i = (int)threadIdx.x + j * kThreads;
        if (kPack) {
            const uint64_t kv = s_kv[i];
            ok[j] = (KeyT)(uint32_t)kv;
            ov[j] = (uint32_t)(kv >> 32);
        } else {
            ok[j] = s_keys[i];
            ov[j] = kPairs ? s_vals[i] : 0u;
        }
    }
#pragma unroll
    for (int j = 0; j < kOutRounds; ++j) {
        const int i = (int)threadIdx.x + j * kThreads;
        opos[j] = s_out[digit_of<kBits>(ok[j], shift) & dmask] + (uint32_t)i;
    }
#pragma unroll
    for (int j = 0; j < kOutRounds; ++j) {
        const int i = (int)threadIdx.x + j * kThreads;
        if (i < kept_count) {
            if (kNarrow) {
                *reinterpret_cast<KeyT*>(reinterpret_cast<char*>(keys_out) + (uint32_t)(opos[j] * sizeof(KeyT))) =
                    ok[j];
                if (kPairs) *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(vals_out) + (opos[j] << 2)) = ov[j];
            } else {
                keys_out[opos[j]] = ok[j];
                if (kPairs) vals_out[opos[j]] = ov[j];
            }
        }
    }
}

}  // namespace gsx_amd

using namespace gsx_amd;

namespace {

// n_dev: see radix_upsweep_kernel. compact_first: the first pass reads all n keys and drops the
// sentinel keys (stably compacting the rest to the front), its downsweep stores the number of
// kept keys in *n_dev, and the later passes sort that many.
// Output byte offsets of n keys of key_bytes bytes (and of their 4-byte values) fit in 32 bits.
inline bool narrow_offsets(int64_t n, size_t key_bytes) {
    return (uint64_t)n * key_bytes <= (uint64_t)1 << 32;
}

template <int kBits, int kChunk>
size_t radix_temp_bytes(int64_t n) {
    int64_t chunks = (n + kChunk - 1) / kChunk;
    if (chunks < 1) chunks = 1;
    const int64_t hist_count = chunks * (1 << kBits);
    // hist + offsets + totals
    return (size_t)(2 * hist_count + (1 << kBits)) * sizeof(uint32_t) + 256;
}

template <bool kPairs, int kBits, int kChunk>
gsx_hip_status radix_sort_u64(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt, int64_t n,
                              uint32_t* n_dev, bool compact_first, int begin_bit, int end_bit, void* temp,
                              int* out_in_alt, hipStream_t stream) {
    constexpr int kBins = 1 << kBits;
    if (begin_bit < 0 || end_bit > 64 || begin_bit > end_bit) return GSX_HIP_ERROR_INVALID_ARGUMENT;
    if (n > (int64_t)UINT32_MAX) return GSX_HIP_ERROR_OUT_OF_RANGE;
    int64_t chunks = (n + kChunk - 1) / kChunk;
    if (chunks < 1) chunks = 1;
    const int64_t hist_count = chunks * kBins;
    uint32_t* hist = static_cast<uint32_t*>(temp);
    uint32_t* offsets = hist + hist_count;
    uint32_t* totals = offsets + hist_count;
    int in_alt = 0;
    if (n > 0) {
        for (int shift = begin_bit; shift < end_bit; shift += kBits) {
            uint64_t* kin = in_alt ? keys_alt : keys;
            uint32_t* vin = in_alt ? vals_alt : vals;
            uint64_t* kout = in_alt ? keys : keys_alt;
            uint32_t* vout = in_alt ? vals : vals_alt;
            const bool drop = compact_first && shift == begin_bit;
            const uint32_t* live = drop ? nullptr : n_dev;
            // the last pass may be narrower than kBits: bits at and above end_bit do not sort
            const int width = end_bit - shift < kBits ? end_bit - shift : kBits;
            const uint32_t dmask = (1u << width) - 1u;
            hipLaunchKernelGGL((radix_upsweep_kernel<kBits, kChunk>), dim3(sort_chunk_grid(chunks)), dim3(kSortThreads),
                               0, stream, kin, n, live, drop, shift, dmask, chunks, hist);
            launch_rowscan(kBins, hist, chunks, offsets, totals, stream);
            if (narrow_offsets(n, sizeof(uint64_t))) {
                hipLaunchKernelGGL((radix_downsweep_kernel<kPairs, kBits, kChunk, uint64_t, true>),
                                   dim3(sort_chunk_grid(chunks)), dim3(kDownThreads), 0, stream, kin, vin, n, live,
                                   drop, shift, dmask, chunks, offsets, totals, kout, vout, drop ? n_dev : nullptr);
            } else {
                hipLaunchKernelGGL((radix_downsweep_kernel<kPairs, kBits, kChunk, uint64_t, false>),
                                   dim3(sort_chunk_grid(chunks)), dim3(kDownThreads), 0, stream, kin, vin, n, live,
                                   drop, shift, dmask, chunks, offsets, totals, kout, vout, drop ? n_dev : nullptr);
            }
            in_alt ^= 1;
        }
    }
    if (out_in_alt) *out_in_alt = in_alt;
    return (gsx_hip_status)hipGetLastError();
}

}  // namespace

namespace gsx_amd {
void set_last_error(const char* what);
}

// Partial sums of gsx_hip_scan_exclusive_u32_noalloc: one per 1024-element block plus the total,
// for at most kNoallocScanMaxBlocks blocks (256 KiB). Each GPU the library runs on holds its
// own copy until the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (scratch_address), never by its name.
constexpr int64_t kNoallocScanMaxBlocks = 65536;
constexpr int64_t kNoallocScanMaxElements = kNoallocScanMaxBlocks * kScanChunk;
static __device__ __align__(256) uint32_t scratch[kNoallocScanMaxBlocks + 1];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint32_t* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
gsx_hip_status scratch_address(uint32_t** out) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) {
        set_last_error("scan without allocation: hipGetDevice failed");
        return (gsx_hip_status)e;
    }
    if (device < 0 || device >= kMaxDevices) {
        set_last_error("scan without allocation: device ordinal above 63");
        return GSX_HIP_ERROR_OUT_OF_RANGE;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[device] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_last_error("scan without allocation: hipGetSymbolAddress(scratch) failed");
            return e != hipSuccess ? (gsx_hip_status)e : GSX_HIP_ERROR_INVALID_STATE;
        }
        g_scratch[device] = static_cast<uint32_t*>(p);
    }
    *out = g_scratch[device];
    return GSX_HIP_SUCCESS;
}

// The three launches of the exclusive scan with the partial sums (blocks + 1 words) at `partials`.
gsx_hip_status scan_exclusive_u32(const uint32_t* in, uint32_t* out, int64_t n, uint32_t* partials,
                                  hipStream_t stream) {
    int64_t blocks = (n + kScanChunk - 1) / kScanChunk;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(scan_reduce_kernel, dim3((unsigned)blocks), dim3(kScanThreads), 0, stream, in, n, partials);
    hipLaunchKernelGGL(scan_partials_kernel, dim3(1), dim3(kScanThreads), 0, stream, partials, blocks);
    hipLaunchKernelGGL(scan_downsweep_kernel, dim3((unsigned)blocks), dim3(kScanThreads), 0, stream, in, n, partials,
                       out);
    return (gsx_hip_status)hipGetLastError();
}

}  // namespace

extern "C" {

size_t gsx_hip_scan_temp_bytes(int64_t n) {
    int64_t blocks = (n + kScanChunk - 1) / kScanChunk;
    if (blocks < 1) blocks = 1;
    return (size_t)(blocks + 1) * sizeof(uint32_t);
}

// out[0..n) = exclusive prefix sums of in[0..n), out[n] = total. out may not alias in.
gsx_hip_status gsx_hip_scan_exclusive_u32(const uint32_t* in, uint32_t* out, int64_t n, void* temp, hipStream_t stream) {
    return scan_exclusive_u32(in, out, n, static_cast<uint32_t*>(temp), stream);
}

// The same scan with its partial sums in `scratch` (see above): no allocation, no workspace.
gsx_hip_status gsx_hip_scan_exclusive_u32_noalloc(const uint32_t* in, uint32_t* out, int64_t n, hipStream_t stream) {
    if (n < 0 || out == nullptr || (in == nullptr && n > 0)) {
        set_last_error("scan: out must be non-null, in non-null when n > 0, n >= 0");
        return GSX_HIP_ERROR_INVALID_ARGUMENT;
    }
    if (n > kNoallocScanMaxElements) {
        set_last_error("scan without allocation: n exceeds the static scratch (at most 67108864 elements)");
        return GSX_HIP_ERROR_OUT_OF_RANGE;
    }
    uint32_t* partials = nullptr;
    const gsx_hip_status st = scratch_address(&partials);
    if (st != GSX_HIP_SUCCESS) return st;
    return scan_exclusive_u32(in, out, n, partials, stream);
}

size_t gsx_hip_radix_sort_temp_bytes(int64_t n) { return radix_temp_bytes<kRadixBits, kSortChunk>(n); }

// Stable LSD sort of n pairs on key bits [begin_bit, end_bit). The result ends in (keys, vals)
// when *out_in_alt == 0, else in (keys_alt, vals_alt).
gsx_hip_status gsx_hip_radix_sort_pairs_u64(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt,
                                            int64_t n, int begin_bit, int end_bit, void* temp, int* out_in_alt,
                                            hipStream_t stream) {
    return radix_sort_u64<true, kRadixBits, kSortChunk>(keys, vals, keys_alt, vals_alt, n, nullptr, false, begin_bit,
                                                        end_bit, temp, out_in_alt, stream);
}

// Stable LSD sort of n keys on bits [begin_bit, end_bit); bits outside the range travel with
// the key (a payload packed into the low bits keeps input order among equal sort bits).
gsx_hip_status gsx_hip_radix_sort_keys_u64(uint64_t* keys, uint64_t* keys_alt, int64_t n, int begin_bit, int end_bit,
                                           void* temp, int* out_in_alt, hipStream_t stream) {
    return radix_sort_u64<false, kRadixBits, kSortChunk>(keys, nullptr, keys_alt, nullptr, n, nullptr, false,
                                                         begin_bit, end_bit, temp, out_in_alt, stream);
}

}  // extern "C"

namespace gsx_amd {

gsx_hip_status scan_partials_in_place(uint32_t* partials, int64_t count, hipStream_t stream, int arrays) {
    hipLaunchKernelGGL(scan_partials_kernel, dim3((unsigned)arrays), dim3(kScanThreads), 0, stream, partials, count);
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status radix_sort_keys_u64_compacting(uint64_t* keys, uint64_t* keys_alt, int64_t n, uint32_t* n_live,
                                              int begin_bit, int end_bit, void* temp, int* out_in_alt,
                                              hipStream_t stream) {
    if (begin_bit >= end_bit) return GSX_HIP_ERROR_INVALID_ARGUMENT;  // the compacting pass must run
    return radix_sort_u64<false, kCompactingRadixBits, kCompactingChunk>(keys, nullptr, keys_alt, nullptr, n, n_live,
                                                                         true, begin_bit, end_bit, temp, out_in_alt,
                                                                         stream);
}

template <int kBits, int kChunk>
gsx_hip_status tile_sort_passes(const uint32_t* tiles, uint32_t* tiles_alt, uint32_t* tiles_sorted, uint32_t* vals_alt,
                                uint32_t* vals_sorted, int64_t n, int tile_bits, int passes, void* temp,
                                hipStream_t stream) {
    constexpr int kBins = 1 << kBits;
    int64_t chunks = (n + kChunk - 1) / kChunk;
    if (chunks < 1) chunks = 1;
    const int64_t hist_count = chunks * kBins;
    uint32_t* hist = static_cast<uint32_t*>(temp);
    uint32_t* offsets = hist + hist_count;
    uint32_t* totals = offsets + hist_count;
    const uint32_t* kin = tiles;
    const uint32_t* vin = nullptr;  // first pass: the values are the input positions
    for (int k = 0; k < passes; ++k) {
        // the last pass lands in the sorted arrays, the one before it in the alternates, ...
        const bool to_sorted = (passes - 1 - k) % 2 == 0;
        uint32_t* kout = to_sorted ? tiles_sorted : tiles_alt;
        uint32_t* vout = to_sorted ? vals_sorted : vals_alt;
        const int shift = k * kBits;
        const int width = tile_bits - shift < kBits ? tile_bits - shift : kBits;
        const uint32_t dmask = width > 0 ? (1u << width) - 1u : 0u;
        hipLaunchKernelGGL((radix_upsweep_kernel<kBits, kChunk, uint32_t>), dim3(sort_chunk_grid(chunks)),
                           dim3(kSortThreads), 0, stream, kin, n, nullptr, false, shift, dmask, chunks, hist);
        launch_rowscan(kBins, hist, chunks, offsets, totals, stream);
        if (narrow_offsets(n, sizeof(uint32_t))) {
            hipLaunchKernelGGL((radix_downsweep_kernel<true, kBits, kChunk, uint32_t, true, kChunk / 8>),
                               dim3(sort_chunk_grid(chunks)), dim3(kChunk / 8), 0, stream, kin, vin, n, nullptr,
                               false, shift, dmask, chunks, offsets, totals, kout, vout, nullptr);
        } else {
            hipLaunchKernelGGL((radix_downsweep_kernel<true, kBits, kChunk, uint32_t, false, kChunk / 8>),
                               dim3(sort_chunk_grid(chunks)), dim3(kChunk / 8), 0, stream, kin, vin, n, nullptr,
                               false, shift, dmask, chunks, offsets, totals, kout, vout, nullptr);
        }
        kin = kout;
        vin = vout;
    }
    return (gsx_hip_status)hipGetLastError();
}

gsx_hip_status tile_sort_u32(const uint32_t* tiles, uint32_t* tiles_alt, uint32_t* tiles_sorted, uint32_t* vals_alt,
                             uint32_t* vals_sorted, int64_t n, int tile_bits, int passes, int digit_bits, void* temp,
                             hipStream_t stream) {
    if (n < 0 || n > (int64_t)UINT32_MAX || passes < 1 || tile_bits < 0 || tile_bits > passes * digit_bits ||
        tiles == tiles_sorted || tiles == tiles_alt) {
        return GSX_HIP_ERROR_INVALID_ARGUMENT;
    }
    if (n == 0) return GSX_HIP_SUCCESS;
#define GSX_TILE_SORT(B, C) \
    tile_sort_passes<B, C>(tiles, tiles_alt, tiles_sorted, vals_alt, vals_sorted, n, tile_bits, passes, temp, stream)
    const bool large = n >= kLargeTileSort;
    switch (digit_bits) {
        case 6: return large ? GSX_TILE_SORT(6, kDigitsChunkLarge) : GSX_TILE_SORT(6, kDigitsChunk);
        case 7: return large ? GSX_TILE_SORT(7, kDigitsChunkLarge) : GSX_TILE_SORT(7, kDigitsChunk);
        case 8: return large ? GSX_TILE_SORT(8, kDigitsChunkLarge) : GSX_TILE_SORT(8, kDigitsChunk);
        default: return GSX_HIP_ERROR_INVALID_ARGUMENT;
    }
#undef GSX_TILE_SORT
}

size_t tile_sort_u32_temp_bytes(int64_t n) { return radix_temp_bytes<8, kDigitsChunk>(n); }


size_t radix_sort_keys_u64_compacting_temp_bytes(int64_t n) {
    return radix_temp_bytes<kCompactingRadixBits, kCompactingChunk>(n);
}

}  // namespace gsx_amd
