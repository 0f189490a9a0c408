// render.hip - the gfx950 render path: preprocess, tile-key emission, tile ranges, blend
// forward, blend backward and projection backward.
//
// Semantics are those of the gsx CPU backend (gsx/src/gsx-cpu/render.c), which is the parity
// oracle: per-pixel order is (depth, Gaussian index), each pixel honours the Gaussian's 3-sigma
// pixel box, the -4.5 power cut, the 1/255 alpha cut and the 1e-4 transmittance cut, and the
// colour clamp max(c + 0.5, 0). The CUDA design this replaces (fastgs, kernels_forward.cuh /
// kernels_backward.cuh) differs in all of those, so none of its arithmetic is used here.
//
// Data layout in HBM (per Gaussian g, written by preprocess, read by emission and both blends),
// 48 B per visible Gaussian in two arrays (culled Gaussians only write tile_count = 0):
//   geo[2g+0] = {mean2d_x, mean2d_y, inv_a, 2*inv_b}      (conic of the dilated 2D covariance)
//   geo[2g+1] = {inv_c, opacity, x_min | x_max << 16, y_min | y_max << 16}   (ints as f32 bits)
//   col[g]    = {color_r, color_g, color_b, depth}
// Emission and tile counting gather records in depth order, one per Gaussian: they need the
// geometry only, a 32 B-aligned read. The blends read both and stage them in LDS as
//   {geo0} {inv_c, opacity, color_r, color_g} {color_b, box lo, box extent, depth}.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"

namespace gsx_amd {

constexpr int kBlendThreads = kTilePixels;  // 256: one pixel per thread, 4 waves per tile

// ---------------------------------------------------------------------------------------------
// Preprocess: render.c:850-1016 per Gaussian (culls, EWA projection, box, sigmoid, SH colour),
// plus the tile count of the box and, for TRAIN forwards, visible_counter += 1 (:980-982).
// ---------------------------------------------------------------------------------------------
// ---------------------------------------------------------------------------------------------
// Kept tiles (tile_cull.h): each tile row of a box keeps one contiguous run of tiles, given in
// closed form by the row's band columns. A wave walks the rows of its 64 Gaussians' boxes as one
// flattened sequence, 64 (Gaussian, row) items per step, so lanes stay busy whatever the box
// heights (a near-plane Gaussian's box can span the whole image, most span a row or two). Each
// lane's span constants live in LDS; a lane finds the owner of its item from the wave's
// exclusive prefix of row counts (marks at the lanes where a box's rows start, and a prefix
// maximum over the lanes). Counting adds each run's length to its owner's count; emission writes
// the runs of a step, 64 instances per sub-step, with a second owner search over the runs.
// ---------------------------------------------------------------------------------------------
constexpr int kWavesPerBlock = 4;
// Boxes of more tiles than this are emitted by a wave of their own (big_box_wave): in depth order
// the near, large boxes are neighbours, and a wave holding many full-image boxes would serialise
// their instances. Counting walks every box in the waves (rows are few).
constexpr uint32_t kBigTiles = 1024;
// preprocess's per-workgroup partials: kept tiles in bits 0..39 (a workgroup keeps fewer than
// 2^34), big boxes in bits 40..51 and visible Gaussians from bit 52 (at most 256 each)
constexpr int kKeptPartBigShift = 40;
constexpr int kKeptPartVisibleShift = 52;

// Sort keys. Gaussians are first sorted by depth: key = (bits(depth) - bits(near)) << index_bits
// | index (visible depths lie in [near, far], where positive floats order like their bit
// patterns, so the offset keeps the order in fewer bits; invisible Gaussians get the offset
// bits(far) - bits(near) + 1 and sort last). Instances are then emitted in that depth order,
// instance_tile[position] = tile, and the tile indices are sorted stably (u32 keys, the emission
// positions as values, implicit in the first pass): each tile's run is in (depth, index) order,
// the CPU backend's order, after two passes at 1080p.

__device__ inline uint32_t box_tiles(float4 geo1) {
    const uint32_t bx = __float_as_uint(geo1.z), by = __float_as_uint(geo1.w);
    return ((bx >> 16) / kTile - (bx & 0xffffu) / kTile + 1) * ((by >> 16) / kTile - (by & 0xffffu) / kTile + 1);
}

// The Gaussian's span constants from its geometry record (the record holds 2 * inv_b; halving
// is exact), as every pass that tests tiles forms them.
__device__ inline gsx_tile_span span_of(float4 r0, float4 r1) {
    const uint32_t bx = __float_as_uint(r1.z), by = __float_as_uint(r1.w);
    return gsx_tile_span_make(r0.x, r0.y, r0.z, r0.w * 0.5f, r1.x, r1.y, (int)(bx & 0xffffu), (int)(bx >> 16),
                              (int)(by & 0xffffu), (int)(by >> 16));
}

// A packed pixel box (box_lo / box_ext form, see in_box_packed) that no pixel lies in.
constexpr uint32_t kEmptyBoxLo = 0xffffffffu;

// The box the blend kernels test pixels against, in packed form (x0 | y0 << 16 and
// (x1 - x0) | (y1 - y0) << 16): the rectangle of the record's box that can hold a contributing
// pixel (gsx_contribution_box, from the record's mean, conic, opacity and box). It leaves out the
// corners of the 3-sigma box and, for all but the most opaque Gaussians, its rim, where every pixel
// fails the CPU's power or alpha cut; fewer pixels, and fewer waves of a tile, meet the entry.
// Preprocess stores it per visible Gaussian; key emission keeps using the record's box.
__device__ inline uint2 contribution_box_packed(float4 r0, float4 r1) {
    const uint32_t bx = __float_as_uint(r1.z), by = __float_as_uint(r1.w);
    int xa, xb, ya, yb;
    gsx_contribution_box(r0.x, r0.y, r0.z, r0.w * 0.5f, r1.x, r1.y, (int)(bx & 0xffffu), (int)(bx >> 16),
                         (int)(by & 0xffffu), (int)(by >> 16), &xa, &xb, &ya, &yb);
    if (xa > xb || ya > yb) return make_uint2(kEmptyBoxLo, 0u);
    return make_uint2((uint32_t)xa | ((uint32_t)ya << 16), (uint32_t)(xb - xa) | ((uint32_t)(yb - ya) << 16));
}

// Kept run of tile row ty of a box: len tiles from tile0 (len = 0 when none).
__device__ inline void row_run(const gsx_tile_span& k, uint32_t bx, uint32_t by, int ty, int32_t tiles_x,
                               uint32_t& len, uint32_t& tile0) {
    const int x0 = (int)(bx & 0xffffu), x1 = (int)(bx >> 16), y0 = (int)(by & 0xffffu), y1 = (int)(by >> 16);
    const int py0 = max(ty * kTile, y0), py1 = min(ty * kTile + kTile - 1, y1);
    int xa, xb;
    gsx_tile_band_columns(&k, x0, x1, py0, py1, &xa, &xb);
    len = 0u;
    tile0 = 0u;
    if (xa <= xb) {
        len = (uint32_t)(xb / kTile - xa / kTile + 1);
        tile0 = (uint32_t)ty * (uint32_t)tiles_x + (uint32_t)(xa / kTile);
    }
}

struct WaveSpans {
    float mx[kWave], my[kWave], b[kWave], ra[kWave], det[kWave], vr[kWave], aqs[kWave];  // gsx_tile_span
    uint32_t bx[kWave], by[kWave];  // box: x0 | x1 << 16, y0 | y1 << 16
    uint32_t excl[kWave];           // exclusive prefix of the lanes' row counts
    uint32_t mark[kWave];           // walk step: base + owner at the lane where that owner's rows start
    uint32_t kept[kWave];           // counting: kept tiles of the lane's box
    uint32_t base[kWave], g[kWave];  // emission: position of the lane's first instance less the walked
                                     // instances of the lanes before it; its Gaussian
    uint32_t run_tile[kWave], run_pos[kWave], run_g[kWave], mark2[kWave];  // emission: a step's runs
};

// Inclusive prefix maximum over the 64 lanes of a wave (DPP row shifts, then the two row
// broadcasts), for non-negative values; every lane must be active.
__device__ inline int wave_inclusive_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true));  // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true));  // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true));  // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true));  // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return v;
}

// Stores lane's span constants and box (no rows when !valid) and returns the wave's total row
// count.
__device__ inline uint32_t stage_spans(WaveSpans& w, bool valid, float4 r0, float4 r1) {
    const uint32_t lane = __lane_id();
    uint32_t rows = 0;
    if (valid) {
        const gsx_tile_span k = span_of(r0, r1);
        const uint32_t bx = __float_as_uint(r1.z), by = __float_as_uint(r1.w);
        w.mx[lane] = k.mx;
        w.my[lane] = k.my;
        w.b[lane] = k.b;
        w.ra[lane] = k.ra;
        w.det[lane] = k.det;
        w.vr[lane] = k.vr;
        w.aqs[lane] = k.aqs;
        w.bx[lane] = bx;
        w.by[lane] = by;
        rows = (by >> 16) / kTile - (by & 0xffffu) / kTile + 1;
    }
    w.kept[lane] = 0;
    const uint32_t incl = wave_inclusive_sum_u32(rows);
    w.excl[lane] = incl - rows;
    wave_lds_sync();
    return (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
}

// Walks the wave's flattened rows. kEmit = false adds each row's kept tiles to kept[owner];
// kEmit = true writes the kept instances (instance_tile, instance_gaussian) of every row, the
// rows of a box in order, at base[owner] + the instances of the walked rows before it.
template <bool kEmit>
__device__ inline void walk_wave_rows(WaveSpans& w, uint32_t wave_rows, int32_t tiles_x,
                                      uint32_t* __restrict__ instance_gaussian, uint32_t* __restrict__ instance_tile) {
    const uint32_t lane = __lane_id();
    // the owner of item p is the last box starting at or before p, i.e. the last non-empty one
    // (an empty box shares its start with the next box): each non-empty box whose rows start in
    // the step marks that lane with base + its lane, and a prefix maximum over the lanes, carried
    // from step to step, names every lane's owner (marks of earlier steps fall below base)
    const uint32_t my_start = w.excl[lane];
    const uint32_t my_count = (lane + 1 < kWave ? w.excl[lane + 1] : wave_rows) - my_start;
    w.mark[lane] = UINT32_MAX;
    uint32_t carry = 0, walked = 0;
    for (uint32_t base = 0; base < wave_rows; base += kWave) {
        const uint32_t p = base + lane;
        wave_lds_sync();  // the previous step's reads of the marks are done
        if (my_count > 0 && my_start - base < (uint32_t)kWave) w.mark[my_start - base] = base + lane;
        wave_lds_sync();
        const uint32_t m = w.mark[lane] - base;
        const uint32_t owner = max(carry, (uint32_t)wave_inclusive_max(m < (uint32_t)kWave ? (int)m : 0));
        carry = (uint32_t)__builtin_amdgcn_readlane((int)owner, kWave - 1);
        uint32_t len = 0, tile0 = 0;
        if (p < wave_rows) {
            gsx_tile_span k;
            k.mx = w.mx[owner];
            k.my = w.my[owner];
            k.b = w.b[owner];
            k.ra = w.ra[owner];
            k.det = w.det[owner];
            k.vr = w.vr[owner];
            k.aqs = w.aqs[owner];
            const uint32_t by = w.by[owner];
            const int ty = (int)((by & 0xffffu) / kTile + (p - w.excl[owner]));
            row_run(k, w.bx[owner], by, ty, tiles_x, len, tile0);
        }
        if (!kEmit) {
            if (len > 0) atomicAdd(&w.kept[owner], len);
        } else {
            // the step's runs, numbered q = start2 .. start2 + len - 1 in row order: run r holds
            // position run_pos[r] + q and tile run_tile[r] + q
            const uint32_t incl = wave_inclusive_sum_u32(len);
            const uint32_t start2 = incl - len;
            const uint32_t total2 = (uint32_t)__builtin_amdgcn_readlane((int)incl, kWave - 1);
            w.run_tile[lane] = tile0 - start2;
            w.run_pos[lane] = w.base[owner] + walked;
            w.run_g[lane] = w.g[owner];
            w.mark2[lane] = UINT32_MAX;
            uint32_t carry2 = 0;
            for (uint32_t base2 = 0; base2 < total2; base2 += kWave) {
                const uint32_t q = base2 + lane;
                wave_lds_sync();  // the run records are stored, the previous sub-step's marks read
                if (len > 0 && start2 - base2 < (uint32_t)kWave) w.mark2[start2 - base2] = base2 + lane;
                wave_lds_sync();
                const uint32_t m2 = w.mark2[lane] - base2;
                const uint32_t run = max(carry2, (uint32_t)wave_inclusive_max(m2 < (uint32_t)kWave ? (int)m2 : 0));
                carry2 = (uint32_t)__builtin_amdgcn_readlane((int)run, kWave - 1);
                if (q < total2) {
                    const uint32_t pos = w.run_pos[run] + q;
                    instance_gaussian[pos] = w.run_g[run];
                    instance_tile[pos] = w.run_tile[run] + q;
                }
            }
            walked += total2;
        }
        __builtin_amdgcn_wave_barrier();
    }
    wave_lds_sync();
}

// The parameter gradient sinks (mean3d, rotation, logscale, opacity, sh0..sh3: `arrays` of
// them, count[a] floats each), zeroed by the blend backward so that the projection backward
// writes only the rows of Gaussians some tile's backward reached. Workgroup b zeroes slice
// b / arrays of array b % arrays; per[a] floats per slice, a multiple of 4, and vec4 bit a when
// the array is 16-byte aligned (16-byte stores); all set by the host.
struct SinkZeroing {
    float* ptr[8];
    int64_t count[8];
    int64_t per[8];
    int arrays;
    uint32_t vec4;
};

// This workgroup's slice: no load and no wait, so the stores leave beside the kernel's own work.
__device__ inline void zero_sink_slice(const SinkZeroing& z, uint32_t blk) {
    if (z.arrays == 0) return;
    const uint32_t a = blk % (uint32_t)z.arrays;
    float* const p = z.ptr[a];
    const int64_t lo = (int64_t)(blk / (uint32_t)z.arrays) * z.per[a];
    const int64_t hi = min(z.count[a], lo + z.per[a]);
    if (lo >= hi) return;  // uniform
    int64_t done = lo;
    if ((z.vec4 >> a) & 1u) {
        const int vecs = (int)((hi - lo) >> 2);
        float4* const q = reinterpret_cast<float4*>(p + lo);
        for (int i = threadIdx.x; i < vecs; i += blockDim.x) q[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        done = lo + 4 * (int64_t)vecs;
    }
    for (int64_t i = done + threadIdx.x; i < hi; i += blockDim.x) p[i] = 0.0f;
}

// Destination of the retained TRAIN state: each field array copied as the forward reads it
// (null dst[0] in an inference forward). Field order mean3d, rotation, logscale, opacity, sh0..sh3.
struct FieldSnapshot {
    float* dst[8];
};

__device__ inline void copy_floats(const float* __restrict__ src, float* __restrict__ dst, int64_t g, int width) {
    for (int k = 0; k < width; ++k) dst[g * width + k] = src[g * width + k];
}

__global__ __launch_bounds__(256) void preprocess_kernel(
    FieldSnapshot snap, int64_t n, const float* __restrict__ mean3d, const float* __restrict__ rotation,
    const float* __restrict__ logscale, const float* __restrict__ opacity, const float* __restrict__ sh0,
    const float* __restrict__ sh1, const float* __restrict__ sh2, const float* __restrict__ sh3, int sh_degree,
    CameraParams cam, float4* __restrict__ rec, float4* __restrict__ col, uint2* __restrict__ cbox,
    float4* __restrict__ cov_coef, uint32_t* __restrict__ tile_count,
    float* __restrict__ visible_counter, uint32_t* __restrict__ big_list, uint32_t* __restrict__ big_count,
    uint32_t* __restrict__ clear0, uint32_t* __restrict__ clear1, uint32_t* __restrict__ clear2,
    unsigned long long* __restrict__ kept_part,
    uint64_t* __restrict__ depth_keys, uint32_t depth_base, uint32_t depth_max, int index_bits,
    uint64_t big_key_flag, int count_shift, uint8_t* __restrict__ touched) {
    __shared__ WaveSpans s_spans[kWavesPerBlock];
    __shared__ uint32_t s_kept[kWavesPerBlock], s_big[kWavesPerBlock];
    WaveSpans& ws = s_spans[threadIdx.x / kWave];
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    // counters that later kernels accumulate into start at zero (plain stores, no fill launch)
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *clear0 = 0u;
        *clear1 = 0u;
        *clear2 = 0u;
    }
    // TRAIN: the blend backward marks the Gaussians it reaches (touched[g] = 1)
    if (touched != nullptr && g < n) touched[g] = 0;
    if (snap.dst[0] != nullptr && g < n) {
        // consecutive lanes copy consecutive rows; preprocess_one then reads them from cache
        copy_floats(mean3d, snap.dst[0], g, 3);
        reinterpret_cast<float4*>(snap.dst[1])[g] = reinterpret_cast<const float4*>(rotation)[g];
        copy_floats(logscale, snap.dst[2], g, 3);
        snap.dst[3][g] = opacity[g];
        copy_floats(sh0, snap.dst[4], g, 3);
        if (sh_degree >= 1) copy_floats(sh1, snap.dst[5], g, 9);
        if (sh_degree >= 2) copy_floats(sh2, snap.dst[6], g, 15);
        if (sh_degree >= 3) copy_floats(sh3, snap.dst[7], g, 21);
    }
    bool visible = false;
    float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0, r2 = r0;
    if (g < n) {
        const Projected p =
            preprocess_one(g, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, sh_degree, cam, true);
        visible = p.visible;
        if (visible) {
            if (visible_counter != nullptr) visible_counter[g] += 1.0f;
            const float inv_a = p.c * p.inv_det;
            const float inv_b = -p.b * p.inv_det;
            const float inv_c = p.a * p.inv_det;
            const uint32_t bx = (uint32_t)p.x_min | ((uint32_t)p.x_max << 16);
            const uint32_t by = (uint32_t)p.y_min | ((uint32_t)p.y_max << 16);
            r0 = make_float4(p.mx, p.my, inv_a, 2.0f * inv_b);
            r1 = make_float4(inv_c, p.opacity, __uint_as_float(bx), __uint_as_float(by));
            r2 = make_float4(p.color[0], p.color[1], p.color[2], p.depth);
            rec[2 * g + 0] = r0;
            rec[2 * g + 1] = r1;
            col[g] = r2;
            cbox[g] = contribution_box_packed(r0, r1);
            if (cov_coef != nullptr) {
                // d(conic)/d(cov2d) coefficients with the CPU's rounding (render.c:1578-1579,
                // 1647-1655): the backward applies them per contribution, as the CPU does,
                // because for near-plane Gaussians with huge footprints the map is close to
                // singular and summing the conic gradients first would round very differently.
                const float det = p.a * p.c - p.b * p.b;
                const float k = 1.0f / (det * det);
                cov_coef[2 * g + 0] =
                    make_float4(-p.c * p.c * k, p.b * p.c * k, -p.b * p.b * k, -(p.a * p.c + p.b * p.b) * k);
                // with the doubled coefficients of the b row (exact: a power-of-two scaling) in the
                // free slots, so the backward forms none of them per pixel
                const float k0y = p.b * p.c * k, k1x = p.a * p.b * k;
                cov_coef[2 * g + 1] = make_float4(k1x, -p.a * p.a * k, 2.0f * k0y, 2.0f * k1x);
            }
        }
    }
    const bool big = visible && box_tiles(r1) > kBigTiles;
    // emitted by big_box_wave; one atomic per wave (a scene can hold millions of big boxes)
    const uint32_t big_slot = wave_append_slot(big_count, big);
    if (big) big_list[big_slot] = (uint32_t)g;
    const uint32_t rows = stage_spans(ws, visible, r0, r1);
    walk_wave_rows<false>(ws, rows, cam.tiles_x, nullptr, nullptr);
    const uint32_t kept = ws.kept[__lane_id()];
    if (g < n) tile_count[g] = kept;
    // depth key of every Gaussian (~0 for invisible ones, which the depth sort drops);
    // big_key_flag (kBigKeyFlag or 0, see there) marks the big boxes for rank_gather_kernel;
    // count_shift > 0: the kept-tile count rides above the sorted bits, so rank_gather_kernel
    // reads it from the sorted key instead of gathering tile_count at random Gaussians
    if (g < n) {
        uint64_t key = ~0ull;
        if (visible) {
            uint32_t rel = __float_as_uint(r2.w) - depth_base;
            if (rel > depth_max) rel = depth_max;  // only for non-finite depths
            key = ((uint64_t)rel << index_bits) | (uint64_t)g | (big ? big_key_flag : 0ull);
            if (count_shift > 0) key |= (uint64_t)kept << count_shift;
        }
        depth_keys[g] = key;
    }
    // the workgroup's kept tiles, big boxes and visible Gaussians to kept_part[block], host
    // memory that the host sums for the instance count, the big-box launch and the visible count
    // (a wave's kept sum is below 64 * 2^24 tiles, a workgroup's below 2^34)
    const uint32_t wave_kept = wave_reduce_sum_u32(kept);
    const uint32_t wave_big = (uint32_t)__popcll(wave_ballot(big));
    const uint32_t wave_visible = (uint32_t)__popcll(wave_ballot(visible && g < n));
    if (__lane_id() == 0) {
        s_kept[threadIdx.x / kWave] = wave_kept;
        s_big[threadIdx.x / kWave] = wave_big | (wave_visible << 16);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long sum = 0, bigs = 0, vis = 0;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) {
            sum += s_kept[w];
            bigs += s_big[w] & 0xffffu;
            vis += s_big[w] >> 16;
        }
        kept_part[blockIdx.x] = sum | (bigs << kKeptPartBigShift) | (vis << kKeptPartVisibleShift);
    }
}

// Marks a big box's depth key (big_box_wave needs its rank). Used only when the sorted depth
// bits end below bit 63, which holds for fewer than 2^31 Gaussians.
constexpr uint64_t kBigKeyFlag = 1ull << 63;

// Instance runs longer than this are summed in chunks by whole waves in the backward (see
// reduce_long_block), shorter ones by one lane each.
constexpr uint32_t kLaneRun = 32;

// After the depth sort of the V visible Gaussians (V = *depth_count): the Gaussian of every
// depth rank, its kept-tile count, the rank of each big box and of each Gaussian whose count
// exceeds long_chunk (the only ranks looked up by Gaussian: by big-box emission and by the
// projection backward for runs of several chunks; every Gaussian's when flagged_only is false)
// and the list of ranks whose count exceeds long_chunk (the backward sums long runs in chunks of
// that many positions). Ranks V..n-1 get count 0 and no Gaussian. Each workgroup also stores the
// sum of its 256 counts in block_sums[block] and its number of counts above kLaneRun in
// block_sums[gridDim.x + 1 + block], the first steps of the offsets scan and of the long-run
// list (emit_block finishes both).
__global__ __launch_bounds__(256) void rank_gather_kernel(int64_t n, const uint32_t* __restrict__ depth_count,
                                                          const uint64_t* __restrict__ sorted_depth_keys,
                                                          uint64_t index_mask, bool flagged_only,
                                                          int count_shift, uint32_t count_mask,
                                                          const uint32_t* __restrict__ tile_count,
                                                          uint32_t* __restrict__ rank_gaussian,
                                                          uint32_t* __restrict__ rank_count,
                                                          uint32_t* __restrict__ gaussian_rank,
                                                          uint32_t long_chunk,
                                                          uint32_t* __restrict__ multi_list,
                                                          uint32_t* __restrict__ multi_count,
                                                          uint32_t* __restrict__ block_sums) {
    __shared__ uint32_t s_sum[kWavesPerBlock];
    __shared__ uint32_t s_long[kWavesPerBlock];
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t c = 0;
    if (r < n) {
        if (r < (int64_t)*depth_count) {
            const uint64_t key = sorted_depth_keys[r];
            const uint32_t g = (uint32_t)(key & index_mask);
            c = count_shift > 0 ? (uint32_t)(key >> count_shift) & count_mask : tile_count[g];
            rank_gaussian[r] = g;
            if (!flagged_only || (key & kBigKeyFlag) != 0 || c > long_chunk) gaussian_rank[g] = (uint32_t)r;
        }
        rank_count[r] = c;
    }
    // runs of several chunks are listed (rare: their boxes span more than long_chunk tiles); one
    // atomic per wave that has any (c is 0 past the visible ranks)
    const uint32_t multi_slot = wave_append_slot(multi_count, c > long_chunk);
    if (c > long_chunk) multi_list[multi_slot] = (uint32_t)r;
    const uint32_t wave_sum = wave_reduce_sum_u32(c);
    const uint32_t wave_long = (uint32_t)__popcll(__ballot(c > kLaneRun));
    if (__lane_id() == 0) {
        s_sum[threadIdx.x / kWave] = wave_sum;
        s_long[threadIdx.x / kWave] = wave_long;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t sum = 0, longs = 0;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) {
            sum += s_sum[w];
            longs += s_long[w];
        }
        block_sums[blockIdx.x] = sum;
        block_sums[gridDim.x + 1 + blockIdx.x] = longs;
    }
}

// ---------------------------------------------------------------------------------------------
// Instance emission in depth order: the Gaussian of rank r owns positions offset[r] ..
// offset[r+1]) of the instance array, one per kept tile of its box in row-major tile order
// (offsets are the exclusive scan of the counts in rank order). instance_tile[position] = tile
// (the sort's keys; the backward's reduction also looks up each position's tile) and
// instance_gaussian[position] = g. A stable sort of the tiles with the positions as values then
// leaves every tile's run in (depth, index) order, i.e. in ascending position.
// The offsets are finished here: block_prefix[b] is the exclusive scan of rank_gather_kernel's
// 256-rank sums, and emission workgroup b (ranks 256 b .. 256 b + 255, rank_gather_kernel's
// blocking) scans its own 256 counts; offsets[0..n] are stored for the later kernels
// (offsets[n] = total).
// ---------------------------------------------------------------------------------------------
__device__ inline void emit_block(uint32_t b, int64_t n, int64_t rank_end, const float4* __restrict__ rec,
                                  const uint32_t* __restrict__ rank_gaussian, const uint32_t* __restrict__ rank_count,
                                  const uint32_t* __restrict__ block_prefix, uint32_t* __restrict__ offsets,
                                  int32_t tiles_x, uint32_t* __restrict__ instance_gaussian,
                                  uint32_t* __restrict__ instance_tile,
                                  const uint32_t* __restrict__ long_prefix, uint32_t* __restrict__ long_list,
                                  WaveSpans* s_spans, uint32_t* s_wave) {
    WaveSpans& ws = s_spans[threadIdx.x / kWave];
    const int64_t r = (int64_t)b * blockDim.x + threadIdx.x;
    // the rank's count and Gaussian load together, then its whole record (one wait each)
    uint32_t cnt = 0, g = 0;
    if (r < n) {
        cnt = rank_count[r];
        g = rank_gaussian[r];
    }
    uint32_t block_total;
    const uint32_t o = block_prefix[b] + block_exclusive_scan_256(cnt, s_wave, block_total);
    if (r < n) offsets[r] = o;
    // offsets[n] (the instance total, read by the ranges pass) from the last rank launched: the
    // launch covers the visible ranks and at least one more, whose counts are 0
    if (r == rank_end - 1) offsets[n] = o + cnt;
    // the long-run list in rank order: long_prefix[b] (scanned per-workgroup counts of
    // rank_gather_kernel) + the rank's place among the workgroup's long runs (s_wave is free
    // again after the scan's last barrier)
    {
        const bool is_long = cnt > kLaneRun;
        const uint64_t lm = __ballot(is_long);
        if (__lane_id() == 0) s_wave[threadIdx.x / kWave] = (uint32_t)__popcll(lm);
        __syncthreads();
        uint32_t at = long_prefix[b] + (uint32_t)__popcll(lm & lanemask_lt());
        for (int w = 0; w < (int)(threadIdx.x / kWave); ++w) at += s_wave[w];
        if (is_long) long_list[at] = (uint32_t)r;
    }
    float4 r0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r1 = r0;
    if (cnt > 0) {
        r0 = rec[2 * (size_t)g + 0];
        r1 = rec[2 * (size_t)g + 1];
    }
    // big boxes are emitted by big_rows_block; the walk numbers the wave's other instances
    // consecutively, so a lane's base is its offset less the walked instances of the lanes
    // before it (the counting walk's identical runs gave the counts)
    const bool walked = cnt > 0 && box_tiles(r1) <= kBigTiles;
    const uint32_t wcnt = walked ? cnt : 0u;
    const uint32_t lane = __lane_id();
    ws.base[lane] = o - (wave_inclusive_sum_u32(wcnt) - wcnt);
    ws.g[lane] = g;
    const uint32_t rows = stage_spans(ws, walked, r0, r1);
    walk_wave_rows<true>(ws, rows, tiles_x, instance_gaussian, instance_tile);
}

// Big boxes: one wave per box of big_list, walking its rows as walk_wave_rows walks a wave's
// boxes (the box in lane 0, the others empty). It runs beside emit_block in one launch, so it
// forms the box's offset itself: block_prefix of the rank's 256-rank block plus the counts of the
// ranks before it in that block. The host sizes the launch with one wave per big box.
__device__ inline void big_box_wave(uint32_t i, const uint32_t* __restrict__ big_list, const float4* __restrict__ rec,
                                    int32_t tiles_x, const uint32_t* __restrict__ rank_count,
                                    const uint32_t* __restrict__ block_prefix,
                                    const uint32_t* __restrict__ gaussian_rank,
                                    uint32_t* __restrict__ instance_gaussian, uint32_t* __restrict__ instance_tile,
                                    WaveSpans& ws) {
    const uint32_t lane = __lane_id();
    const uint32_t g = big_list[i];
    const float4 r0 = rec[2 * (size_t)g + 0], r1 = rec[2 * (size_t)g + 1];
    const uint32_t rr = gaussian_rank[g];
    const uint32_t b0 = rr & ~255u;
    uint32_t v = 0;
#pragma unroll
    for (uint32_t k = 0; k < 256; k += kWave) v += b0 + k + lane < rr ? rank_count[b0 + k + lane] : 0u;
    ws.base[lane] = block_prefix[rr >> 8] + wave_reduce_sum_u32(v);
    ws.g[lane] = g;
    const uint32_t rows = stage_spans(ws, lane == 0, r0, r1);
    walk_wave_rows<true>(ws, rows, tiles_x, instance_gaussian, instance_tile);
}

// All emission in one launch: workgroups [0, big_blocks) hold one wave per big box, first so
// that their longer walks start early; the rest are the emission workgroups of the ranks.
__global__ __launch_bounds__(256) void emit_kernel(int64_t n, const float4* __restrict__ rec,
                                                   const uint32_t* __restrict__ rank_gaussian,
                                                   const uint32_t* __restrict__ rank_count,
                                                   const uint32_t* __restrict__ block_prefix,
                                                   uint32_t* __restrict__ offsets, int32_t tiles_x,
                                                   const uint32_t* __restrict__ big_list,
                                                   const uint32_t* __restrict__ big_count, uint32_t big_blocks,
                                                   const uint32_t* __restrict__ gaussian_rank,
                                                   uint32_t* __restrict__ instance_gaussian,
                                                   uint32_t* __restrict__ instance_tile,
                                                   const uint32_t* __restrict__ long_prefix,
                                                   uint32_t* __restrict__ long_list) {
    __shared__ WaveSpans s_spans[kWavesPerBlock];
    __shared__ uint32_t s_wave[kWavesPerBlock];
    if (blockIdx.x < big_blocks) {
        // no workgroup barrier on this path: each wave takes its own box
        const uint32_t i = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
        if (i < *big_count)
            big_box_wave(i, big_list, rec, tiles_x, rank_count, block_prefix, gaussian_rank, instance_gaussian,
                         instance_tile, s_spans[threadIdx.x / kWave]);
        return;
    }
    // the rank workgroups cover ranks [0, rank_end): the visible ones and at least one past them
    // (ranks of invisible Gaussians emit nothing, and no kernel reads their offsets)
    const int64_t rank_end = min(n, (int64_t)(gridDim.x - big_blocks) * blockDim.x);
    emit_block(blockIdx.x - big_blocks, n, rank_end, rec, rank_gaussian, rank_count, block_prefix, offsets, tiles_x,
               instance_gaussian, instance_tile, long_prefix, long_list, s_spans, s_wave);
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t count, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

__global__ __launch_bounds__(256) void fill_f32_kernel(float* __restrict__ p, int64_t count, float v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

// [start, end) of each tile's run in the sorted tile indices. Tiles without instances get
// (0, 0): the thread of the last instance before such a gap (or of the first instance, for the
// tiles before it) writes them, so no fill of all tiles is needed beforehand. count >= 1 (with
// no instances the caller fills the ranges). Each thread takes 4 consecutive sorted tiles (one
// 16-byte load), plus the tiles just before and after them for the boundaries.
__global__ __launch_bounds__(256) void tile_ranges_kernel(const uint32_t* __restrict__ sorted_tiles,
                                                          const uint32_t* count_ptr, uint32_t tiles,
                                                          uint2* __restrict__ ranges) {
    const uint32_t count = *count_ptr;
    const uint32_t i0 = 4u * (blockIdx.x * blockDim.x + threadIdx.x);
    if (i0 >= count) return;
    const uint32_t m = min(4u, count - i0);
    // the neighbours load with the thread's own (clamped in-range positions, not branches)
    const uint32_t t_prev = sorted_tiles[i0 == 0 ? 0u : i0 - 1u];
    const uint32_t t_next = sorted_tiles[min(i0 + m, count - 1u)];
    uint32_t t[4];
    if (m == 4) {
        const uint4 q = *reinterpret_cast<const uint4*>(sorted_tiles + i0);
        t[0] = q.x;
        t[1] = q.y;
        t[2] = q.z;
        t[3] = q.w;
    } else {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) t[j] = j < m ? sorted_tiles[i0 + j] : 0u;
    }
    const uint32_t prev = i0 == 0 ? UINT32_MAX : t_prev;
    const uint32_t next = i0 + m == count ? tiles : t_next;
    if (i0 == 0) {
        for (uint32_t u = 0; u < t[0]; ++u) ranges[u] = make_uint2(0u, 0u);
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        if (j < m) {
            const uint32_t before = j == 0 ? prev : t[j - 1];
            const uint32_t after = j == m - 1 ? next : t[j + 1];
            if (before != t[j]) ranges[t[j]].x = i0 + j;
            if (after != t[j]) {
                ranges[t[j]].y = i0 + j + 1;
                for (uint32_t u = t[j] + 1; u < after; ++u) ranges[u] = make_uint2(0u, 0u);
            }
        }
    }
}

// The same ranges for large instance counts: one thread per tile finds the lower bounds of its
// tile and of the next in the sorted tiles by binary search, the two searches in lockstep
// (ceil(log2(count + 1)) steps of two loads each, the same for every lane) instead of a pass over
// every instance. Tiles without instances get (0, 0).
__global__ __launch_bounds__(256) void tile_ranges_search_kernel(const uint32_t* __restrict__ sorted_tiles,
                                                                 uint32_t count, uint32_t tiles, int steps,
                                                                 uint2* __restrict__ ranges) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= tiles) return;
    uint32_t lo0 = 0, hi0 = count, lo1 = 0, hi1 = count;
    for (int k = 0; k < steps; ++k) {
        const uint32_t m0 = lo0 + ((hi0 - lo0) >> 1), m1 = lo1 + ((hi1 - lo1) >> 1);
        // both loads in flight (positions clamped into the array; a finished search keeps lo = hi)
        const uint32_t v0 = sorted_tiles[min(m0, count - 1u)], v1 = sorted_tiles[min(m1, count - 1u)];
        if (lo0 < hi0) {
            if (v0 < t) lo0 = m0 + 1u; else hi0 = m0;
        }
        if (lo1 < hi1) {
            if (v1 < t + 1u) lo1 = m1 + 1u; else hi1 = m1;
        }
    }
    ranges[t] = lo0 < lo1 ? make_uint2(lo0, lo1) : make_uint2(0u, 0u);
}

// Workgroup -> tile mapping: consecutive workgroups are dealt round-robin to the 8 XCDs, so give
// each XCD a contiguous band of tiles (neighbouring tiles share Gaussians, and each XCD has its
// own L2).
__device__ inline int xcd_tile_index(int block, int tiles) {
    const int per = (tiles + 7) / 8;
    const int xcd = block & 7;
    const int local = block >> 3;
    const int t = xcd * per + local;
    return t;
}

// Pixel of thread t of a tile's 256-thread workgroup. Each wave takes an 8 x 8 quadrant of the
// tile (wave w: quadrant (w & 1, w >> 1), lane l: pixel (l & 7, l >> 3) in it), not four 16-pixel
// rows: a Gaussian's footprint meets fewer waves of a tile when the waves are square, and each
// wave that meets it works on every lane. The DPP rows of 16 lanes are two pixel rows of a
// quadrant; the backward's per-row partial sums do not depend on which pixels a row holds.
__device__ inline int2 tile_pixel_of_thread(int t) {
    const int w = t >> 6, l = t & 63;
    return make_int2(((w & 1) << 3) | (l & 7), ((w >> 1) << 3) | (l >> 3));
}

// The box test in packed 16-bit halves, three vector instructions: (px, py) lies in
// [x0, x1] x [y0, y1] iff both halves of (px | py << 16) - (x0 | y0 << 16) (each wrapping mod
// 2^16) are at most those of (x1 - x0) | (y1 - y0) << 16. The blend kernels stage each
// contribution box (contribution_box_packed) in this form (kEmptyBoxLo / 0 for none: no pixel
// coordinate is 65535).
typedef uint16_t gsx_u16x2 __attribute__((ext_vector_type(2)));
__device__ inline bool in_box_packed(uint32_t pxy, uint32_t lo, uint32_t ext) {
    const gsx_u16x2 d = __builtin_bit_cast(gsx_u16x2, pxy) - __builtin_bit_cast(gsx_u16x2, lo);
    const gsx_u16x2 m = __builtin_elementwise_min(d, __builtin_bit_cast(gsx_u16x2, ext));
    return __builtin_bit_cast(uint32_t, m) == __builtin_bit_cast(uint32_t, d);
}

// Transmittance checkpoints: the backward needs every contribution's exact T_before (the CPU
// records it, render.c:1501-1506; recomputing it by division perturbs the last bit, which the
// near-singular covariance gradient of near-plane Gaussians amplifies without bound). A TRAIN
// forward therefore stores each pixel's T at the start of every 8-entry bucket of its tile's
// list. Bucket k of a tile whose list starts at position x lives in slot x/8 + tile + k, which
// is collision-free and needs at most I/8 + tiles + 1 slots of 256 floats.
constexpr int kBucket = 8;

__device__ inline size_t checkpoint_slot(uint32_t range_start, int tile, uint32_t position) {
    return (size_t)(range_start / kBucket) + (size_t)tile + (size_t)((position - range_start) / kBucket);
}

// ---------------------------------------------------------------------------------------------
// Blend forward: render.c:1018-1088, per pixel in per-tile (depth, index) order. Records of the
// tile's Gaussians are staged through LDS in batches of 256; a tile stops early once every pixel
// has T < 1e-4. Writes out_rgb (CHW, background composed: C + T*bg), final T, the exclusive end
// of the last contributing position, and (TRAIN) the bucket checkpoints.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(kBlendThreads) void blend_forward_kernel(
    const uint2* __restrict__ ranges, const uint32_t* __restrict__ values,
    const uint32_t* __restrict__ instance_gaussian, const float4* __restrict__ rec, const float4* __restrict__ col,
    const uint2* __restrict__ cbox, uint32_t* __restrict__ sorted_g,
    CameraParams cam, float* __restrict__ out_rgb,
    float* __restrict__ out_t, uint32_t* __restrict__ out_last, float* __restrict__ ckpt) {
    __shared__ float4 s_r0[kBlendThreads];
    __shared__ float4 s_r1[kBlendThreads];
    __shared__ float4 s_r2[kBlendThreads];
    __shared__ uint64_t s_exp2[GSX_EXPF_BLEND_TABLE_SIZE];
    const int tiles = cam.tiles_x * cam.tiles_y;
    const int tile = xcd_tile_index(blockIdx.x, tiles);
    if (tile >= tiles) return;
    if (threadIdx.x < GSX_EXPF_BLEND_TABLE_SIZE) s_exp2[threadIdx.x] = gsx_expf_blend_entry(threadIdx.x);
    const int tx = tile % cam.tiles_x, ty = tile / cam.tiles_x;
    const int2 tp = tile_pixel_of_thread((int)threadIdx.x);
    const int px = tx * kTile + tp.x;
    const int py = ty * kTile + tp.y;
    const bool inside = px < cam.width && py < cam.height;
    const uint2 range = ranges[tile];
    const float fpx = (float)px + 0.5f;
    const float fpy = (float)py + 0.5f;
    const uint32_t pxy = (uint32_t)px | ((uint32_t)py << 16);  // for in_box_packed
    // t only falls, and a pixel is done once an accepted contribution takes it below the
    // threshold, so "done" is t < threshold; pixels outside the image start done (t = 0, never
    // written out)
    float t = inside ? 1.0f : 0.0f, c0 = 0.0f, c1 = 0.0f, c2 = 0.0f;
    uint32_t last = range.x;
    for (uint32_t base = range.x; base < range.y; base += kBlendThreads) {
        if (__syncthreads_count(t < kTransmittanceThreshold ? 1 : 0) == kBlendThreads) break;
        const uint32_t j = base + threadIdx.x;
        if (j < range.y) {
            const uint32_t g = instance_gaussian[values[j]];
            if (sorted_g != nullptr) sorted_g[j] = g;  // TRAIN: the backward reads it
            const float4 geo1 = rec[2 * (size_t)g + 1], c = col[g];
            const uint2 box = cbox[g];
            s_r0[threadIdx.x] = rec[2 * (size_t)g + 0];
            s_r1[threadIdx.x] = make_float4(geo1.x, geo1.y, c.x, c.y);
            s_r2[threadIdx.x] = make_float4(c.z, __uint_as_float(box.x), __uint_as_float(box.y), c.w);
        } else {
            // past the list: a box no pixel lies in, so the last bucket can run whole
            s_r2[threadIdx.x] = make_float4(0.0f, __uint_as_float(kEmptyBoxLo), 0.0f, 0.0f);
        }
        __syncthreads();
        // wave-uniform bound, held in a scalar register, rounded up to whole buckets
        const int count = __builtin_amdgcn_readfirstlane((int)min((uint32_t)kBlendThreads, range.y - base));
        const int padded = (count + kBucket - 1) & ~(kBucket - 1);
        // the lanes not done (t only changes where an entry is evaluated, so the mask is
        // re-formed there, not per entry)
        uint64_t open_mask = wave_ballot(t >= kTransmittanceThreshold);
        // buckets of kBucket entries, each unrolled: the checkpoint at the bucket's start and
        // the loop control cost no instructions per entry
        for (int k0 = 0; k0 < padded; k0 += kBucket) {
            if (mask_none(open_mask)) break;  // uniform: every pixel of this wave is saturated
            if (ckpt != nullptr && t >= kTransmittanceThreshold)
                ckpt[checkpoint_slot(range.x, tile, base + (uint32_t)k0) * kBlendThreads + threadIdx.x] = t;
#pragma unroll
            for (int i = 0; i < kBucket; ++i) {
                const int k = k0 + i;
                const float4 r2 = s_r2[k];
                const bool ib = in_box_packed(pxy, __float_as_uint(r2.y), __float_as_uint(r2.z));
                const uint64_t live_mask = open_mask & wave_ballot(ib);
                if (mask_none(live_mask)) continue;  // uniform
                const bool live = __builtin_amdgcn_inverse_ballot_w64(live_mask);
                // branch-free evaluation for the wave; lanes outside the box or done keep their state
                const float4 r0 = s_r0[k];
                const float4 r1 = s_r1[k];
                const float dx = fpx - r0.x;
                const float dy = fpy - r0.y;
                float power = -0.5f * (r0.z * dx * dx + r0.w * dx * dy + r1.x * dy * dy);
                power = power > 0.0f ? 0.0f : power;
                bool ok = live & (power >= kPowerThreshold);
                const float gval = gsx_expf_blend(fmaxf(power, kPowerThreshold), s_exp2);
                const float alpha = fminf(kMaxFragmentAlpha, r1.y * gval);
                ok = ok & (alpha >= kMinAlpha);
                // a lane that does not take the entry uses alpha = 0: it adds (0 * colour) = +-0,
                // which leaves its sums exactly as they are (they start at +0 and stay finite), and
                // multiplies t by 1, so one select serves the colour sums and t
                const float a_used = ok ? alpha : 0.0f;
                const float w = a_used * t;
                c0 = c0 + w * r1.z;
                c1 = c1 + w * r1.w;
                c2 = c2 + w * r2.x;
                t = t * (1.0f - a_used);
                last = ok ? base + (uint32_t)k + 1u : last;
                open_mask = wave_ballot(t >= kTransmittanceThreshold);
                if (mask_none(open_mask)) break;  // uniform
            }
        }
        __syncthreads();
    }
    if (inside) {
        const size_t pix = (size_t)py * (size_t)cam.width + (size_t)px;
        const size_t plane = (size_t)cam.width * (size_t)cam.height;
        out_rgb[pix] = c0 + t * cam.bg[0];
        out_rgb[plane + pix] = c1 + t * cam.bg[1];
        out_rgb[2 * plane + pix] = c2 + t * cam.bg[2];
        out_t[pix] = t;
        out_last[pix] = last;
    }
}

// Per-Gaussian screen-space gradient accumulator, 9 floats per Gaussian:
//   dmean2d x, y | dcov2d a, b, c | dcolor r, g, b | dopacity (w.r.t. the sigmoid value)
constexpr int kGrad2d = 9;
constexpr int kGradRecord = 8;  // per-instance partials: channels 0-7 in one 32-byte record

// ---------------------------------------------------------------------------------------------
// Blend backward: render.c:1559-1666 restated per pixel, back to front, with the CPU's exact
// T_before: for each 8-entry bucket (last first) the pixel reloads the bucket's checkpointed T,
// replays the bucket forward (same operations as the forward, so T_before, G and the contribution
// set are bit-identical to the CPU's) and then walks it backwards accumulating the suffix colour
// exactly as the CPU does. Per contribution the gradient terms are the CPU's, including the
// d(conic)/d(cov2d) map applied per contribution.
// Reduction without atomics: each 16-pixel row sums its lanes' 9 partials per entry with DPP
// moves (row_reduce_scatter9), the 16 row totals are combined through LDS, and the tile writes
// one 9-float partial per reached instance at its emission position (channels 0-7 as one 32-byte
// record of instance_grad, channel 8, the opacity term, in instance_grad_op) and its cut
// position (tile_cut: the instances past it were not reached and have no partial);
// reduce_instance_grads_kernel then sums each Gaussian's contiguous run of positions. The result
// is deterministic and immune to the contention of full-screen Gaussians (present in every tile),
// and the instances behind saturated pixels cost the backward nothing.
// ---------------------------------------------------------------------------------------------
constexpr int kWavesPerTile = kBlendThreads / kWave;
constexpr int kRowsPerTile = kTile;  // 16 DPP rows of 16 lanes per workgroup

// The backward stages 64 entries per batch (8 buckets of 8): the kernel fits 71 VGPRs and 19 KB
// of LDS, i.e. 7 waves per SIMD (16-entry buckets need 87 VGPRs and 28 KB: 5 waves; the
// checkpoints of the smaller buckets cost the forward less than the occupancy gains here).
constexpr int kBackBatch = 64;
constexpr int kBatchBuckets = kBackBatch / kBucket;

__global__ __launch_bounds__(kBlendThreads) void blend_backward_kernel(
    const uint2* __restrict__ ranges, const uint32_t* __restrict__ values, const uint32_t* __restrict__ sorted_g,
    const float4* __restrict__ rec, const float4* __restrict__ col, const uint2* __restrict__ cbox,
    const float4* __restrict__ cov_coef, const float* __restrict__ ckpt,
    CameraParams cam, const float* __restrict__ grad_rgb, const float* __restrict__ final_t,
    const uint32_t* __restrict__ last_contrib, float* __restrict__ instance_grad,
    float* __restrict__ instance_grad_op, uint32_t* __restrict__ tile_cut, uint8_t* __restrict__ touched,
    SinkZeroing sinks) {
    __shared__ float4 s_r0[kBackBatch];
    __shared__ float4 s_r1[kBackBatch];
    __shared__ float4 s_r2[kBackBatch];
    __shared__ float4 s_k0[kBackBatch];
    __shared__ float4 s_k1[kBackBatch];
    __shared__ uint32_t s_pos[kBackBatch];
    __shared__ float s_ck[kBatchBuckets][kBlendThreads];
    __shared__ float s_acc[kRowsPerTile][kBucket][kGrad2d];
    __shared__ uint64_t s_exp2[GSX_EXPF_BLEND_TABLE_SIZE];
    __shared__ uint32_t s_max_last;
    // every workgroup, the padding ones included, zeroes its slice of the gradient sinks first
    zero_sink_slice(sinks, blockIdx.x);
    const int tiles = cam.tiles_x * cam.tiles_y;
    const int tile = xcd_tile_index(blockIdx.x, tiles);
    if (tile >= tiles) return;
    if (threadIdx.x < GSX_EXPF_BLEND_TABLE_SIZE) s_exp2[threadIdx.x] = gsx_expf_blend_entry(threadIdx.x);
    const int tx = tile % cam.tiles_x, ty = tile / cam.tiles_x;
    const int2 tp = tile_pixel_of_thread((int)threadIdx.x);
    const int px = tx * kTile + tp.x;
    const int py = ty * kTile + tp.y;
    const int row = threadIdx.x / kTile;  // DPP row of the workgroup (16 lanes)
    const bool inside = px < cam.width && py < cam.height;
    const uint2 range = ranges[tile];
    const size_t pix = (size_t)py * (size_t)cam.width + (size_t)px;
    const size_t plane = (size_t)cam.width * (size_t)cam.height;
    const float fpx = (float)px + 0.5f;
    const float fpy = (float)py + 0.5f;
    const uint32_t pxy = (uint32_t)px | ((uint32_t)py << 16);  // for in_box_packed
    float t_final = 0.0f, d0 = 0.0f, d1 = 0.0f, d2 = 0.0f;
    uint32_t last = range.x;
    if (inside) {
        t_final = final_t[pix];
        last = last_contrib[pix];
        d0 = grad_rgb[pix];
        d1 = grad_rgb[plane + pix];
        d2 = grad_rgb[2 * plane + pix];
    }
    // render.c:1552-1557: the suffix starts as T_final * background
    float s0 = t_final * cam.bg[0], s1 = t_final * cam.bg[1], s2 = t_final * cam.bg[2];
    if (threadIdx.x == 0) s_max_last = range.x;
    __syncthreads();
    atomicMax(&s_max_last, last);
    __syncthreads();
    const uint32_t end_all = s_max_last;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    // Entries from zero_from on (whole buckets past the last entry any pixel of the tile reaches)
    // get no partial: their gradient is zero. Positions ascend along the tile's run, so the run's
    // entries with a partial are exactly those whose position is below tile_cut[tile], the
    // position of the first entry without one (UINT32_MAX: all have one); the reduction adds +0
    // for the others instead of reading them.
    const uint32_t zero_from =
        end_all <= range.x ? range.x : range.x + ((end_all - range.x + kBucket - 1) / kBucket) * kBucket;
    if (threadIdx.x == 0) tile_cut[tile] = zero_from < range.y ? values[zero_from] : UINT32_MAX;
    if (end_all <= range.x) return;  // uniform

    // Batches of kBackBatch entries are walked back to front; records and the batch's bucket
    // checkpoints reach LDS at the start of each batch.
    const uint32_t first_batch = range.x + ((end_all - 1u - range.x) / kBackBatch) * kBackBatch;
    for (int64_t bstart = first_batch; bstart >= (int64_t)range.x; bstart -= kBackBatch) {
        const int count = (int)min((uint32_t)kBackBatch, range.y - (uint32_t)bstart);
        // the batch's checkpoints load together, ahead of the records (not under branches: a
        // pixel that needs no checkpoint of a bucket reads the batch's first slot, which exists,
        // and keeps 0)
        float ck[kBatchBuckets];
#pragma unroll
        for (int b = 0; b < kBatchBuckets; ++b) {
            const uint32_t j0 = (uint32_t)bstart + (uint32_t)(b * kBucket);
            const uint32_t js = (inside && j0 < last) ? j0 : (uint32_t)bstart;
            ck[b] = ckpt[checkpoint_slot(range.x, tile, js) * kBlendThreads + threadIdx.x];
        }
        if (threadIdx.x < count) {
            const uint32_t j = (uint32_t)bstart + threadIdx.x;
            s_pos[threadIdx.x] = values[j];
            // sorted_g is written by the TRAIN forward for every batch it loaded, and every entry
            // below end_all lies in such a batch; entries from end_all on contribute nothing
            if (j < end_all) {
                const uint32_t g = sorted_g[j];
                touched[g] = 1;
                const float4 geo1 = rec[2 * (size_t)g + 1], c = col[g];
                const uint2 box = cbox[g];
                s_r0[threadIdx.x] = rec[2 * (size_t)g + 0];
                s_r1[threadIdx.x] = make_float4(geo1.x, geo1.y, c.x, c.y);
                s_r2[threadIdx.x] = make_float4(c.z, __uint_as_float(box.x), __uint_as_float(box.y), c.w);
                s_k0[threadIdx.x] = cov_coef[2 * (size_t)g + 0];
                s_k1[threadIdx.x] = cov_coef[2 * (size_t)g + 1];
            } else {
                const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                s_r0[threadIdx.x] = z;
                s_r1[threadIdx.x] = z;
                s_r2[threadIdx.x] = make_float4(0.0f, __uint_as_float(kEmptyBoxLo), 0.0f, 0.0f);  // no pixel
                s_k0[threadIdx.x] = z;
                s_k1[threadIdx.x] = z;
            }
        }
#pragma unroll
        for (int b = 0; b < kBatchBuckets; ++b) {
            const uint32_t j0 = (uint32_t)bstart + (uint32_t)(b * kBucket);
            s_ck[b][threadIdx.x] = (inside && j0 < last) ? ck[b] : 0.0f;
        }
        __syncthreads();
        const int sb_first = (count - 1) / kBucket;
        for (int sb = sb_first; sb >= 0; --sb) {
            const uint32_t j0 = (uint32_t)bstart + (uint32_t)(sb * kBucket);
            if (j0 < end_all) {  // uniform; buckets from end_all on get no partial (tile_cut)
            const int n_in = min(kBucket, count - sb * kBucket);
            float tb[kBucket];
            float gv[kBucket];
            // forward replay of the bucket from its checkpoint (render.c:1476-1515)
            {
                float tt = s_ck[sb][threadIdx.x];
                const bool pixel_live = inside && j0 < last;
                const uint64_t pixel_mask = wave_ballot(pixel_live);
#pragma unroll
                for (int i = 0; i < kBucket; ++i) {
                    tb[i] = tt;
                    gv[i] = 0.0f;
                    if (i >= n_in) continue;  // uniform
                    const int kk = sb * kBucket + i;
                    const float4 r2 = s_r2[kk];
                    const bool ib = in_box_packed(pxy, __float_as_uint(r2.y), __float_as_uint(r2.z));
                    const bool before_last = j0 + (uint32_t)i < last;
                    const bool live = pixel_live & before_last & ib;
                    if (mask_none(pixel_mask & wave_ballot(before_last) & wave_ballot(ib))) continue;
                    const float4 r0 = s_r0[kk];
                    const float4 r1 = s_r1[kk];
                    const float dx = fpx - r0.x;
                    const float dy = fpy - r0.y;
                    float power = -0.5f * (r0.z * dx * dx + r0.w * dx * dy + r1.x * dy * dy);
                    power = power > 0.0f ? 0.0f : power;
                    bool ok = live & (power >= kPowerThreshold);
                    const float gval = gsx_expf_blend(fmaxf(power, kPowerThreshold), s_exp2);
                    const float alpha = fminf(kMaxFragmentAlpha, r1.y * gval);
                    ok = ok & (alpha >= kMinAlpha);
                    gv[i] = ok ? gval : 0.0f;
                    tt = ok ? tt * (1.0f - alpha) : tt;
                }
            }
            // back to front over the bucket (render.c:1559-1666 per contribution)
#pragma unroll
            for (int i = kBucket - 1; i >= 0; --i) {
                if (i >= n_in) continue;  // uniform
                const int kk = sb * kBucket + i;
                // a contribution has G = exp(power) >= exp(-4.5) > 0 and the others keep G = 0
                if (mask_none(wave_ballot(gv[i] != 0.0f))) {  // uniform: no pixel of this wave
                    if (lane < 4 * kGrad2d) s_acc[wave * 4 + lane / kGrad2d][i][lane % kGrad2d] = 0.0f;
                    continue;
                }
                const float4 r0 = s_r0[kk];
                const float4 r1 = s_r1[kk];
                const float4 r2 = s_r2[kk];
                const float dx = fpx - r0.x;
                const float dy = fpy - r0.y;
                const float gval = gv[i];
                const float op = r1.y;
                const float alpha = fminf(kMaxFragmentAlpha, op * gval);
                const float t_before = tb[i];
                // A lane that does not contribute holds G = 0, hence alpha = 0: its weight w, dpow
                // and opacity term below are (signed) zeros by arithmetic, and it leaves the suffix
                // unchanged, so no per-lane select on the contribution is needed (all values are
                // finite).
                const float w = alpha * t_before;
                float dalpha = t_before * (r1.z * d0 + r1.w * d1 + r2.x * d2);
                // a correctly rounded division as the CPU's: near-plane Gaussians' covariance
                // gradients amplify even 1-ulp differences of this term. alpha <= 0.999, so
                // 1 - alpha lies in [0.001, 1]: the CPU's |1 - alpha| > 1e-6 guard always holds,
                // the scaling steps of the general division are not needed, and a zero numerator
                // gives a zero quotient.
                const float num = s0 * d0 + s1 * d1 + s2 * d2;
                dalpha -= div_rn_normal(num, 1.0f - alpha);
                const bool unclamped = op * gval < kMaxFragmentAlpha;
                const float dg = unclamped ? dalpha * op : 0.0f;
                const float g_op = unclamped ? dalpha * gval : 0.0f;
                const float dpow = dg * gval;
                const float inv_a = r0.z, inv_b = r0.w * 0.5f, inv_c = r1.x;
                const float dia = dpow * (-0.5f * dx * dx);
                const float dib = dpow * (-dx * dy);
                const float dic = dpow * (-0.5f * dy * dy);
                const float4 k0 = s_k0[kk];
                const float4 k1 = s_k1[kk];  // k1.z = 2 k0.y, k1.w = 2 k1.x
                // the mean2d terms may fuse; the covariance terms keep the CPU's rounding, since
                // near-plane Gaussians' covariance maps are close to singular
                float v[kGrad2d] = {dpow * __builtin_fmaf(inv_a, dx, inv_b * dy),
                                    dpow * __builtin_fmaf(inv_b, dx, inv_c * dy),
                                    dia * k0.x + dib * k0.y + dic * k0.z,
                                    dia * k1.z + dib * k0.w + dic * k1.w,
                                    dia * k0.z + dib * k1.x + dic * k1.y,
                                    w * d0,
                                    w * d1,
                                    w * d2,
                                    g_op};
                s0 += w * r1.z;
                s1 += w * r1.w;
                s2 += w * r2.x;
                float total8;
                float scattered = row_reduce_scatter9(v, total8);
                // both totals are complete before the stores below: otherwise the compiler sinks the
                // last DPP adds into the masked store blocks, where they cannot fuse
                asm volatile("" : "+v"(scattered), "+v"(total8));
                const uint32_t col = threadIdx.x & (kTile - 1);  // lane within the DPP row
                if ((col & 1u) == 0u) s_acc[row][i][col >> 1] = scattered;
                if (col == 0u) s_acc[row][i][8] = total8;
            }
            __syncthreads();
            // combine the 16 row partials and write the bucket's per-instance partials
            for (int o = threadIdx.x; o < n_in * kGrad2d; o += kBlendThreads) {
                const int e = o / kGrad2d, c = o % kGrad2d;
                float q[kRowsPerTile];
#pragma unroll
                for (int r = 0; r < kRowsPerTile; ++r) q[r] = s_acc[r][e][c];
#pragma unroll
                for (int h = kRowsPerTile / 2; h > 0; h >>= 1) {
#pragma unroll
                    for (int r = 0; r < h; ++r) q[r] += q[r + h];
                }
                const size_t pos = s_pos[sb * kBucket + e];
                if (c < kGradRecord) {
                    instance_grad[pos * kGradRecord + c] = q[0];
                } else {
                    instance_grad_op[pos] = q[0];
                }
            }
            __syncthreads();
            }
        }
    }
}

// grad2d[g] = sum of the partials over the emission positions [offset[r], offset[r+1]) of g, r its
// depth rank; every Gaussian's sum is taken in a fixed order, so the result is deterministic.
// Position p has a partial iff p < tile_cut[instance_tile[p]] (the blend backward's cut of p's
// tile); the others count as +0, read from neither array. A Gaussian that no tile reached
// (touched[g] == 0) has no partial at all: its sums are not formed, and projection_backward_kernel
// writes its zero gradients without reading them.
//  * runs of at most kLaneRun instances (reduce_short_block): the 64 runs of a wave's ranks are
//    one contiguous span; the wave stages it through its own LDS piece by piece with coalesced
//    loads, jumping over long runs, and each lane sums its run in position order into grad2d;
//  * longer runs (in depth order the near, large Gaussians sit side by side, and the largest
//    cover nearly every tile) are cut into at most kLongChunks chunks of `chunk` positions, and
//    one wave sums a chunk (DPP tree, reduce_run_chunk). reduce_long_block takes chunk 0 of every
//    long run (long_list, in rank order, written by emit_block) and chunks 1.. of the runs longer
//    than one chunk (multi_list, from rank_gather_kernel), the entries dealt round-robin over the
//    waves: the near, large Gaussians are neighbours in depth order, and a wave of their own
//    would serialise them. A run of one chunk is done; the others leave each chunk's sums in
//    place at its first position, and projection_backward_kernel adds them in chunk order.
// All of it runs in one launch (reduce_instance_grads_kernel).
constexpr uint32_t kShortPiece = 256;  // instances per LDS piece and wave (9 KB)
constexpr uint32_t kLongChunks = 16;

__device__ inline void add_record(float acc[kGrad2d], float4 a, float4 b, float op) {
    acc[0] += a.x;
    acc[1] += a.y;
    acc[2] += a.z;
    acc[3] += a.w;
    acc[4] += b.x;
    acc[5] += b.y;
    acc[6] += b.z;
    acc[7] += b.w;
    acc[8] += op;
}

// Position p's partial (three loads), or +0 where the blend backward wrote none.
struct InstancePartial {
    float4 a, b;
    float op;
};
__device__ inline InstancePartial load_partial(const float4* __restrict__ rec4, const float* __restrict__ instance_grad_op,
                                               const uint32_t* __restrict__ instance_tile,
                                               const uint32_t* __restrict__ tile_cut, uint32_t p) {
    InstancePartial v;
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (p < tile_cut[instance_tile[p]]) {
        v.a = rec4[2 * (size_t)p];
        v.b = rec4[2 * (size_t)p + 1];
        v.op = instance_grad_op[p];
    } else {
        v.a = z;
        v.b = z;
        v.op = 0.0f;
    }
    return v;
}

// Chunk k of the long run [b, e) of Gaussian g, summed by the whole wave (b, e, g, k wave-uniform).
// A run of one chunk gets its sums in grad2d, a longer one its chunk's sums at the chunk's first
// position.
__device__ inline void reduce_run_chunk(uint32_t b, uint32_t e, uint32_t g, uint32_t k, uint32_t chunk,
                                        float* __restrict__ instance_grad, float* __restrict__ instance_grad_op,
                                        const uint32_t* __restrict__ instance_tile,
                                        const uint32_t* __restrict__ tile_cut, float* __restrict__ grad2d) {
    const uint32_t lane = __lane_id();
    const float4* rec4 = reinterpret_cast<const float4*>(instance_grad);
    const uint32_t cb = b + k * chunk;
    const uint32_t ce = min(e, cb + chunk);
    float acc[kGrad2d];
#pragma unroll
    for (int c = 0; c < kGrad2d; ++c) acc[c] = 0.0f;
    for (uint32_t p0 = cb; p0 < ce; p0 += 4 * kWave) {
        // all loads of the round are in flight together: none sits under a branch (lanes past
        // the chunk re-read its last position and add nothing)
        InstancePartial v[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t p = min(p0 + u * kWave + lane, ce - 1);
            v[u] = load_partial(rec4, instance_grad_op, instance_tile, tile_cut, p);
        }
        // lanes past the chunk add -0, the identity of + (an unconditional use keeps the loads
        // ahead of the adds)
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const bool in = p0 + u * kWave + lane < ce;
            const float4 z = make_float4(-0.0f, -0.0f, -0.0f, -0.0f);
            add_record(acc, in ? v[u].a : z, in ? v[u].b : z, in ? v[u].op : -0.0f);
        }
    }
#pragma unroll
    for (int c = 0; c < kGrad2d; ++c) acc[c] = wave_reduce_sum(acc[c]);
    if (lane != 0) return;
    if (e - b <= chunk) {
#pragma unroll
        for (int c = 0; c < kGrad2d; ++c) grad2d[(size_t)g * kGrad2d + c] = acc[c];
        return;
    }
    // every lane's loads of the chunk fed the sums above, so overwriting position cb is safe
    float4* dst = reinterpret_cast<float4*>(instance_grad) + 2 * (size_t)cb;
    dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    instance_grad_op[cb] = acc[8];
}

// The +0 sums of chunk k of a long run that no tile reached, stored by one lane.
// Chunk k of the long runs of the wave's lanes (run [b, e) of Gaussian g where `live`): the
// touched ones are summed by the wave one after another (the untouched ones have no sums: the
// projection backward skips their Gaussians).
__device__ inline void reduce_wave_long_runs(bool live, uint32_t b, uint32_t e, uint32_t g, uint32_t k,
                                             uint32_t chunk, float* __restrict__ instance_grad,
                                             float* __restrict__ instance_grad_op,
                                             const uint32_t* __restrict__ instance_tile,
                                             const uint32_t* __restrict__ tile_cut,
                                             const uint8_t* __restrict__ touched, float* __restrict__ grad2d) {
    const bool hit = live && touched[g] != 0;
    for (uint64_t todo = __ballot(hit); todo != 0ull; todo &= todo - 1ull) {
        const int src = __builtin_ctzll(todo);
        reduce_run_chunk((uint32_t)__builtin_amdgcn_readlane((int)b, src),
                         (uint32_t)__builtin_amdgcn_readlane((int)e, src),
                         (uint32_t)__builtin_amdgcn_readlane((int)g, src), k, chunk, instance_grad, instance_grad_op,
                         instance_tile, tile_cut, grad2d);
    }
}

__device__ inline void reduce_short_block(uint32_t blk, int64_t n, const uint32_t* __restrict__ depth_count,
                                          const uint32_t* __restrict__ offsets,
                                          const uint32_t* __restrict__ rank_gaussian, uint32_t chunk,
                                          float* __restrict__ instance_grad, float* __restrict__ instance_grad_op,
                                          const uint32_t* __restrict__ instance_tile,
                                          const uint32_t* __restrict__ tile_cut, const uint8_t* __restrict__ touched,
                                          float* __restrict__ grad2d, float4 (*s_rec)[2 * kShortPiece],
                                          float (*s_op)[kShortPiece]) {
    const uint32_t lane = __lane_id(), wave = threadIdx.x / kWave;
    n = min(n, (int64_t)*depth_count);  // ranks of visible Gaussians
    const int64_t r = (int64_t)blk * blockDim.x + threadIdx.x;
    const int64_t r_first = r - lane;  // first rank of this wave (waves wholly past n find no work)
    const bool valid = r < n;
    uint32_t b = 0, e = 0, g = 0;
    if (valid) {
        b = offsets[r];
        e = offsets[r + 1];
        g = rank_gaussian[r];
    }
    const bool mine = valid && e - b <= kLaneRun;
    const bool has = mine && e > b && touched[g] != 0;
    const uint32_t span_end = offsets[min(r_first + (int64_t)kWave, n)];
    const float4* rec4 = reinterpret_cast<const float4*>(instance_grad);
    float4* sr = s_rec[wave];
    float* so = s_op[wave];
    float acc[kGrad2d];
#pragma unroll
    for (int c = 0; c < kGrad2d; ++c) acc[c] = 0.0f;
    for (uint32_t cur = offsets[min(r_first, n)];;) {
        // the piece starts at the lowest position a short run of the wave still needs
        const uint32_t p0 = wave_min_u32(has && e > cur ? max(b, cur) : UINT32_MAX);
        if (p0 == UINT32_MAX) break;  // uniform
        const uint32_t p1 = min(p0 + kShortPiece, span_end);
        wave_lds_sync();  // the previous piece has been read
        // every load of the piece is issued before the first store waits on one: the loads are
        // not under a branch (lanes past the piece re-read its last position, p1 > p0)
        constexpr int kPieceRounds = (int)(kShortPiece / kWave);
        const uint32_t len = p1 - p0;
        InstancePartial v[kPieceRounds];
#pragma unroll
        for (int u = 0; u < kPieceRounds; ++u) {
            const uint32_t q = min(lane + (uint32_t)u * kWave, len - 1);
            v[u] = load_partial(rec4, instance_grad_op, instance_tile, tile_cut, p0 + q);
        }
        // (unconditional stores: lanes past the piece write its last position's own values again)
#pragma unroll
        for (int u = 0; u < kPieceRounds; ++u) {
            const uint32_t q = min(lane + (uint32_t)u * kWave, len - 1);
            sr[2 * q] = v[u].a;
            sr[2 * q + 1] = v[u].b;
            so[q] = v[u].op;
        }
        wave_lds_sync();
        if (has) {
            const uint32_t lo = max(b, p0), hi = min(e, p1);
            for (uint32_t p = lo; p < hi; ++p) add_record(acc, sr[2 * (p - p0)], sr[2 * (p - p0) + 1], so[p - p0]);
        }
        cur = p1;
    }
    if (has) {
#pragma unroll
        for (int c = 0; c < kGrad2d; ++c) grad2d[(size_t)g * kGrad2d + c] = acc[c];
    }
}

// Chunk k of the runs on `list`, by the gx * 4 waves of the workgroups of column k: lane l of
// wave w takes entries w + W (l + 64 j), j = 0, 1, ... (W waves), so neighbouring entries go to
// different waves.
__device__ inline void reduce_long_block(uint32_t x, uint32_t k, uint32_t gx, const uint32_t* __restrict__ list,
                                         const uint32_t* __restrict__ list_count,
                                         const uint32_t* __restrict__ offsets,
                                         const uint32_t* __restrict__ rank_gaussian, uint32_t chunk,
                                         float* __restrict__ instance_grad, float* __restrict__ instance_grad_op,
                                         const uint32_t* __restrict__ instance_tile,
                                         const uint32_t* __restrict__ tile_cut, const uint8_t* __restrict__ touched,
                                         float* __restrict__ grad2d) {
    const uint32_t count = *list_count;
    const uint32_t waves = gx * (blockDim.x / kWave);
    const uint32_t w = x * (blockDim.x / kWave) + threadIdx.x / kWave;
    for (uint32_t j = 0; w + waves * j * kWave < count; ++j) {
        const uint32_t i = w + waves * (j * kWave + __lane_id());
        uint32_t b = 0, e = 0, g = 0;
        bool live = false;
        if (i < count) {
            const uint32_t r = list[i];
            b = offsets[r];
            e = offsets[r + 1];
            g = rank_gaussian[r];
            live = b + k * chunk < e;
        }
        reduce_wave_long_runs(live, b, e, g, k, chunk, instance_grad, instance_grad_op, instance_tile, tile_cut,
                              touched, grad2d);
    }
}

// Both reductions in one launch: workgroups [0, gx0) take chunk 0 of the long runs, the next
// gx * (kLongChunks - 1) chunks 1.. of the runs longer than one chunk (x = index % gx, chunk
// k = 1 + index / gx), the rest the short runs of the ranks (256 each).
__global__ __launch_bounds__(256) void reduce_instance_grads_kernel(
    int64_t n, const uint32_t* __restrict__ depth_count, const uint32_t* __restrict__ offsets,
    const uint32_t* __restrict__ rank_gaussian, const uint32_t* __restrict__ long_list,
    const uint32_t* __restrict__ long_count, const uint32_t* __restrict__ multi_list,
    const uint32_t* __restrict__ multi_count, uint32_t gx0, uint32_t gx, uint32_t chunk,
    float* __restrict__ instance_grad,
    float* __restrict__ instance_grad_op, const uint32_t* __restrict__ instance_tile,
    const uint32_t* __restrict__ tile_cut, const uint8_t* __restrict__ touched, float* __restrict__ grad2d) {
    __shared__ float4 s_rec[kWavesPerBlock][2 * kShortPiece];
    __shared__ float s_op[kWavesPerBlock][kShortPiece];
    if (blockIdx.x < gx0) {
        reduce_long_block(blockIdx.x, 0, gx0, long_list, long_count, offsets, rank_gaussian, chunk, instance_grad,
                          instance_grad_op, instance_tile, tile_cut, touched, grad2d);
        return;
    }
    const uint32_t long_blocks = gx0 + gx * (kLongChunks - 1);
    if (blockIdx.x < long_blocks) {
        const uint32_t bi = blockIdx.x - gx0;
        reduce_long_block(bi % gx, 1 + bi / gx, gx, multi_list, multi_count, offsets, rank_gaussian, chunk,
                          instance_grad, instance_grad_op, instance_tile, tile_cut, touched, grad2d);
        return;
    }
    reduce_short_block(blockIdx.x - long_blocks, n, depth_count, offsets, rank_gaussian, chunk, instance_grad,
                       instance_grad_op, instance_tile, tile_cut, touched, grad2d, s_rec, s_op);
}

__device__ inline void add3(float* p, float x, float y, float z) {
    p[0] += x;
    p[1] += y;
    p[2] += z;
}

// render.c:714-728
__device__ inline void add_dir(float ddir[3], const float dcol[3], const float* coeff, float bx, float by, float bz) {
    const float s = dcol[0] * coeff[0] + dcol[1] * coeff[1] + dcol[2] * coeff[2];
    ddir[0] += s * bx;
    ddir[1] += s * by;
    ddir[2] += s * bz;
}

// ---------------------------------------------------------------------------------------------
// Projection backward: render.c:1667-1969 per Gaussian, from the accumulated screen-space
// gradients. Sinks are overwritten (the CPU zeroes them first, render.c:1537-1550); invisible
// Gaussians get zeros.
// ---------------------------------------------------------------------------------------------
// Instantiated per SH degree (0-3): the higher degrees' gradient arrays then exist only where
// they are used (degree 0 needs 45 fewer live registers).
// Stores the rows of a kWidth-float field for the workgroup's Gaussians [first, first + count)
// (thread t holds row first + t) as whole 16-byte vectors: the rows go through LDS, then
// consecutive threads store consecutive vectors of the block's contiguous span (a row of 3, 9, 15
// or 21 floats would otherwise take that many 4-byte stores at a stride of the row). dst must be
// 16-byte aligned; the span's last floats past its last whole vector are stored one by one. Every
// thread of the workgroup calls it.
template <int kWidth>
__device__ inline void block_store_rows(float* __restrict__ dst, int64_t first, int count, const float (&row)[kWidth],
                                        float* s_stage) {
    __syncthreads();  // the previous field's stores have read s_stage
#pragma unroll
    for (int k = 0; k < kWidth; ++k) s_stage[threadIdx.x * kWidth + k] = row[k];
    __syncthreads();
    const int total = count * kWidth;
    const int vecs = total / 4;
    float* base = dst + first * kWidth;
    for (int i = threadIdx.x; i < vecs; i += blockDim.x)
        reinterpret_cast<float4*>(base)[i] = reinterpret_cast<const float4*>(s_stage)[i];
    for (int i = vecs * 4 + (int)threadIdx.x; i < total; i += blockDim.x) base[i] = s_stage[i];
}

template <int kShDegree>
__global__ __launch_bounds__(256) void projection_backward_kernel(
    int64_t n, const float* __restrict__ mean3d, const float* __restrict__ rotation,
    const float* __restrict__ logscale, const float* __restrict__ opacity, const float* __restrict__ sh0,
    const float* __restrict__ sh1, const float* __restrict__ sh2, const float* __restrict__ sh3,
    CameraParams cam, const float* __restrict__ grad2d, const uint32_t* __restrict__ tile_count,
    const uint32_t* __restrict__ gaussian_rank, const uint32_t* __restrict__ offsets, uint32_t chunk,
    const float* __restrict__ instance_grad, const float* __restrict__ instance_grad_op,
    const uint8_t* __restrict__ touched, float* __restrict__ g_mean3d,
    float* __restrict__ g_rotation, float* __restrict__ g_logscale, float* __restrict__ g_opacity,
    float* __restrict__ g_sh0, float* __restrict__ g_sh1, float* __restrict__ g_sh2, float* __restrict__ g_sh3,
    int vector_stores) {
    constexpr int sh_degree = kShDegree;
    constexpr int kStageWidth = kShDegree >= 3 ? 21 : (kShDegree == 2 ? 15 : (kShDegree == 1 ? 9 : 3));
    // the exp table in LDS: its lookups wait on LDS, not on a global load each
    __shared__ uint64_t s_exp[GSX_EXP2_TABLE_SIZE];
    // the block's rows of one gradient field on their way to whole-vector stores
    __shared__ __align__(16) float s_stage[256 * kStageWidth];
    const int64_t first = (int64_t)blockIdx.x * blockDim.x;
    const int64_t gi = first + threadIdx.x;
    const bool valid = gi < n;  // every thread stays for the block's staged stores
    // a Gaussian that no tile's backward reached (touched[gi] == 0: invisible ones included) has
    // a +0 screen-space gradient and so zero parameter gradients, which the blend backward has
    // already stored in every sink (zero_sink_slice): a block with no reached Gaussian is done
    const bool reached = valid && touched[gi] != 0;
    if (!__syncthreads_or(reached ? 1 : 0)) return;
    // A reached Gaussian was emitted, so preprocess_one found it visible in the forward; of its
    // projection the backward uses only the camera-space mean, the view direction and the clamped
    // colour, recomputed here by the same operations (not the covariance, conic and box, whose
    // dependent chain would set the time of a block holding one of the few reached Gaussians).
    // Every input is loaded before the exp table's barrier, so their latency overlaps it.
    ProjectedView p{};
    p.visible = reached;
    uint32_t run_length = 0;
    uint32_t rank = 0;
    float4 q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float ls[3] = {0.0f, 0.0f, 0.0f};
    if (reached) {
        // the rank is used only by a run of several chunks; read here, coalesced, it takes a load
        // round off that chain
        run_length = tile_count[gi];
        rank = gaussian_rank[gi];
        q = reinterpret_cast<const float4*>(rotation)[gi];
        ls[0] = logscale[gi * 3 + 0];
        ls[1] = logscale[gi * 3 + 1];
        ls[2] = logscale[gi * 3 + 2];
        p = project_view(gi, mean3d, sh0, sh1, sh2, sh3, sh_degree, cam);
    }
    if (threadIdx.x < GSX_EXP2_TABLE_SIZE) s_exp[threadIdx.x] = gsx_exp2_table_entry(threadIdx.x);
    __syncthreads();
    const uint64_t* exp_tab = s_exp;
    __builtin_assume(exp_tab != nullptr);  // no run-time choice of table per lookup
    float gm[3] = {0.0f, 0.0f, 0.0f};
    float gr[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float gl[3] = {0.0f, 0.0f, 0.0f};
    float gop = 0.0f;
    float gs0[3] = {0.0f, 0.0f, 0.0f};
    float gs1[9];
    float gs2[15];
    float gs3[21];
#pragma unroll
    for (int i = 0; i < 9; ++i) gs1[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 15; ++i) gs2[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 21; ++i) gs3[i] = 0.0f;
    float a2[kGrad2d];
#pragma unroll
    for (int c = 0; c < kGrad2d; ++c) a2[c] = 0.0f;
    const bool multi = p.visible && run_length > chunk;
    if (p.visible && !multi) {
#pragma unroll
        for (int c = 0; c < kGrad2d; ++c) a2[c] = grad2d[(size_t)gi * kGrad2d + c];
    }
    {
        // A run of several chunks: the sums of its chunks (reduce_long_block), added in chunk
        // order from +0. The wave loads one such run's chunk sums at once, lane k taking chunk k,
        // and every lane adds them in lane order (the owner keeps the result): one load round per
        // run instead of one per chunk, whose serial latency would set the kernel's time.
        const int lane = (int)(threadIdx.x & (kWave - 1));
        uint32_t rb = 0, re = 0;
        if (multi) {
            rb = offsets[rank];
            re = offsets[rank + 1];
        }
        for (uint64_t runs = wave_ballot(multi); runs != 0; runs &= runs - 1) {
            const int src = __builtin_ctzll(runs);
            const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)rb, src);
            const uint32_t len = (uint32_t)__builtin_amdgcn_readlane((int)re, src) - b;
            float v[kGrad2d];
#pragma unroll
            for (int c = 0; c < kGrad2d; ++c) v[c] = 0.0f;
            if ((uint32_t)lane * chunk < len) {
                const uint32_t cb = b + (uint32_t)lane * chunk;
                const float4* rec4 = reinterpret_cast<const float4*>(instance_grad) + 2 * (size_t)cb;
                const float4 x = rec4[0], y = rec4[1];
                v[0] = x.x, v[1] = x.y, v[2] = x.z, v[3] = x.w;
                v[4] = y.x, v[5] = y.y, v[6] = y.z, v[7] = y.w;
                v[8] = instance_grad_op[cb];
            }
            float acc[kGrad2d];
#pragma unroll
            for (int c = 0; c < kGrad2d; ++c) acc[c] = 0.0f;
            for (int k = 0; k < kWave && (uint32_t)k * chunk < len; ++k) {
#pragma unroll
                for (int c = 0; c < kGrad2d; ++c)
                    acc[c] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[c]), k));
            }
            if (lane == src) {
#pragma unroll
                for (int c = 0; c < kGrad2d; ++c) a2[c] = acc[c];
            }
        }
    }
    if (p.visible) {
        const float dmx = a2[0], dmy = a2[1];
        const float dca = a2[2], dcb = a2[3], dcc = a2[4];
        const float dcx = a2[5], dcy = a2[6], dcz = a2[7];
        const float dop = a2[8];
        const Mat3 w = camera_rotation(cam);
        const Mat3 rot = rotation_from_xyzw(q.x, q.y, q.z, q.w);
        const float sx = gsx_expf_table(ls[0], exp_tab), sy = gsx_expf_table(ls[1], exp_tab),
                    sz = gsx_expf_table(ls[2], exp_tab);
        // R S, and the covariance (R S)(R S)^T by cov3d_from's operations
        Mat3 srot = rot;
#pragma unroll
        for (int row = 0; row < 3; ++row) {
            srot.m[row][0] *= sx;
            srot.m[row][1] *= sy;
            srot.m[row][2] *= sz;
        }
        const Mat3 cov3d = mat3_mul_t(srot, srot);
        const float zc = p.zc, xc = p.xc, yc = p.yc;
        const float j00 = cam.fx / zc;
        const float j02 = -cam.fx * xc / (zc * zc);
        const float j11 = cam.fy / zc;
        const float j12 = -cam.fy * yc / (zc * zc);
        // colour: render.c:1667-1828
        {
            const float dcol[3] = {dcx * (p.color[0] > 0.0f ? 1.0f : 0.0f), dcy * (p.color[1] > 0.0f ? 1.0f : 0.0f),
                                   dcz * (p.color[2] > 0.0f ? 1.0f : 0.0f)};
            float ddir[3] = {0.0f, 0.0f, 0.0f};
            const float x = p.dir[0], y = p.dir[1], z = p.dir[2];
            const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
            gs0[0] = kShC0 * dcol[0];
            gs0[1] = kShC0 * dcol[1];
            gs0[2] = kShC0 * dcol[2];
            if (sh_degree >= 1) {
                const float* c1 = sh1 + gi * 9;
                float s;
                s = -kShC1 * y;
                add3(gs1 + 0, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                s = kShC1 * z;
                add3(gs1 + 3, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                s = -kShC1 * x;
                add3(gs1 + 6, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c1 + 0, 0.0f, -kShC1, 0.0f);
                add_dir(ddir, dcol, c1 + 3, 0.0f, 0.0f, kShC1);
                add_dir(ddir, dcol, c1 + 6, -kShC1, 0.0f, 0.0f);
            }
            if (sh_degree >= 2) {
                const float* c2 = sh2 + gi * 15;
                float s;
                s = kShC2[0] * xy;
                add3(gs2 + 0, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c2 + 0, kShC2[0] * y, kShC2[0] * x, 0.0f);
                s = kShC2[1] * yz;
                add3(gs2 + 3, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c2 + 3, 0.0f, kShC2[1] * z, kShC2[1] * y);
                s = kShC2[2] * (2.0f * zz - xx - yy);
                add3(gs2 + 6, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c2 + 6, -2.0f * kShC2[2] * x, -2.0f * kShC2[2] * y, 4.0f * kShC2[2] * z);
                s = kShC2[3] * xz;
                add3(gs2 + 9, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c2 + 9, kShC2[3] * z, 0.0f, kShC2[3] * x);
                s = kShC2[4] * (xx - yy);
                add3(gs2 + 12, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c2 + 12, 2.0f * kShC2[4] * x, -2.0f * kShC2[4] * y, 0.0f);
            }
            if (sh_degree >= 3) {
                const float* c3 = sh3 + gi * 21;
                float s;
                s = kShC3[0] * y * (3.0f * xx - yy);
                add3(gs3 + 0, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 0, 6.0f * kShC3[0] * x * y, 3.0f * kShC3[0] * (xx - yy), 0.0f);
                s = kShC3[1] * xy * z;
                add3(gs3 + 3, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 3, kShC3[1] * y * z, kShC3[1] * x * z, kShC3[1] * xy);
                s = kShC3[2] * y * (4.0f * zz - xx - yy);
                add3(gs3 + 6, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 6, -2.0f * kShC3[2] * x * y, kShC3[2] * (4.0f * zz - xx - 3.0f * yy),
                        8.0f * kShC3[2] * y * z);
                s = kShC3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
                add3(gs3 + 9, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 9, -6.0f * kShC3[3] * x * z, -6.0f * kShC3[3] * y * z,
                        kShC3[3] * (6.0f * zz - 3.0f * xx - 3.0f * yy));
                s = kShC3[4] * x * (4.0f * zz - xx - yy);
                add3(gs3 + 12, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 12, kShC3[4] * (4.0f * zz - 3.0f * xx - yy), -2.0f * kShC3[4] * x * y,
                        8.0f * kShC3[4] * x * z);
                s = kShC3[5] * z * (xx - yy);
                add3(gs3 + 15, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 15, 2.0f * kShC3[5] * x * z, -2.0f * kShC3[5] * y * z, kShC3[5] * (xx - yy));
                s = kShC3[6] * x * (xx - 3.0f * yy);
                add3(gs3 + 18, dcol[0] * s, dcol[1] * s, dcol[2] * s);
                add_dir(ddir, dcol, c3 + 18, 3.0f * kShC3[6] * (xx - yy), -6.0f * kShC3[6] * x * y, 0.0f);
            }
            if (sh_degree >= 1) {
                const float vx = mean3d[gi * 3 + 0] - cam.centre[0];
                const float vy = mean3d[gi * 3 + 1] - cam.centre[1];
                const float vz = mean3d[gi * 3 + 2] - cam.centre[2];
                const float vn = sqrtf(vx * vx + vy * vy + vz * vz);
                if (vn > 0.0f) {
                    const float dd = ddir[0] * x + ddir[1] * y + ddir[2] * z;
                    const float s = 1.0f / vn;
                    gm[0] += (ddir[0] - x * dd) * s;
                    gm[1] += (ddir[1] - y * dd) * s;
                    gm[2] += (ddir[2] - z * dd) * s;
                }
            }
        }
        // opacity: render.c:1830
        {
            const float sg = sigmoid_render(opacity[gi], exp_tab);
            gop += dop * (sg * (1.0f - sg));
        }
        // mean through the projection: render.c:1832-1845
        {
            const float inv_z = 1.0f / zc;
            const float inv_z2 = inv_z * inv_z;
            const float dmc0 = dmx * cam.fx * inv_z;
            const float dmc1 = dmy * cam.fy * inv_z;
            const float dmc2 = dmx * (-cam.fx * xc * inv_z2) + dmy * (-cam.fy * yc * inv_z2);
            gm[0] += w.m[0][0] * dmc0 + w.m[1][0] * dmc1 + w.m[2][0] * dmc2;
            gm[1] += w.m[0][1] * dmc0 + w.m[1][1] * dmc1 + w.m[2][1] * dmc2;
            gm[2] += w.m[0][2] * dmc0 + w.m[1][2] * dmc1 + w.m[2][2] * dmc2;
        }
        // covariance to scale and rotation: render.c:1847-1937
        {
            float mm[2][3];
#pragma unroll
            for (int col = 0; col < 3; ++col) {
                mm[0][col] = j00 * w.m[0][col] + j02 * w.m[2][col];
                mm[1][col] = j11 * w.m[1][col] + j12 * w.m[2][col];
            }
            Mat3 dcov3;
#pragma unroll
            for (int row = 0; row < 3; ++row)
#pragma unroll
                for (int col = 0; col < 3; ++col)
                    dcov3.m[row][col] = mm[0][row] * (dca * mm[0][col] + 0.5f * dcb * mm[1][col]) +
                                        mm[1][row] * (0.5f * dcb * mm[0][col] + dcc * mm[1][col]);
            Mat3 dsum;
#pragma unroll
            for (int row = 0; row < 3; ++row)
#pragma unroll
                for (int col = 0; col < 3; ++col) dsum.m[row][col] = dcov3.m[row][col] + dcov3.m[col][row];
            const Mat3 drs = mat3_mul(dsum, srot);
            gl[0] = (drs.m[0][0] * rot.m[0][0] + drs.m[1][0] * rot.m[1][0] + drs.m[2][0] * rot.m[2][0]) * sx;
            gl[1] = (drs.m[0][1] * rot.m[0][1] + drs.m[1][1] * rot.m[1][1] + drs.m[2][1] * rot.m[2][1]) * sy;
            gl[2] = (drs.m[0][2] * rot.m[0][2] + drs.m[1][2] * rot.m[1][2] + drs.m[2][2] * rot.m[2][2]) * sz;
            Mat3 dr;
#pragma unroll
            for (int row = 0; row < 3; ++row) {
                dr.m[row][0] = drs.m[row][0] * sx;
                dr.m[row][1] = drs.m[row][1] * sy;
                dr.m[row][2] = drs.m[row][2] * sz;
            }
            float nx, ny, nz, nw;
            if (quat_normalize(q.x, q.y, q.z, q.w, nx, ny, nz, nw)) {
                const float inv_norm = 1.0f / sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
                float dqw = 0.0f, dqx = 0.0f, dqy = 0.0f, dqz = 0.0f;
                dqw += dr.m[0][1] * (-2.0f * nz);
                dqw += dr.m[0][2] * (2.0f * ny);
                dqw += dr.m[1][0] * (2.0f * nz);
                dqw += dr.m[1][2] * (-2.0f * nx);
                dqw += dr.m[2][0] * (-2.0f * ny);
                dqw += dr.m[2][1] * (2.0f * nx);
                dqx += dr.m[0][1] * (2.0f * ny);
                dqx += dr.m[0][2] * (2.0f * nz);
                dqx += dr.m[1][0] * (2.0f * ny);
                dqx += dr.m[1][1] * (-4.0f * nx);
                dqx += dr.m[1][2] * (-2.0f * nw);
                dqx += dr.m[2][0] * (2.0f * nz);
                dqx += dr.m[2][1] * (2.0f * nw);
                dqx += dr.m[2][2] * (-4.0f * nx);
                dqy += dr.m[0][0] * (-4.0f * ny);
                dqy += dr.m[0][1] * (2.0f * nx);
                dqy += dr.m[0][2] * (2.0f * nw);
                dqy += dr.m[1][0] * (2.0f * nx);
                dqy += dr.m[1][2] * (2.0f * nz);
                dqy += dr.m[2][0] * (-2.0f * nw);
                dqy += dr.m[2][1] * (2.0f * nz);
                dqy += dr.m[2][2] * (-4.0f * ny);
                dqz += dr.m[0][0] * (-4.0f * nz);
                dqz += dr.m[0][1] * (-2.0f * nw);
                dqz += dr.m[0][2] * (2.0f * nx);
                dqz += dr.m[1][0] * (2.0f * nw);
                dqz += dr.m[1][1] * (-4.0f * nz);
                dqz += dr.m[1][2] * (2.0f * ny);
                dqz += dr.m[2][0] * (2.0f * nx);
                dqz += dr.m[2][1] * (2.0f * ny);
                const float dot = nx * dqx + ny * dqy + nz * dqz + nw * dqw;
                gr[0] = (dqx - nx * dot) * inv_norm;
                gr[1] = (dqy - ny * dot) * inv_norm;
                gr[2] = (dqz - nz * dot) * inv_norm;
                gr[3] = (dqw - nw * dot) * inv_norm;
            }
        }
        // Jacobian's dependence on the camera-space mean: render.c:1939-1969
        {
            const Mat3 cov_cam = mat3_mul_t(mat3_mul(w, cov3d), w);
            const float inv_z = 1.0f / zc;
            const float inv_z2 = inv_z * inv_z;
            const float inv_z3 = inv_z2 * inv_z;
            float dj[2][3];
#pragma unroll
            for (int col = 0; col < 3; ++col) {
                dj[0][col] = 2.0f * dca * (j00 * cov_cam.m[0][col] + j02 * cov_cam.m[2][col]) +
                             dcb * (j11 * cov_cam.m[1][col] + j12 * cov_cam.m[2][col]);
                dj[1][col] = dcb * (j00 * cov_cam.m[0][col] + j02 * cov_cam.m[2][col]) +
                             2.0f * dcc * (j11 * cov_cam.m[1][col] + j12 * cov_cam.m[2][col]);
            }
            const float m0 = dj[0][2] * (-cam.fx * inv_z2);
            const float m1 = dj[1][2] * (-cam.fy * inv_z2);
            const float m2 = dj[0][0] * (-cam.fx * inv_z2) + dj[0][2] * (2.0f * cam.fx * xc * inv_z3) +
                             dj[1][1] * (-cam.fy * inv_z2) + dj[1][2] * (2.0f * cam.fy * yc * inv_z3);
            gm[0] += w.m[0][0] * m0 + w.m[1][0] * m1 + w.m[2][0] * m2;
            gm[1] += w.m[0][1] * m0 + w.m[1][1] * m1 + w.m[2][1] * m2;
            gm[2] += w.m[0][2] * m0 + w.m[1][2] * m1 + w.m[2][2] * m2;
        }
    }
    if (valid) {
        // rows of 16 and 4 bytes: consecutive lanes already store consecutive addresses
        reinterpret_cast<float4*>(g_rotation)[gi] = make_float4(gr[0], gr[1], gr[2], gr[3]);
        g_opacity[gi] = gop;
    }
    if (vector_stores) {  // uniform: every 3-float (and SH) sink is 16-byte aligned
        const int count = (int)min((int64_t)blockDim.x, n - first);
        block_store_rows<3>(g_mean3d, first, count, gm, s_stage);
        block_store_rows<3>(g_logscale, first, count, gl, s_stage);
        block_store_rows<3>(g_sh0, first, count, gs0, s_stage);
        if (sh_degree >= 1) block_store_rows<9>(g_sh1, first, count, gs1, s_stage);
        if (sh_degree >= 2) block_store_rows<15>(g_sh2, first, count, gs2, s_stage);
        if (sh_degree >= 3) block_store_rows<21>(g_sh3, first, count, gs3, s_stage);
        return;
    }
    if (!valid) return;
    g_mean3d[gi * 3 + 0] = gm[0];
    g_mean3d[gi * 3 + 1] = gm[1];
    g_mean3d[gi * 3 + 2] = gm[2];
    g_logscale[gi * 3 + 0] = gl[0];
    g_logscale[gi * 3 + 1] = gl[1];
    g_logscale[gi * 3 + 2] = gl[2];
    g_sh0[gi * 3 + 0] = gs0[0];
    g_sh0[gi * 3 + 1] = gs0[1];
    g_sh0[gi * 3 + 2] = gs0[2];
    if (sh_degree >= 1)
        for (int i = 0; i < 9; ++i) g_sh1[gi * 9 + i] = gs1[i];
    if (sh_degree >= 2)
        for (int i = 0; i < 15; ++i) g_sh2[gi * 15 + i] = gs2[i];
    if (sh_degree >= 3)
        for (int i = 0; i < 21; ++i) g_sh3[gi * 21 + i] = gs3[i];
}

}  // namespace gsx_amd
