// abi.hip - host side of libgsx_hip.so: device plumbing, the render context (pooled buffers,
// retained TRAIN state, stage timing) and the forward/backward pipelines.
//
// Forward (one stream, in order):
//   preprocess (+ per-Gaussian depth keys) -> radix sort of the depth keys -> tile counts in
//   depth order -> exclusive scan -> [host reads the instance count] -> key emission in depth
//   order -> stable radix sort on the tile bits -> tile ranges -> blend.
// Backward:
//   blend backward (per-instance partials, no atomics) -> per-Gaussian sums of each Gaussian's
//   run of partials -> projection backward.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <new>

#include "../../include/gsx_hip.h"
#include "common.hpp"

// The render kernels are compiled in this translation unit so their launches need no
// relocatable device code.
#include "render.hip"

using namespace gsx_amd;

namespace gsx_amd {
// Plain streaming copy: 16 B per lane per iteration, grid-stride.
__global__ __launch_bounds__(256) void copy_f32_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                       int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// The Gaussian field arrays a TRAIN forward retains (gsx-cpu/render.c:263-380): up to 8 arrays
// of floats, compared with the context's copy in one launch, blockIdx.y selecting the array.
// 16-byte vectors where the caller's array and the copy are both 16-byte aligned.
constexpr int kStateFields = 8;
struct StateArrays {
    const float* live[kStateFields];
    float* snap[kStateFields];
    int64_t count[kStateFields];  // floats
};

__device__ inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// *changed = 1 when any bit of live differs from snap (a NaN payload or the sign of a zero
// counts as a change, as any other write would).
__global__ __launch_bounds__(256) void train_state_kernel(StateArrays a, uint32_t* __restrict__ changed) {
    const int f = blockIdx.y;
    const float* live = a.live[f];
    const float* snap = a.snap[f];
    const int64_t n = a.count[f];
    if (live == nullptr || n == 0) return;  // uniform
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    bool diff = false;
    if (aligned16(live) && aligned16(snap)) {
        const int64_t n4 = n / 4;
        const uint4* l4 = reinterpret_cast<const uint4*>(live);
        const uint4* s4 = reinterpret_cast<const uint4*>(snap);
        // four 16-byte pairs per thread and round, all loads issued before the first compare
        // (positions past the end re-read the last vector, which cannot differ from itself)
        constexpr int kRound = 4;
        for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n4; i0 += kRound * stride) {
            uint4 v[kRound], w[kRound];
#pragma unroll
            for (int u = 0; u < kRound; ++u) {
                const int64_t i = min(i0 + u * stride, n4 - 1);
                v[u] = l4[i];
                w[u] = s4[i];
            }
#pragma unroll
            for (int u = 0; u < kRound; ++u)
                diff |= (v[u].x != w[u].x) | (v[u].y != w[u].y) | (v[u].z != w[u].z) | (v[u].w != w[u].w);
        }
        for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
            diff |= __float_as_uint(live[i]) != __float_as_uint(snap[i]);
    } else {
        for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
            diff |= __float_as_uint(live[i]) != __float_as_uint(snap[i]);
    }
    if (wave_ballot(diff) != 0ull && __lane_id() == 0) *changed = 1u;
}
}  // namespace gsx_amd

namespace {

thread_local char g_message[256] = "";

gsx_hip_status fail(gsx_hip_status code, const char* what) {
    snprintf(g_message, sizeof(g_message), "%s", what);
    return code;
}

}  // namespace

namespace gsx_amd {
void set_last_error(const char* what) { snprintf(g_message, sizeof(g_message), "%s", what); }
}  // namespace gsx_amd

namespace {

gsx_hip_status hip_fail(hipError_t e, const char* what) {
    snprintf(g_message, sizeof(g_message), "%s: %s", what, hipGetErrorString(e));
    return (gsx_hip_status)e;
}

#define GSX_HIP_TRY(expr, what)                 \
    do {                                        \
        hipError_t e_ = (expr);                 \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

#define GSX_TRY(expr)                           \
    do {                                        \
        gsx_hip_status s_ = (expr);             \
        if (s_ != GSX_HIP_SUCCESS) return s_;   \
    } while (0)

// Grow-only device buffer: the render context keeps its intermediates across calls, so steady
// state training performs no allocation (gsx's CPU/CUDA contexts reset and re-grow arenas on
// every forward, gsx/src/gsx-cuda/render.c:346-377). Memory comes from the stream-ordered pool
// (pool.hip): every call reserves each buffer it uses on its stream, and an outgrown or released
// buffer returns to the pool behind that stream's queued work.
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipStream_t stream = nullptr;  // the stream of the last call that reserved it

    gsx_hip_status reserve(size_t need, const char* what, hipStream_t s) {
        stream = s;
        if (need <= bytes) return GSX_HIP_SUCCESS;
        size_t grow = need + need / 4 + 4096;
        if (ptr != nullptr) {
            gsx_hip_status st = gsx_hip_pool_free(ptr, s);
            ptr = nullptr;
            bytes = 0;
            if (st != GSX_HIP_SUCCESS) return st;
        }
        gsx_hip_status st = gsx_hip_pool_malloc(&ptr, grow, s);
        if (st != GSX_HIP_SUCCESS) {
            ptr = nullptr;
            return st == GSX_HIP_ERROR_OUT_OF_MEMORY ? fail(st, what) : st;
        }
        bytes = grow;
        return GSX_HIP_SUCCESS;
    }
    void release() {
        if (ptr != nullptr) (void)gsx_hip_pool_free(ptr, stream);
        ptr = nullptr;
        bytes = 0;
    }
    template <typename T>
    T* as() const {
        return static_cast<T*>(ptr);
    }
};

// Grow-only pinned host buffer that kernels write through its device mapping (the per-workgroup
// partial instance counts the host sums once the counting kernels have run).
struct PinnedBuffer {
    void* host = nullptr;
    void* dev = nullptr;
    size_t bytes = 0;

    gsx_hip_status reserve(size_t need, const char* what) {
        if (need <= bytes) return GSX_HIP_SUCCESS;
        const size_t grow = need + need / 4 + 4096;
        release();
        hipError_t e = hipHostMalloc(&host, grow, hipHostMallocDefault);
        if (e == hipSuccess) e = hipHostGetDevicePointer(&dev, host, 0);
        if (e != hipSuccess) {
            release();
            return hip_fail(e, what);
        }
        bytes = grow;
        return GSX_HIP_SUCCESS;
    }
    void release() {
        if (host != nullptr) (void)hipHostFree(host);
        host = nullptr;
        dev = nullptr;
        bytes = 0;
    }
};

// Instance counts from which the tile ranges come from a binary search per tile rather than a
// pass over the sorted tiles (the search's cost does not grow with the count)
constexpr int64_t kRangesSearchMin = (int64_t)1 << 25;
// Workgroups of the long-run reduction (4 waves each, each wave 64 list entries at a time): for
// chunk 0, which every long run has, and per later chunk.
constexpr unsigned kLongRunBlocks0 = 1024;
constexpr unsigned kLongRunBlocks = 128;

// Long instance runs are summed in chunks of this many positions: a run has at most `tiles`
// instances, so at most kLongChunks chunks.
uint32_t long_chunk_of(int32_t tiles) {
    return std::max<uint32_t>(kWave,
                              ((uint32_t)(tiles + (int)kLongChunks - 1) / kLongChunks + kWave - 1) / kWave * kWave);
}

unsigned blocks_for(int64_t n, int threads) {
    int64_t b = (n + threads - 1) / threads;
    return (unsigned)(b < 1 ? 1 : b);
}

// Pose quaternion to world-to-camera matrix and camera centre, with the CPU's arithmetic
// (render.c:561-581, 603-609), evaluated once on the host.
CameraParams make_camera_params(const gsx_hip_camera& c) {
    CameraParams p;
    float qx = c.rot[0], qy = c.rot[1], qz = c.rot[2], qw = c.rot[3];
    float norm_sq = qx * qx + qy * qy + qz * qz + qw * qw;
    if (norm_sq <= kMinQuatNormSq) {
        qx = 0.0f;
        qy = 0.0f;
        qz = 0.0f;
        qw = 1.0f;
    } else {
        float inv_norm = 1.0f / sqrtf(norm_sq);
        qx = qx * inv_norm;
        qy = qy * inv_norm;
        qz = qz * inv_norm;
        qw = qw * inv_norm;
    }
    p.w[0][0] = 1.0f - 2.0f * (qy * qy + qz * qz);
    p.w[0][1] = 2.0f * (qx * qy - qw * qz);
    p.w[0][2] = 2.0f * (qx * qz + qw * qy);
    p.w[1][0] = 2.0f * (qx * qy + qw * qz);
    p.w[1][1] = 1.0f - 2.0f * (qx * qx + qz * qz);
    p.w[1][2] = 2.0f * (qy * qz - qw * qx);
    p.w[2][0] = 2.0f * (qx * qz - qw * qy);
    p.w[2][1] = 2.0f * (qy * qz + qw * qx);
    p.w[2][2] = 1.0f - 2.0f * (qx * qx + qy * qy);
    for (int i = 0; i < 3; ++i) p.t[i] = c.transl[i];
    for (int i = 0; i < 3; ++i) {
        float v = p.w[0][i] * c.transl[0] + p.w[1][i] * c.transl[1] + p.w[2][i] * c.transl[2];
        p.centre[i] = v * -1.0f;
    }
    p.fx = c.fx;
    p.fy = c.fy;
    p.cx = c.cx;
    p.cy = c.cy;
    p.near_plane = c.near_plane;
    p.far_plane = c.far_plane;
    for (int i = 0; i < 3; ++i) p.bg[i] = c.background[i];
    p.width = c.width;
    p.height = c.height;
    p.tiles_x = (c.width + kTile - 1) / kTile;
    p.tiles_y = (c.height + kTile - 1) / kTile;
    return p;
}

int bits_for(uint32_t v) {
    int b = 0;
    while (b < 32 && (1ull << b) < (uint64_t)v + 1ull) ++b;
    return b;
}

}  // namespace

struct gsx_hip_render_context {
    DeviceBuffer rec, cov_coef, ckpt, inst_gauss, inst_tile, tiles_alt, tiles_sorted, vals_alt, vals, tile_cut, touched,
        inst_grad, tile_count, big_list, offsets, scan_temp, sort_temp, ranges, sorted_g, final_t, last, grad2d,
        depth_keys, depth_keys_alt, rank_g, rank_count, g_rank, long_list, multi_list, counters,
        depth_sort_temp;
    // partial instance counts written by preprocess (one u64 per workgroup), summed on the host
    // after count_ev
    PinnedBuffer kept_parts;
    hipEvent_t count_ev = nullptr;
    // Retained TRAIN state (gsx-cpu/render.c:263-380): the Gaussian fields as the forward read
    // them, copied into `snap`, which the backward reads (gs points into it). A borrowed state
    // also keeps the caller's arrays (`live`): the backward first compares them with `snap`
    // (`changed`, host-mapped, read after state_ev) and, when the caller has changed them, re-runs
    // the forward on their current values (into refresh_rgb), as gsx-cuda/render.c:662-756 does.
    DeviceBuffer snap, refresh_rgb;
    PinnedBuffer changed;
    hipEvent_t state_ev = nullptr;
    // the comparison runs on a stream of its own (default priority), forked from the caller's
    // stream at fork_ev, beside the backward: it reads HBM while the blend kernels are bound by
    // their vector ALUs
    hipStream_t check_stream = nullptr;
    // the stream of the current forward or backward call: its buffer reserves are ordered on it
    hipStream_t call_stream = nullptr;
    hipEvent_t fork_ev = nullptr;
    gsx_hip_gaussians live{};
    gsx_hip_camera camera{};
    int32_t train_mode = GSX_HIP_FORWARD_INFERENCE;
    // counters: [0] visible Gaussians (depth keys), [1] unused, [2 + big_slot] big boxes
    // of the next forward (each forward's preprocess clears the other slot for its successor),
    // [4] runs of more than one long-run chunk
    bool counters_ready = false;
    int big_slot = 0;
    CameraParams cam{};
    gsx_hip_gaussians gs{};
    int64_t instance_count = 0;
    int64_t gaussian_count = 0;
    int64_t visible_count = 0;  // Gaussians past the projection culls in the last forward
    int32_t tile_count_total = 0;
    int32_t sort_passes = 0;
    int32_t depth_sort_passes = 0;
    int32_t tile_bits = 0;            // bits of the tile index the sort orders
    uint32_t* sorted_vals = nullptr;  // emission position of each sorted instance
    bool has_train_state = false;
    // Stage timing: a ring of event sets, one set per forward/backward pair, so that a timed
    // loop records without synchronising; get_timings averages over the recorded sets.
    static constexpr int kEventsPerSet = GSX_HIP_RENDER_STAGE_COUNT + 2;
    bool timing = false;
    int32_t ring = 0;           // number of event sets
    hipEvent_t* events = nullptr;
    int32_t cur = -1;           // set of the current forward/backward pair
    int32_t fwd_sets = 0;       // sets with a recorded forward (capped at ring)
    int32_t bwd_sets = 0;
    uint8_t* has_fwd = nullptr;
    uint8_t* has_bwd = nullptr;
};

namespace {

gsx_hip_status record(gsx_hip_render_context* ctx, int idx, hipStream_t stream) {
    if (!ctx->timing || ctx->cur < 0) return GSX_HIP_SUCCESS;
    GSX_HIP_TRY(hipEventRecord(ctx->events[ctx->cur * gsx_hip_render_context::kEventsPerSet + idx], stream),
                "hipEventRecord");
    return GSX_HIP_SUCCESS;
}

void release_events(gsx_hip_render_context* ctx) {
    if (ctx->events != nullptr) {
        for (int i = 0; i < ctx->ring * gsx_hip_render_context::kEventsPerSet; ++i) (void)hipEventDestroy(ctx->events[i]);
    }
    delete[] ctx->events;
    delete[] ctx->has_fwd;
    delete[] ctx->has_bwd;
    ctx->events = nullptr;
    ctx->has_fwd = nullptr;
    ctx->has_bwd = nullptr;
    ctx->ring = 0;
}

// Field order of the retained state: mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3.
constexpr int kFieldWidth[kStateFields] = {3, 4, 3, 1, 3, 9, 15, 21};

const float* field_ptr(const gsx_hip_gaussians& g, int f) {
    const float* p[kStateFields] = {g.mean3d, g.rotation, g.logscale, g.opacity, g.sh0, g.sh1, g.sh2, g.sh3};
    return p[f];
}

int field_count(const gsx_hip_gaussians& g) { return 5 + g.sh_degree; }

// Lays the snapshot of g out in one buffer (each array 64-byte aligned) and points `snap_gs` at it.
gsx_hip_status snapshot_layout(gsx_hip_render_context* ctx, const gsx_hip_gaussians& g, gsx_hip_gaussians* snap_gs,
                               StateArrays* arrays) {
    size_t off[kStateFields] = {};
    size_t total = 0;
    const size_t n = (size_t)g.count;
    for (int f = 0; f < field_count(g); ++f) {
        off[f] = total;
        total += (n * (size_t)kFieldWidth[f] + 15u) / 16u * 16u;
    }
    GSX_TRY(ctx->snap.reserve((total > 0 ? total : 1) * sizeof(float), "train state snapshot", ctx->call_stream));
    float* base = ctx->snap.as<float>();
    float* fp[kStateFields] = {};
    *arrays = StateArrays{};
    for (int f = 0; f < kStateFields; ++f) {
        const bool used = f < field_count(g);
        fp[f] = used ? base + off[f] : nullptr;
        arrays->live[f] = used ? field_ptr(g, f) : nullptr;
        arrays->snap[f] = fp[f];
        arrays->count[f] = used ? (int64_t)(n * (size_t)kFieldWidth[f]) : 0;
    }
    *snap_gs = g;
    snap_gs->mean3d = fp[0];
    snap_gs->rotation = fp[1];
    snap_gs->logscale = fp[2];
    snap_gs->opacity = fp[3];
    snap_gs->sh0 = fp[4];
    snap_gs->sh1 = fp[5];
    snap_gs->sh2 = fp[6];
    snap_gs->sh3 = fp[7];
    return GSX_HIP_SUCCESS;
}

// Workgroups per field array of the borrowed-state comparison, which runs beside the backward
constexpr unsigned kCheckBlocks = 16;

unsigned state_blocks(int64_t n) {
    // enough workgroups per array to fill the GPU, capped for small sets
    const int64_t b = (n * 3 + 1023) / 1024;
    return (unsigned)std::min<int64_t>(std::max<int64_t>(b, 1), 1024);
}

gsx_hip_status validate_gaussians(const gsx_hip_gaussians* g) {
    if (g == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "gaussians must be non-null");
    if (g->count < 0 || g->count > 0x7fffffffll) return fail(GSX_HIP_ERROR_OUT_OF_RANGE, "gaussian count out of range");
    if (g->sh_degree < 0 || g->sh_degree > 3) return fail(GSX_HIP_ERROR_OUT_OF_RANGE, "sh_degree must be in [0,3]");
    if (g->count > 0 && (g->mean3d == nullptr || g->rotation == nullptr || g->logscale == nullptr ||
                         g->opacity == nullptr || g->sh0 == nullptr)) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "mean3d, rotation, logscale, opacity and sh0 must be non-null");
    }
    if ((g->sh_degree >= 1 && g->sh1 == nullptr) || (g->sh_degree >= 2 && g->sh2 == nullptr) ||
        (g->sh_degree >= 3 && g->sh3 == nullptr)) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "sh1..sh3 must be non-null up to sh_degree");
    }
    if ((reinterpret_cast<uintptr_t>(g->rotation) & 15u) != 0) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "rotation must be 16-byte aligned");
    }
    return GSX_HIP_SUCCESS;
}

}  // namespace

extern "C" {

const char* gsx_hip_last_error_message(void) { return g_message; }

gsx_hip_status gsx_hip_device_count(int32_t* out_count) {
    if (out_count == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_count must be non-null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *out_count = 0;
        return hip_fail(e, "hipGetDeviceCount");
    }
    *out_count = n;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_device_name(int32_t device, char* out_name, size_t capacity) {
    if (out_name == nullptr || capacity == 0) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_name must be non-null");
    hipDeviceProp_t prop;
    GSX_HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    snprintf(out_name, capacity, "%s (%s)", prop.name, prop.gcnArchName);
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_malloc(void** out_ptr, size_t bytes) {
    if (out_ptr == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_ptr must be non-null");
    GSX_HIP_TRY(hipMalloc(out_ptr, bytes == 0 ? 1 : bytes), "hipMalloc");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_free(void* ptr) {
    GSX_HIP_TRY(hipFree(ptr), "hipFree");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_memcpy_htod(void* dst, const void* src, size_t bytes) {
    GSX_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    GSX_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_memcpy_dtod_async(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    GSX_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync D2D");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_memcpy_async(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return GSX_HIP_SUCCESS;
    if (dst == nullptr || src == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "copy pointers must be non-null");
    GSX_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, stream), "hipMemcpyAsync");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_set_device(int32_t device) {
    GSX_HIP_TRY(hipSetDevice(device), "hipSetDevice");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_device_total_memory(int32_t device, size_t* out_bytes) {
    if (out_bytes == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_bytes must be non-null");
    hipDeviceProp_t prop;
    GSX_HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    *out_bytes = prop.totalGlobalMem;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_host_alloc(void** out_host, size_t bytes) {
    if (out_host == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_host must be non-null");
    *out_host = nullptr;
    GSX_HIP_TRY(hipHostMalloc(out_host, bytes == 0 ? 1 : bytes, hipHostMallocDefault), "hipHostMalloc");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_host_free(void* host) {
    if (host == nullptr) return GSX_HIP_SUCCESS;
    GSX_HIP_TRY(hipHostFree(host), "hipHostFree");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_host_device_pointer(void* host, void** out_device) {
    if (host == nullptr || out_device == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "pointers must be non-null");
    GSX_HIP_TRY(hipHostGetDevicePointer(out_device, host, 0), "hipHostGetDevicePointer");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_stream_create(hipStream_t* out_stream) {
    if (out_stream == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_stream must be non-null");
    GSX_HIP_TRY(hipStreamCreateWithFlags(out_stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_stream_destroy(hipStream_t stream) {
    GSX_HIP_TRY(hipStreamDestroy(stream), "hipStreamDestroy");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_stream_synchronize(hipStream_t stream) {
    GSX_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_event_create(hipEvent_t* out_event) {
    if (out_event == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_event must be non-null");
    GSX_HIP_TRY(hipEventCreateWithFlags(out_event, hipEventDisableTiming), "hipEventCreateWithFlags");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_event_destroy(hipEvent_t event) {
    GSX_HIP_TRY(hipEventDestroy(event), "hipEventDestroy");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_event_record(hipEvent_t event, hipStream_t stream) {
    GSX_HIP_TRY(hipEventRecord(event, stream), "hipEventRecord");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_event_synchronize(hipEvent_t event) {
    GSX_HIP_TRY(hipEventSynchronize(event), "hipEventSynchronize");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_stream_wait_event(hipStream_t stream, hipEvent_t event) {
    GSX_HIP_TRY(hipStreamWaitEvent(stream, event, 0), "hipStreamWaitEvent");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_fill_f32(float* dst, int64_t count, float value, hipStream_t stream) {
    if (count <= 0) return GSX_HIP_SUCCESS;
    if (dst == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "dst must be non-null");
    hipLaunchKernelGGL(fill_f32_kernel, dim3(blocks_for(count, 256)), dim3(256), 0, stream, dst, count, value);
    GSX_HIP_TRY(hipGetLastError(), "fill_f32_kernel");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_copy_f32(float* dst, const float* src, int64_t count, hipStream_t stream) {
    if (count <= 0) return GSX_HIP_SUCCESS;
    if (dst == nullptr || src == nullptr || (count & 3) != 0 ||
        ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) != 0) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "copy needs 16-byte aligned buffers and a multiple of 4 floats");
    }
    const int64_t n4 = count / 4;
    unsigned blocks = blocks_for(n4, 256);
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(copy_f32_kernel, dim3(blocks), dim3(256), 0, stream, reinterpret_cast<const float4*>(src),
                       reinterpret_cast<float4*>(dst), n4);
    GSX_HIP_TRY(hipGetLastError(), "copy_f32_kernel");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_context_create(gsx_hip_render_context** out_context) {
    if (out_context == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_context must be non-null");
    *out_context = nullptr;
    gsx_hip_render_context* ctx = new (std::nothrow) gsx_hip_render_context();
    if (ctx == nullptr) return fail(GSX_HIP_ERROR_OUT_OF_MEMORY, "render context allocation failed");
    hipError_t e = hipEventCreateWithFlags(&ctx->count_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->state_ev, hipEventDisableTiming);
    // fork_ev only orders the comparison's stream after the caller's (device-side): no
    // system-scope fence (its cache flush would idle the GPU before every borrowed backward)
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming | hipEventDisableSystemFence);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->check_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        (void)gsx_hip_render_context_destroy(ctx);
        return hip_fail(e, "render context creation");
    }
    *out_context = ctx;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_context_destroy(gsx_hip_render_context* ctx) {
    if (ctx == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context must be non-null");
    DeviceBuffer* all[] = {&ctx->rec,       &ctx->cov_coef, &ctx->ckpt,      &ctx->inst_gauss, &ctx->inst_tile,
                           &ctx->tiles_alt, &ctx->tiles_sorted, &ctx->vals_alt, &ctx->vals,
                           &ctx->tile_cut,  &ctx->touched,  &ctx->inst_grad,
                           &ctx->tile_count, &ctx->big_list, &ctx->offsets,   &ctx->scan_temp,
                           &ctx->sort_temp,  &ctx->ranges,
                           &ctx->sorted_g,   &ctx->final_t,  &ctx->last,      &ctx->grad2d,     &ctx->depth_keys,
                           &ctx->depth_keys_alt, &ctx->rank_g, &ctx->rank_count, &ctx->g_rank,
                           &ctx->long_list, &ctx->multi_list, &ctx->counters,
                           &ctx->depth_sort_temp, &ctx->snap, &ctx->refresh_rgb};
    for (DeviceBuffer* b : all) b->release();
    ctx->kept_parts.release();
    ctx->changed.release();
    if (ctx->count_ev != nullptr) (void)hipEventDestroy(ctx->count_ev);
    if (ctx->state_ev != nullptr) (void)hipEventDestroy(ctx->state_ev);
    if (ctx->fork_ev != nullptr) (void)hipEventDestroy(ctx->fork_ev);
    if (ctx->check_stream != nullptr) (void)hipStreamDestroy(ctx->check_stream);
    release_events(ctx);
    delete ctx;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_context_set_timing(gsx_hip_render_context* ctx, int32_t capacity) {
    if (ctx == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context must be non-null");
    if (capacity < 0 || capacity > 100000) return fail(GSX_HIP_ERROR_OUT_OF_RANGE, "timing capacity out of range");
    release_events(ctx);
    ctx->timing = capacity > 0;
    ctx->cur = -1;
    ctx->fwd_sets = 0;
    ctx->bwd_sets = 0;
    if (capacity == 0) return GSX_HIP_SUCCESS;
    const int total = capacity * gsx_hip_render_context::kEventsPerSet;
    ctx->events = new (std::nothrow) hipEvent_t[total];
    ctx->has_fwd = new (std::nothrow) uint8_t[capacity]();
    ctx->has_bwd = new (std::nothrow) uint8_t[capacity]();
    if (ctx->events == nullptr || ctx->has_fwd == nullptr || ctx->has_bwd == nullptr) {
        release_events(ctx);
        ctx->timing = false;
        return fail(GSX_HIP_ERROR_OUT_OF_MEMORY, "timing ring allocation failed");
    }
    for (int i = 0; i < total; ++i) {
        // timing only: no system-scope fence at each stage boundary (its cache writeback would be
        // counted in the stage it follows, and would slow the next one)
        hipError_t e = hipEventCreateWithFlags(&ctx->events[i], hipEventDisableSystemFence);
        if (e != hipSuccess) {
            for (int k = 0; k < i; ++k) (void)hipEventDestroy(ctx->events[k]);
            delete[] ctx->events;
            ctx->events = nullptr;
            ctx->ring = 0;
            release_events(ctx);
            ctx->timing = false;
            return hip_fail(e, "hipEventCreateWithFlags");
        }
    }
    ctx->ring = capacity;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_context_get_timings(gsx_hip_render_context* ctx, float* out_ms, int32_t capacity,
                                                  int32_t* out_written) {
    if (ctx == nullptr || out_ms == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context/out_ms null");
    if (!ctx->timing) return fail(GSX_HIP_ERROR_INVALID_STATE, "timing is not enabled");
    // per set: 0 fwd start, 1 preprocess, 2 depth order (+count readback), 3 emit, 4 sort, 5 ranges,
    //          6 blend; 7 bwd start, 8 blend bwd, 9 instance reduce, 10 projection bwd
    double sum[GSX_HIP_RENDER_STAGE_COUNT] = {0.0};
    int nf = 0, nb = 0;
    for (int set = 0; set < ctx->ring; ++set) {
        hipEvent_t* ev = ctx->events + set * gsx_hip_render_context::kEventsPerSet;
        if (ctx->has_fwd[set]) {
            GSX_HIP_TRY(hipEventSynchronize(ev[6]), "hipEventSynchronize");
            for (int i = 0; i < 6; ++i) {
                float ms = 0.0f;
                GSX_HIP_TRY(hipEventElapsedTime(&ms, ev[i], ev[i + 1]), "hipEventElapsedTime");
                sum[i] += ms;
            }
            ++nf;
        }
        if (ctx->has_bwd[set]) {
            GSX_HIP_TRY(hipEventSynchronize(ev[10]), "hipEventSynchronize");
            for (int i = 0; i < 3; ++i) {
                float ms = 0.0f;
                GSX_HIP_TRY(hipEventElapsedTime(&ms, ev[7 + i], ev[8 + i]), "hipEventElapsedTime");
                sum[6 + i] += ms;
            }
            ++nb;
        }
    }
    const int n = capacity < GSX_HIP_RENDER_STAGE_COUNT ? capacity : GSX_HIP_RENDER_STAGE_COUNT;
    for (int i = 0; i < n; ++i) {
        const int denom = i < 6 ? nf : nb;
        out_ms[i] = denom > 0 ? (float)(sum[i] / denom) : 0.0f;
    }
    if (out_written) *out_written = n;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_forward(gsx_hip_render_context* ctx, const gsx_hip_camera* camera,
                                      const gsx_hip_gaussians* gaussians, int32_t train, float* out_rgb,
                                      float* visible_counter, hipStream_t stream) {
    if (ctx == nullptr || camera == nullptr || out_rgb == nullptr) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context, camera and out_rgb must be non-null");
    }
    GSX_TRY(validate_gaussians(gaussians));
    if (camera->width <= 0 || camera->height <= 0 || camera->width > 32767 || camera->height > 32767) {
        return fail(GSX_HIP_ERROR_OUT_OF_RANGE, "image width/height must be in [1, 32767]");
    }
    if (!(camera->near_plane > 0.0f) || !(camera->far_plane > camera->near_plane) || !isfinite(camera->far_plane)) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "near_plane and far_plane must be finite with 0 < near < far");
    }
    if (train != GSX_HIP_FORWARD_INFERENCE && train != GSX_HIP_FORWARD_TRAIN_BORROW &&
        train != GSX_HIP_FORWARD_TRAIN_CLONE) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "forward type must be a GSX_HIP_FORWARD_* value");
    }
    ctx->has_train_state = false;
    ctx->call_stream = stream;
    const CameraParams cam = make_camera_params(*camera);
    const int64_t n = gaussians->count;
    const int32_t tiles = cam.tiles_x * cam.tiles_y;
    const int64_t pixels = (int64_t)cam.width * cam.height;
    const int tile_bits = bits_for((uint32_t)(tiles > 0 ? tiles - 1 : 0));
    ctx->cam = cam;
    ctx->gs = *gaussians;  // replaced by the snapshot below for a TRAIN forward
    ctx->gaussian_count = n;
    ctx->visible_count = 0;
    ctx->tile_count_total = tiles;

    const size_t n1 = (size_t)(n > 0 ? n : 1);
    // per Gaussian: geometry (2 float4), colour / depth (float4) at 2n, contribution box (uint2) at 3n
    GSX_TRY(ctx->rec.reserve(n1 * (3 * sizeof(float4) + sizeof(uint2)), "rec", ctx->call_stream));
    if (train) GSX_TRY(ctx->cov_coef.reserve(n1 * 2 * sizeof(float4), "cov_coef", ctx->call_stream));
    if (train) GSX_TRY(ctx->touched.reserve(n1, "touched", ctx->call_stream));
    GSX_TRY(ctx->tile_count.reserve(n1 * sizeof(uint32_t), "tile_count", ctx->call_stream));
    GSX_TRY(ctx->counters.reserve(8 * sizeof(uint32_t), "counters", ctx->call_stream));
    GSX_TRY(ctx->big_list.reserve(n1 * sizeof(uint32_t), "big_list", ctx->call_stream));
    GSX_TRY(ctx->offsets.reserve((size_t)(n + 1) * sizeof(uint32_t), "offsets", ctx->call_stream));
    // per 256-rank workgroup: its tile-count sum, then its long-run count (two scanned arrays)
    GSX_TRY(ctx->scan_temp.reserve(2 * ((size_t)blocks_for(n, 256) + 1) * sizeof(uint32_t), "rank_block_sums", ctx->call_stream));
    GSX_TRY(ctx->long_list.reserve(n1 * sizeof(uint32_t), "long_list", ctx->call_stream));
    GSX_TRY(ctx->depth_keys.reserve(n1 * sizeof(uint64_t), "depth_keys", ctx->call_stream));
    GSX_TRY(ctx->depth_keys_alt.reserve(n1 * sizeof(uint64_t), "depth_keys_alt", ctx->call_stream));
    GSX_TRY(ctx->rank_g.reserve(n1 * sizeof(uint32_t), "rank_gaussian", ctx->call_stream));
    GSX_TRY(ctx->rank_count.reserve(n1 * sizeof(uint32_t), "rank_count", ctx->call_stream));
    GSX_TRY(ctx->g_rank.reserve(n1 * sizeof(uint32_t), "gaussian_rank", ctx->call_stream));
    GSX_TRY(ctx->multi_list.reserve(n1 * sizeof(uint32_t), "multi_list", ctx->call_stream));
    GSX_TRY(ctx->depth_sort_temp.reserve(radix_sort_keys_u64_compacting_temp_bytes(n), "depth_sort_temp", ctx->call_stream));
    GSX_TRY(ctx->ranges.reserve((size_t)tiles * sizeof(uint2), "ranges", ctx->call_stream));
    GSX_TRY(ctx->final_t.reserve((size_t)pixels * sizeof(float), "final_t", ctx->call_stream));
    GSX_TRY(ctx->last.reserve((size_t)pixels * sizeof(uint32_t), "last", ctx->call_stream));
    uint32_t* counters = ctx->counters.as<uint32_t>();
    const unsigned pre_blocks = blocks_for(n, 256);
    GSX_TRY(ctx->kept_parts.reserve((size_t)pre_blocks * sizeof(unsigned long long), "kept_parts"));
    uint32_t* big_count = counters + 2 + ctx->big_slot;

    // depth keys of the visible Gaussians: (bits(depth) - bits(near)) << index_bits | index (see
    // KeyLayout), at most 31 + 32 bits, so never the all-ones key that marks invisible ones
    const uint32_t near_bits = gsx_f32_bits(cam.near_plane), far_bits = gsx_f32_bits(cam.far_plane);
    const uint32_t depth_max = far_bits - near_bits;
    const int index_bits = std::max(1, bits_for((uint32_t)(n > 0 ? n - 1 : 0)));
    const int depth_bits = bits_for(depth_max);
    ctx->depth_sort_passes = (depth_bits + kCompactingRadixBits - 1) / kCompactingRadixBits;
    const int depth_end_bit = std::min(64, index_bits + ctx->depth_sort_passes * kCompactingRadixBits);
    // big boxes are flagged in bit 63 of their depth key when the sort never reaches that bit
    const bool big_flag = depth_end_bit <= 63;
    // the kept-tile count (at most `tiles`) rides in the bits above the sorted ones when they fit
    // below the big-box flag; its field is never all ones, so no visible key is the all-ones key
    // the depth sort drops
    const int count_bits = bits_for((uint32_t)tiles + 1u);
    const int count_shift = (big_flag && depth_end_bit + count_bits <= 63) ? depth_end_bit : 0;

    if (ctx->timing) {
        ctx->cur = (ctx->cur + 1) % ctx->ring;
        ctx->has_fwd[ctx->cur] = 0;
        ctx->has_bwd[ctx->cur] = 0;
    }
    GSX_TRY(record(ctx, 0, stream));
    FieldSnapshot snap{};
    if (train) {
        // the retained state: preprocess copies the fields as it reads them
        gsx_hip_gaussians snap_gs;
        StateArrays arrays;
        GSX_TRY(snapshot_layout(ctx, *gaussians, &snap_gs, &arrays));
        for (int f = 0; f < kStateFields; ++f) snap.dst[f] = arrays.snap[f];
        ctx->gs = snap_gs;
        ctx->live = *gaussians;
        ctx->camera = *camera;
    }
    ctx->train_mode = train;
    if (n > 0) {
        if (!ctx->counters_ready) {
            hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, stream, counters, (int64_t)8, 0u);
            GSX_HIP_TRY(hipGetLastError(), "fill_u32_kernel");
            ctx->counters_ready = true;
        }
        hipLaunchKernelGGL(preprocess_kernel, dim3(pre_blocks), dim3(256), 0, stream, snap, n, gaussians->mean3d,
                           gaussians->rotation, gaussians->logscale, gaussians->opacity, gaussians->sh0,
                           gaussians->sh1, gaussians->sh2, gaussians->sh3, (int)gaussians->sh_degree, cam,
                           ctx->rec.as<float4>(), ctx->rec.as<float4>() + 2 * n,
                           reinterpret_cast<uint2*>(ctx->rec.as<float4>() + 3 * n),
                           train ? ctx->cov_coef.as<float4>() : nullptr,
                           ctx->tile_count.as<uint32_t>(), train ? visible_counter : nullptr,
                           ctx->big_list.as<uint32_t>(), big_count, counters + 1, counters + 2 + (ctx->big_slot ^ 1),
                           counters + 4,
                           static_cast<unsigned long long*>(ctx->kept_parts.dev), ctx->depth_keys.as<uint64_t>(),
                           near_bits,
                           depth_max, index_bits, big_flag ? kBigKeyFlag : 0ull, count_shift,
                           train ? ctx->touched.as<uint8_t>() : nullptr);
        GSX_HIP_TRY(hipGetLastError(), "preprocess_kernel");
        ctx->big_slot ^= 1;  // the slot this preprocess cleared
    }
    // the counting kernels leave the instance count as per-workgroup partials in host memory;
    // the depth order and the count scan are queued behind them, so the GPU keeps working while
    // the host waits for the partials, sums them and sizes the instance buffers
    GSX_HIP_TRY(hipEventRecord(ctx->count_ev, stream), "hipEventRecord(count)");
    GSX_TRY(record(ctx, 1, stream));
    // depth order of the Gaussians, then their tile counts in that order and its scan
    const uint64_t* sorted_depth = ctx->depth_keys.as<uint64_t>();
    if (n > 0) {
        int depth_in_alt = 0;
        GSX_TRY(radix_sort_keys_u64_compacting(ctx->depth_keys.as<uint64_t>(), ctx->depth_keys_alt.as<uint64_t>(), n,
                                               counters, index_bits, depth_end_bit, ctx->depth_sort_temp.ptr,
                                               &depth_in_alt, stream));
        if (depth_in_alt) sorted_depth = ctx->depth_keys_alt.as<uint64_t>();
        hipLaunchKernelGGL(rank_gather_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, stream, n, counters,
                           sorted_depth, (uint64_t)((1ull << index_bits) - 1ull), big_flag, count_shift,
                           (uint32_t)((1ull << count_bits) - 1ull), ctx->tile_count.as<uint32_t>(),
                           ctx->rank_g.as<uint32_t>(), ctx->rank_count.as<uint32_t>(), ctx->g_rank.as<uint32_t>(),
                           long_chunk_of(tiles),
                           ctx->multi_list.as<uint32_t>(), counters + 4, ctx->scan_temp.as<uint32_t>());
        GSX_HIP_TRY(hipGetLastError(), "rank_gather_kernel");
        // exclusive scan of the 256-rank sums; emit_keys_kernel completes the offsets
        GSX_TRY(scan_partials_in_place(ctx->scan_temp.as<uint32_t>(), pre_blocks, stream, 2));
    }
    GSX_TRY(record(ctx, 2, stream));
    GSX_HIP_TRY(hipEventSynchronize(ctx->count_ev), "instance count sync");
    unsigned long long total = 0, big_total = 0, visible_total = 0;
    if (n > 0) {
        const unsigned long long* pre = static_cast<const unsigned long long*>(ctx->kept_parts.host);
        for (unsigned b = 0; b < pre_blocks; ++b) {
            total += pre[b] & ((1ull << kKeptPartBigShift) - 1ull);
            big_total += (pre[b] >> kKeptPartBigShift) & ((1ull << (kKeptPartVisibleShift - kKeptPartBigShift)) - 1ull);
            visible_total += pre[b] >> kKeptPartVisibleShift;
        }
    }
    ctx->visible_count = (int64_t)visible_total;
    if (total > (unsigned long long)UINT32_MAX) {
        // positions, offsets and the sort run in 32 bits; nothing has been emitted yet
        return fail(GSX_HIP_ERROR_OUT_OF_RANGE, "more than 2^32 - 1 (tile, Gaussian) instances");
    }
    const int64_t count = (int64_t)total;
    ctx->instance_count = count;
    const size_t c1 = (size_t)(count > 0 ? count : 1);
    // per instance: its tile (emission order, the sort's input, kept for the backward), the middle
    // pass's tiles and positions, the sorted tiles and positions, its Gaussian
    GSX_TRY(ctx->inst_tile.reserve(c1 * sizeof(uint32_t), "instance_tile", ctx->call_stream));
    GSX_TRY(ctx->tiles_alt.reserve(c1 * sizeof(uint32_t), "tiles_alt", ctx->call_stream));
    GSX_TRY(ctx->tiles_sorted.reserve(c1 * sizeof(uint32_t), "tiles_sorted", ctx->call_stream));
    GSX_TRY(ctx->vals_alt.reserve(c1 * sizeof(uint32_t), "vals_alt", ctx->call_stream));
    GSX_TRY(ctx->vals.reserve(c1 * sizeof(uint32_t), "vals", ctx->call_stream));
    GSX_TRY(ctx->inst_gauss.reserve(c1 * sizeof(uint32_t), "instance_gaussian", ctx->call_stream));
    GSX_TRY(ctx->sorted_g.reserve(c1 * sizeof(uint32_t), "sorted_g", ctx->call_stream));
    GSX_TRY(ctx->sort_temp.reserve(tile_sort_u32_temp_bytes(count), "sort_temp", ctx->call_stream));
    if (train) {
        // bucket checkpoints: at most I/kBucket + tiles + 1 slots of 256 floats
        GSX_TRY(ctx->ckpt.reserve(((size_t)count / kBucket + (size_t)tiles + 2) * 256 * sizeof(float),
                                  "checkpoints", ctx->call_stream));
    }
    if (n > 0) {
        // one wave per big box; rank workgroups up to one rank past the visible ones
        const uint32_t big_blocks = (uint32_t)((big_total + kWavesPerBlock - 1) / kWavesPerBlock);
        const unsigned emit_blocks = std::min(pre_blocks, (unsigned)(visible_total / 256u + 1u));
        hipLaunchKernelGGL(emit_kernel, dim3(big_blocks + emit_blocks), dim3(256), 0, stream, n, ctx->rec.as<float4>(),
                           ctx->rank_g.as<uint32_t>(), ctx->rank_count.as<uint32_t>(), ctx->scan_temp.as<uint32_t>(),
                           ctx->offsets.as<uint32_t>(), cam.tiles_x, ctx->big_list.as<uint32_t>(), big_count,
                           big_blocks, ctx->g_rank.as<uint32_t>(), ctx->inst_gauss.as<uint32_t>(), ctx->inst_tile.as<uint32_t>(),
                           ctx->scan_temp.as<uint32_t>() + pre_blocks + 1, ctx->long_list.as<uint32_t>());
        GSX_HIP_TRY(hipGetLastError(), "emit_kernel");
    }
    GSX_TRY(record(ctx, 3, stream));
    // tile bits in ceil(bits / 8) passes (at least one) of equal digits of 6 to 8 bits (1080p:
    // 13 bits, 2 x 7)
    ctx->sort_passes = std::max(1, (tile_bits + 7) / 8);
    ctx->tile_bits = tile_bits;
    {
        const int digit_bits = std::max(6, (tile_bits + ctx->sort_passes - 1) / ctx->sort_passes);
        GSX_TRY(tile_sort_u32(ctx->inst_tile.as<uint32_t>(), ctx->tiles_alt.as<uint32_t>(),
                              ctx->tiles_sorted.as<uint32_t>(), ctx->vals_alt.as<uint32_t>(), ctx->vals.as<uint32_t>(),
                              count, tile_bits, ctx->sort_passes, digit_bits, ctx->sort_temp.ptr, stream));
        ctx->sorted_vals = ctx->vals.as<uint32_t>();
    }
    GSX_TRY(record(ctx, 4, stream));
    if (count >= kRangesSearchMin) {
        int steps = 0;
        while (((uint64_t)1 << steps) <= (uint64_t)count) ++steps;  // ceil(log2(count + 1))
        hipLaunchKernelGGL(tile_ranges_search_kernel, dim3(blocks_for(tiles, 256)), dim3(256), 0, stream,
                           ctx->tiles_sorted.as<uint32_t>(), (uint32_t)count, (uint32_t)tiles, steps,
                           ctx->ranges.as<uint2>());
    } else if (count > 0) {
        hipLaunchKernelGGL(tile_ranges_kernel, dim3(blocks_for((count + 3) / 4, 256)), dim3(256), 0, stream,
                           ctx->tiles_sorted.as<uint32_t>(), ctx->offsets.as<uint32_t>() + n, (uint32_t)tiles,
                           ctx->ranges.as<uint2>());
    } else {
        hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks_for((int64_t)tiles * 2, 256)), dim3(256), 0, stream,
                           ctx->ranges.as<uint32_t>(), (int64_t)tiles * 2, 0u);
    }
    GSX_HIP_TRY(hipGetLastError(), "tile_ranges_kernel");
    GSX_TRY(record(ctx, 5, stream));
    const int tiles_padded = ((tiles + 7) / 8) * 8;
    hipLaunchKernelGGL(blend_forward_kernel, dim3((unsigned)tiles_padded), dim3(256), 0, stream,
                       ctx->ranges.as<uint2>(), ctx->sorted_vals, ctx->inst_gauss.as<uint32_t>(),
                       ctx->rec.as<float4>(), ctx->rec.as<float4>() + 2 * n,
                       reinterpret_cast<const uint2*>(ctx->rec.as<float4>() + 3 * n),
                       train ? ctx->sorted_g.as<uint32_t>() : nullptr, cam, out_rgb,
                       ctx->final_t.as<float>(),
                       ctx->last.as<uint32_t>(), train ? ctx->ckpt.as<float>() : nullptr);
    GSX_HIP_TRY(hipGetLastError(), "blend_forward_kernel");
    GSX_TRY(record(ctx, 6, stream));
    if (ctx->timing && ctx->cur >= 0) ctx->has_fwd[ctx->cur] = 1;
    ctx->has_train_state = train != 0;
    return GSX_HIP_SUCCESS;
}

}  // extern "C"

namespace {

// The backward's launches for the retained state (inputs validated by the caller).
gsx_hip_status enqueue_backward(gsx_hip_render_context* ctx, const float* grad_rgb,
                                const gsx_hip_gaussian_grads* grads, hipStream_t stream) {
    const int64_t n = ctx->gaussian_count;
    const gsx_hip_gaussians& gs = ctx->gs;
    GSX_TRY(ctx->grad2d.reserve((size_t)(n > 0 ? n : 1) * 9 * sizeof(float), "grad2d", ctx->call_stream));
    GSX_TRY(ctx->inst_grad.reserve((size_t)(ctx->instance_count > 0 ? ctx->instance_count : 1) * 9 * sizeof(float),
                                   "instance_grad", ctx->call_stream));
    const CameraParams& cam = ctx->cam;
    const int32_t tiles = cam.tiles_x * cam.tiles_y;
    GSX_TRY(ctx->tile_cut.reserve((size_t)(tiles > 0 ? tiles : 1) * sizeof(uint32_t), "tile_cut", ctx->call_stream));
    const uint32_t* svals = ctx->sorted_vals;
    const uint32_t* counters = ctx->counters.as<uint32_t>();  // as the forward left them
    // per-instance partials: [I][8] records, then the [I] opacity terms
    float* inst_grad_op = ctx->inst_grad.as<float>() + (size_t)ctx->instance_count * 8;
    const uint32_t long_chunk = long_chunk_of(tiles);
    const unsigned pre_blocks = blocks_for(n, 256);  // the forward's rank workgroups
    GSX_TRY(record(ctx, 7, stream));
    // the gradient sinks, zeroed by the blend backward's workgroups beside their own work (the
    // projection backward then writes only the rows of reached Gaussians)
    SinkZeroing sinks{};
    if (n > 0) {
        float* const fields[8] = {grads->mean3d, grads->rotation, grads->logscale, grads->opacity,
                                  grads->sh0,    grads->sh1,      grads->sh2,      grads->sh3};
        const int widths[8] = {3, 4, 3, 1, 3, 9, 15, 21};
        const int arrays = 5 + (int)gs.sh_degree;
        const int64_t blocks = ((tiles + 7) / 8) * 8;  // the launch below
        const int64_t slices = blocks / arrays;        // workgroups per array (at least 1: blocks >= 8)
        for (int f = 0; f < arrays; ++f) {
            sinks.ptr[f] = fields[f];
            sinks.count[f] = n * widths[f];
            sinks.per[f] = (((sinks.count[f] + slices - 1) / slices) + 3) & ~(int64_t)3;
            if ((reinterpret_cast<uintptr_t>(fields[f]) & 15u) == 0) sinks.vec4 |= 1u << f;
        }
        sinks.arrays = arrays;
    }
    const int tiles_padded = ((tiles + 7) / 8) * 8;
    hipLaunchKernelGGL(blend_backward_kernel, dim3((unsigned)tiles_padded), dim3(256), 0, stream,
                       ctx->ranges.as<uint2>(), svals, ctx->sorted_g.as<uint32_t>(), ctx->rec.as<float4>(),
                       ctx->rec.as<float4>() + 2 * n, reinterpret_cast<const uint2*>(ctx->rec.as<float4>() + 3 * n),
                       ctx->cov_coef.as<float4>(), ctx->ckpt.as<float>(), cam, grad_rgb, ctx->final_t.as<float>(),
                       ctx->last.as<uint32_t>(), ctx->inst_grad.as<float>(), inst_grad_op,
                       ctx->tile_cut.as<uint32_t>(), ctx->touched.as<uint8_t>(), sinks);
    GSX_HIP_TRY(hipGetLastError(), "blend_backward_kernel");
    GSX_TRY(record(ctx, 8, stream));
    if (n > 0) {
        hipLaunchKernelGGL(reduce_instance_grads_kernel,
                           dim3(kLongRunBlocks0 + kLongRunBlocks * (kLongChunks - 1) + blocks_for(n, 256)),
                           dim3(256), 0, stream, n, counters, ctx->offsets.as<uint32_t>(), ctx->rank_g.as<uint32_t>(),
                           ctx->long_list.as<uint32_t>(), ctx->scan_temp.as<uint32_t>() + 2 * (size_t)pre_blocks + 1,
                           ctx->multi_list.as<uint32_t>(), counters + 4, kLongRunBlocks0, kLongRunBlocks, long_chunk,
                           ctx->inst_grad.as<float>(), inst_grad_op, ctx->inst_tile.as<uint32_t>(),
                           ctx->tile_cut.as<uint32_t>(), ctx->touched.as<uint8_t>(), ctx->grad2d.as<float>());
        GSX_HIP_TRY(hipGetLastError(), "reduce_instance_grads_kernel");
    }
    GSX_TRY(record(ctx, 9, stream));
    if (n > 0) {
        const unsigned pblocks = blocks_for(n, 256);
        float* const gi_op = inst_grad_op;
#define GSX_PROJECTION_BACKWARD(D)                                                                              \
    hipLaunchKernelGGL(projection_backward_kernel<D>, dim3(pblocks), dim3(256), 0, stream, n, gs.mean3d, gs.rotation, \
                       gs.logscale, gs.opacity, gs.sh0, gs.sh1, gs.sh2, gs.sh3, cam, ctx->grad2d.as<float>(),        \
                       ctx->tile_count.as<uint32_t>(), ctx->g_rank.as<uint32_t>(), ctx->offsets.as<uint32_t>(),      \
                       long_chunk, ctx->inst_grad.as<float>(), gi_op, ctx->touched.as<uint8_t>(), grads->mean3d,      \
                       grads->rotation, grads->logscale, grads->opacity, grads->sh0, grads->sh1, grads->sh2, grads->sh3, \
                       vector_stores)
        // the 3-float and SH sinks take whole 16-byte vector stores when they are 16-byte aligned
        auto aligned16 = [](const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
        const int vector_stores = aligned16(grads->mean3d) && aligned16(grads->logscale) && aligned16(grads->sh0) &&
                                  (gs.sh_degree < 1 || aligned16(grads->sh1)) &&
                                  (gs.sh_degree < 2 || aligned16(grads->sh2)) &&
                                  (gs.sh_degree < 3 || aligned16(grads->sh3));
        switch (gs.sh_degree) {
            case 0: GSX_PROJECTION_BACKWARD(0); break;
            case 1: GSX_PROJECTION_BACKWARD(1); break;
            case 2: GSX_PROJECTION_BACKWARD(2); break;
            default: GSX_PROJECTION_BACKWARD(3); break;
        }
#undef GSX_PROJECTION_BACKWARD
        GSX_HIP_TRY(hipGetLastError(), "projection_backward_kernel");
    }
    GSX_TRY(record(ctx, 10, stream));
    if (ctx->timing && ctx->cur >= 0) ctx->has_bwd[ctx->cur] = 1;
    return GSX_HIP_SUCCESS;
}

}  // namespace

extern "C" {

gsx_hip_status gsx_hip_render_backward(gsx_hip_render_context* ctx, const float* grad_rgb,
                                       const gsx_hip_gaussian_grads* grads, hipStream_t stream) {
    if (ctx == nullptr || grad_rgb == nullptr || grads == nullptr) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context, grad_rgb and grads must be non-null");
    }
    if (!ctx->has_train_state) {
        return fail(GSX_HIP_ERROR_INVALID_STATE, "backward requires a retained TRAIN forward on the same context");
    }
    const int64_t n = ctx->gaussian_count;
    const gsx_hip_gaussians& gs = ctx->gs;
    if (n > 0 && (grads->mean3d == nullptr || grads->rotation == nullptr || grads->logscale == nullptr ||
                  grads->opacity == nullptr || grads->sh0 == nullptr)) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "gradient sinks mean3d..sh0 must be non-null");
    }
    if ((gs.sh_degree >= 1 && grads->sh1 == nullptr) || (gs.sh_degree >= 2 && grads->sh2 == nullptr) ||
        (gs.sh_degree >= 3 && grads->sh3 == nullptr)) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "sh gradient sinks must be non-null up to sh_degree");
    }
    if ((reinterpret_cast<uintptr_t>(grads->rotation) & 15u) != 0) {
        return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "rotation gradient must be 16-byte aligned");
    }
    ctx->call_stream = stream;
    if (ctx->train_mode == GSX_HIP_FORWARD_TRAIN_BORROW && n > 0) {
        // borrowed state: the gradient is taken at the values the caller's arrays hold now. The
        // comparison with the retained copy runs on check_stream, after everything queued so far
        // on the caller's stream, while the backward is queued on the caller's stream at once, so
        // the GPU does not wait for the host's look at the result; the backward writes only the
        // context's scratch and the sinks, which a refresh overwrites, and reads neither array
        // the comparison reads.
        GSX_TRY(ctx->changed.reserve(sizeof(uint32_t), "train state flag"));
        volatile uint32_t* changed = static_cast<volatile uint32_t*>(ctx->changed.host);
        *changed = 0u;
        StateArrays arrays{};
        for (int f = 0; f < field_count(ctx->live); ++f) {
            arrays.live[f] = field_ptr(ctx->live, f);
            arrays.snap[f] = const_cast<float*>(field_ptr(ctx->gs, f));
            arrays.count[f] = n * kFieldWidth[f];
        }
        GSX_HIP_TRY(hipEventRecord(ctx->fork_ev, stream), "hipEventRecord(fork)");
        GSX_HIP_TRY(hipStreamWaitEvent(ctx->check_stream, ctx->fork_ev, 0), "hipStreamWaitEvent(check)");
        // few workgroups: the comparison needs a fraction of the HBM bandwidth to finish well inside
        // the backward, and leaves the blend kernels their CU slots
        hipLaunchKernelGGL(train_state_kernel, dim3(std::min(state_blocks(n), kCheckBlocks),
                                                    (unsigned)field_count(ctx->live)),
                           dim3(256), 0, ctx->check_stream, arrays, static_cast<uint32_t*>(ctx->changed.dev));
        GSX_HIP_TRY(hipGetLastError(), "train_state_kernel");
        GSX_HIP_TRY(hipEventRecord(ctx->state_ev, ctx->check_stream), "hipEventRecord(state)");
        GSX_TRY(enqueue_backward(ctx, grad_rgb, grads, stream));
        GSX_HIP_TRY(hipEventSynchronize(ctx->state_ev), "train state sync");
        if (*changed != 0u) {
            // the caller changed its arrays: re-run the TRAIN forward on the current values (its
            // image is not returned), then the backward again. The queued backward must finish
            // first: the refresh may regrow the buffers it reads.
            GSX_HIP_TRY(hipStreamSynchronize(stream), "train state refresh sync");
            const bool timing = ctx->timing;
            const gsx_hip_gaussians live = ctx->live;
            const gsx_hip_camera camera = ctx->camera;
            GSX_TRY(ctx->refresh_rgb.reserve((size_t)3 * camera.width * camera.height * sizeof(float),
                                             "refresh image", ctx->call_stream));
            ctx->timing = false;
            const gsx_hip_status st = gsx_hip_render_forward(ctx, &camera, &live, GSX_HIP_FORWARD_TRAIN_BORROW,
                                                             ctx->refresh_rgb.as<float>(), nullptr, stream);
            ctx->timing = timing;
            if (st != GSX_HIP_SUCCESS) return st;
            GSX_TRY(enqueue_backward(ctx, grad_rgb, grads, stream));
        }
    } else {
        GSX_TRY(enqueue_backward(ctx, grad_rgb, grads, stream));
    }
    ctx->has_train_state = false;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_context_get_stats(const gsx_hip_render_context* ctx, gsx_hip_render_stats* out) {
    if (ctx == nullptr || out == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context/out must be non-null");
    out->gaussian_count = ctx->gaussian_count;
    // summed on the host from preprocess's partials when the forward read back its instance count
    out->visible_count = ctx->visible_count;
    out->instance_count = ctx->instance_count;
    out->tile_count = ctx->tile_count_total;
    out->sort_passes = ctx->sort_passes;
    out->depth_sort_passes = ctx->depth_sort_passes;
    out->tile_bits = ctx->tile_bits;
    out->sorted_tile_bytes = (int32_t)sizeof(uint32_t);
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_render_context_get_buffers(const gsx_hip_render_context* ctx, gsx_hip_render_buffers* out) {
    if (ctx == nullptr || out == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "context/out must be non-null");
    out->sorted_tiles = ctx->tiles_sorted.as<uint32_t>();
    out->sorted_values = ctx->sorted_vals;
    out->tile_ranges = ctx->ranges.as<uint32_t>();
    out->records = ctx->rec.as<float>();
    out->tile_counts = ctx->tile_count.as<uint32_t>();
    out->instance_gaussian = ctx->inst_gauss.as<uint32_t>();
    out->final_transmittance = ctx->final_t.as<float>();
    out->last_contributor = ctx->last.as<uint32_t>();
    return GSX_HIP_SUCCESS;
}

}  // extern "C"
