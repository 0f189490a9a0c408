// pool.hip - stream-ordered caching allocator for device memory.
//
// The gsx core reallocates whole Gaussian sets on every density-control commit
// (gsx_gs_resize -> gsx_gs_rebuild_storage, gsx/src/gsx-core.c:2811-2869) and the optimizer
// reallocates its moments with them; the reference CUDA backend pays a cudaMalloc and a
// synchronising cudaFree for each (gsx-cuda/buffer.c). Here a freed block goes back to a per-device
// cache instead, behind an event recorded on the stream it was freed on:
//   - a request is rounded up to a size class (8 classes per power of two, at least 512 bytes:
//     at most 12.5% waste) and served by the smallest cached block of its class or of the next two
//     classes (at most 25% waste in all);
//   - a block reused on the stream it was freed on needs no wait (stream order covers its earlier
//     uses); on another stream, that stream waits on the block's event first;
//   - a request the cache cannot serve calls hipMalloc; if that runs out of memory the cache is
//     released (after a device synchronisation) and the request retried once;
//   - gsx_hip_pool_trim releases every cached block of the current device.
// Freeing never synchronises the host. Counters (gsx_hip_pool_get_stats) show how often the pool
// went to hipMalloc and how often it reused a block.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/gsx_hip.h"

#include <stdio.h>

namespace gsx_amd {
void set_last_error(const char* what);
}  // namespace gsx_amd

namespace {

gsx_hip_status fail(gsx_hip_status code, const char* what) {
    gsx_amd::set_last_error(what);
    return code;
}

gsx_hip_status hip_fail(hipError_t e, const char* what) {
    char msg[256];
    snprintf(msg, sizeof(msg), "%s: %s", what, hipGetErrorString(e));
    gsx_amd::set_last_error(msg);
    return (gsx_hip_status)e;
}

struct Block {
    void* ptr = nullptr;
    size_t size = 0;
    int device = 0;
    hipStream_t stream = nullptr;  // the stream it was last freed on
    hipEvent_t event = nullptr;    // recorded there at that free
};

struct Pool {
    std::mutex mu;
    std::map<int, std::multimap<size_t, Block>> cached;  // device -> size -> free blocks
    std::unordered_map<void*, Block> live;
    std::vector<hipEvent_t> spare_events;
    gsx_hip_pool_stats stats{};
};

Pool& pool() {
    static Pool* p = new Pool();  // process lifetime: never torn down while the runtime exits
    return *p;
}

size_t size_class(size_t bytes) {
    if (bytes < 512) return 512;
    int log2 = 63 - __builtin_clzll((unsigned long long)bytes);
    size_t granule = log2 > 12 ? (size_t)1 << (log2 - 3) : 512;
    return (bytes + granule - 1) / granule * granule;
}

// the next size class above `c`
size_t next_class(size_t c) { return size_class(c + 1); }

// releases every cached block of `device` (caller holds the lock; the device is current)
hipError_t release_cached(Pool& p, int device) {
    auto it = p.cached.find(device);
    if (it == p.cached.end() || it->second.empty()) return hipSuccess;
    hipError_t first = hipDeviceSynchronize();
    for (auto& kv : it->second) {
        hipError_t e = hipFree(kv.second.ptr);
        if (first == hipSuccess) first = e;
        if (kv.second.event != nullptr) p.spare_events.push_back(kv.second.event);
        p.stats.device_releases += 1;
        p.stats.bytes_cached -= kv.second.size;
    }
    it->second.clear();
    return first;
}

}  // namespace

extern "C" {

gsx_hip_status gsx_hip_pool_malloc(void** out_ptr, size_t bytes, hipStream_t stream) {
    if (out_ptr == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_ptr must be non-null");
    *out_ptr = nullptr;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const size_t want = size_class(bytes);
    const size_t limit = next_class(next_class(want));
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    p.stats.requests += 1;
    auto& free_blocks = p.cached[device];
    auto it = free_blocks.lower_bound(want);
    if (it != free_blocks.end() && it->first <= limit) {
        Block b = it->second;
        free_blocks.erase(it);
        p.stats.bytes_cached -= b.size;
        if (b.stream != stream && b.event != nullptr) {
            e = hipStreamWaitEvent(stream, b.event, 0);
            if (e != hipSuccess) {
                free_blocks.emplace(b.size, b);
                p.stats.bytes_cached += b.size;
                return hip_fail(e, "hipStreamWaitEvent (pool block reuse)");
            }
        }
        if (b.event != nullptr) p.spare_events.push_back(b.event);
        b.event = nullptr;
        b.stream = nullptr;
        p.live[b.ptr] = b;
        p.stats.reuses += 1;
        p.stats.bytes_in_use += b.size;
        *out_ptr = b.ptr;
        return GSX_HIP_SUCCESS;
    }
    void* ptr = nullptr;
    e = hipMalloc(&ptr, want);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        hipError_t r = release_cached(p, device);
        if (r != hipSuccess) return hip_fail(r, "releasing cached pool blocks");
        e = hipMalloc(&ptr, want);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return e == hipErrorOutOfMemory ? fail(GSX_HIP_ERROR_OUT_OF_MEMORY, "device allocation failed")
                                        : hip_fail(e, "hipMalloc");
    }
    Block b;
    b.ptr = ptr;
    b.size = want;
    b.device = device;
    p.live[ptr] = b;
    p.stats.device_allocations += 1;
    p.stats.bytes_in_use += want;
    *out_ptr = ptr;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_pool_free(void* ptr, hipStream_t stream) {
    if (ptr == nullptr) return GSX_HIP_SUCCESS;
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    auto it = p.live.find(ptr);
    if (it == p.live.end()) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "pointer was not allocated by the pool");
    Block b = it->second;
    hipEvent_t ev = nullptr;
    if (!p.spare_events.empty()) {
        ev = p.spare_events.back();
        p.spare_events.pop_back();
    } else {
        hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags (pool)");
    }
    hipError_t e = hipEventRecord(ev, stream);
    if (e != hipSuccess) {
        p.spare_events.push_back(ev);
        return hip_fail(e, "hipEventRecord (pool free)");
    }
    p.live.erase(it);
    b.stream = stream;
    b.event = ev;
    p.cached[b.device].emplace(b.size, b);
    p.stats.bytes_in_use -= b.size;
    p.stats.bytes_cached += b.size;
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_pool_trim(void) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    e = release_cached(p, device);
    if (e != hipSuccess) return hip_fail(e, "releasing cached pool blocks");
    return GSX_HIP_SUCCESS;
}

gsx_hip_status gsx_hip_pool_get_stats(gsx_hip_pool_stats* out_stats) {
    if (out_stats == nullptr) return fail(GSX_HIP_ERROR_INVALID_ARGUMENT, "out_stats must be non-null");
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    *out_stats = p.stats;
    return GSX_HIP_SUCCESS;
}

}  // extern "C"
