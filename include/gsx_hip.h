/*
 * gsx_hip.h - C ABI of the gfx950 (MI355X) backend library libgsx_hip.so.
 *
 * This is the layer the gsx backend vtables call (gsx/src/gsx-impl.h:229-533 for the vtables,
 * gsx/src/gsx-cuda/internal.h:274-675 for the launcher layer it replaces): plain device
 * pointers, sizes and a hipStream_t, C linkage, no C++ or framework types. All device work is
 * enqueued on the given stream in order; nothing here synchronises the host except where a
 * function says so. Every call returns 0 on success, a hipError_t value (> 0) for a HIP
 * runtime error, or a negative GSX_HIP_ERROR_* code; gsx_hip_last_error_message() names the
 * failing condition (thread-local, static storage).
 *
 * Conventions shared with gsx (gsx/include/gsx/gsx-render.h:64-140, gsx-base.h:191-216):
 *   Gaussians: mean3d [N,3], rotation [N,4] (xyzw), logscale [N,3], opacity [N] (logit),
 *   sh0 [N,3], sh1 [N,3,3], sh2 [N,5,3], sh3 [N,7,3], all float32 row-major on the device;
 *   images: float32 CHW [3,H,W]; camera: pinhole, world-to-camera pose, +z forward, y down.
 */
#ifndef GSX_HIP_H
#define GSX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef HIP_INCLUDE_HIP_HIP_RUNTIME_API_H
typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;
#endif

typedef int gsx_hip_status;

enum {
    GSX_HIP_SUCCESS = 0,
    GSX_HIP_ERROR_INVALID_ARGUMENT = -1, /* gsx GSX_ERROR_INVALID_ARGUMENT */
    GSX_HIP_ERROR_INVALID_STATE = -2,    /* gsx GSX_ERROR_INVALID_STATE (e.g. backward w/o TRAIN forward) */
    GSX_HIP_ERROR_OUT_OF_RANGE = -3,     /* gsx GSX_ERROR_OUT_OF_RANGE (sizes, gather indices) */
    GSX_HIP_ERROR_OUT_OF_MEMORY = -4,    /* gsx GSX_ERROR_OUT_OF_MEMORY */
    GSX_HIP_ERROR_NOT_SUPPORTED = -5     /* gsx GSX_ERROR_NOT_SUPPORTED */
};

/* Human-readable reason for the last non-zero status returned on this thread. */
const char* gsx_hip_last_error_message(void);

/* ---- device plumbing (replaces the cudaMalloc/cudaMemcpy use of gsx-cuda/buffer.c) -------- */
gsx_hip_status gsx_hip_device_count(int32_t* out_count);
gsx_hip_status gsx_hip_device_name(int32_t device, char* out_name, size_t capacity);
gsx_hip_status gsx_hip_malloc(void** out_ptr, size_t bytes);
gsx_hip_status gsx_hip_free(void* ptr);

/* Stream-ordered caching device allocator (the backend's device buffers, optimizer moments and
 * density-control workspaces; replaces the cudaMalloc / synchronising cudaFree pairs of
 * gsx-cuda/buffer.c and gsx-cuda/optim.c that every gsx_gs_resize commit,
 * gsx/src/gsx-core.c:2811-2869, goes through). A request is rounded up to one of 8 size classes per
 * power of two (at least 512 bytes) and served from cached blocks of its class or the next two
 * when one is free; otherwise hipMalloc (on running out of memory the cache is released and the
 * request retried). pool_free returns a block to the cache behind an event recorded on `stream`
 * (no host synchronisation): reuse on the same stream is ordered by the stream, reuse on another
 * stream waits on that event. Blocks stay cached until gsx_hip_pool_trim (current device; it
 * synchronises the device first) or process exit. Thread-safe. */
typedef struct gsx_hip_pool_stats {
    uint64_t requests;            /* pool_malloc calls */
    uint64_t reuses;              /* requests served from cached blocks */
    uint64_t device_allocations;  /* hipMalloc calls made by the pool */
    uint64_t device_releases;     /* hipFree calls made by the pool (trim, out-of-memory retry) */
    uint64_t bytes_in_use;        /* rounded sizes of the blocks handed out */
    uint64_t bytes_cached;        /* rounded sizes of the cached blocks */
} gsx_hip_pool_stats;
gsx_hip_status gsx_hip_pool_malloc(void** out_ptr, size_t bytes, hipStream_t stream);
gsx_hip_status gsx_hip_pool_free(void* ptr, hipStream_t stream);
gsx_hip_status gsx_hip_pool_trim(void);
gsx_hip_status gsx_hip_pool_get_stats(gsx_hip_pool_stats* out_stats);
gsx_hip_status gsx_hip_memcpy_htod(void* dst, const void* src, size_t bytes);
gsx_hip_status gsx_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
gsx_hip_status gsx_hip_memcpy_dtod_async(void* dst, const void* src, size_t bytes, hipStream_t stream);
/* Ordered copy on `stream` between any two of host, pinned host and device memory (the direction
 * is taken from the pointers, hipMemcpyDefault); gsx-cuda/buffer.c's cudaMemcpyAsync uses. */
gsx_hip_status gsx_hip_memcpy_async(void* dst, const void* src, size_t bytes, hipStream_t stream);
gsx_hip_status gsx_hip_set_device(int32_t device);
gsx_hip_status gsx_hip_device_total_memory(int32_t device, size_t* out_bytes);
/* Page-locked host memory (the HOST_PINNED buffer type) and its device-side address. */
gsx_hip_status gsx_hip_host_alloc(void** out_host, size_t bytes);
gsx_hip_status gsx_hip_host_free(void* host);
gsx_hip_status gsx_hip_host_device_pointer(void* host, void** out_device);
gsx_hip_status gsx_hip_stream_create(hipStream_t* out_stream);
gsx_hip_status gsx_hip_stream_destroy(hipStream_t stream);
gsx_hip_status gsx_hip_stream_synchronize(hipStream_t stream);
/* Events (no timing) ordering work between streams: the async dataloader's helper stream and the
 * major stream (gsx-cuda/async_dl.cu orders them by host synchronisation instead). An event
 * never recorded counts as complete. */
gsx_hip_status gsx_hip_event_create(hipEvent_t* out_event);
gsx_hip_status gsx_hip_event_destroy(hipEvent_t event);
gsx_hip_status gsx_hip_event_record(hipEvent_t event, hipStream_t stream);
gsx_hip_status gsx_hip_event_synchronize(hipEvent_t event);
gsx_hip_status gsx_hip_stream_wait_event(hipStream_t stream, hipEvent_t event);
/* Fill `count` floats with `value` (a kernel, not hipMemset, so it is safe under graph capture). */
gsx_hip_status gsx_hip_fill_f32(float* dst, int64_t count, float value, hipStream_t stream);
/* Streaming device copy of `count` floats (16-byte aligned, count % 4 == 0); also the known-size
 * reference kernel against which HBM traffic counters are calibrated. */
gsx_hip_status gsx_hip_copy_f32(float* dst, const float* src, int64_t count, hipStream_t stream);

/* ---- render ---------------------------------------------------------------------------------
 * Replaces gsx_cuda_fastgs_forward_launch / gsx_cuda_fastgs_backward_launch
 * (gsx/src/gsx-cuda/internal.h:545-630) and the renderer vtable behaviour of the CPU oracle
 * (gsx/src/gsx-cpu/render.c:1254-1975). The render context owns every intermediate buffer
 * (pooled, grow-only; the fastgs resize callbacks and per-forward allocations are gone) and
 * the state a TRAIN forward retains for the backward.
 */
typedef struct gsx_hip_camera {
    float fx, fy, cx, cy;   /* gsx_camera_intrinsics (gsx-base.h:191-205) */
    int32_t width, height;
    float rot[4];           /* gsx_camera_pose.rot, world-to-camera quaternion, xyzw */
    float transl[3];        /* gsx_camera_pose.transl */
    float near_plane, far_plane;
    float background[3];
} gsx_hip_camera;

typedef struct gsx_hip_gaussians {
    int64_t count;
    int32_t sh_degree;      /* 0..3; sh1..sh3 required up to this degree, ignored above */
    const float* mean3d;
    const float* rotation;  /* 16-byte aligned (one float4 per Gaussian); the others 4-byte */
    const float* logscale;
    const float* opacity;
    const float* sh0;
    const float* sh1;
    const float* sh2;
    const float* sh3;
} gsx_hip_gaussians;

typedef struct gsx_hip_gaussian_grads {
    float* mean3d;          /* sinks are overwritten, as gsx-cpu/render.c:1537-1550 */
    float* rotation;        /* 16-byte aligned, as gsx_hip_gaussians.rotation; the others 4-byte */
    float* logscale;
    float* opacity;
    float* sh0;
    float* sh1;
    float* sh2;
    float* sh3;
} gsx_hip_gaussian_grads;

typedef struct gsx_hip_render_context gsx_hip_render_context;

typedef struct gsx_hip_render_stats {
    int64_t gaussian_count;
    int64_t visible_count;   /* Gaussians that pass the projection culls (depth-sorted) in the
                                context's last forward, summed on the host when the forward read
                                back its instance count: get_stats reads no device memory */
    int64_t instance_count;  /* (tile, Gaussian) pairs sorted */
    int32_t tile_count;
    int32_t sort_passes;       /* radix passes over the instance tiles */
    int32_t depth_sort_passes; /* radix passes over the per-Gaussian depth keys */
    /* instances are emitted in (depth, index) order of their Gaussians and their tile indices
     * (tile_bits bits) sorted stably with the emission positions as values, which yields the gsx
     * per-tile (depth, index) order */
    int32_t tile_bits;
    int32_t sorted_tile_bytes; /* element size of sorted_tiles (4) */
} gsx_hip_render_stats;

/* Device pointers of the intermediates a forward retains (valid until the next forward). */
typedef struct gsx_hip_render_buffers {
    const uint32_t* sorted_tiles;  /* [instance_count] tile index of each sorted instance */
    const uint32_t* sorted_values; /* [instance_count] emission position of each sorted instance */
    const uint32_t* tile_ranges;   /* [tile_count][2] start, end */
    const float* records;          /* [N][8] geometry then [N][4] colour+depth blend records */
    const uint32_t* tile_counts;   /* [N] tiles touched per Gaussian (0 = culled) */
    const uint32_t* instance_gaussian; /* [instance_count] Gaussian index of each emission position */
    const float* final_transmittance; /* [H*W] */
    const uint32_t* last_contributor; /* [H*W] exclusive end of the last contributing position */
} gsx_hip_render_buffers;

gsx_hip_status gsx_hip_render_context_create(gsx_hip_render_context** out_context);
gsx_hip_status gsx_hip_render_context_destroy(gsx_hip_render_context* context);

/* Forward types (gsx_render_forward_type and borrow_train_state of gsx_render_forward_request,
 * gsx/include/gsx/gsx-render.h:54-58, 101; semantics of gsx/src/gsx-cpu/render.c:263-380,
 * 1406-1440 and gsx/src/gsx-cuda/render.c:551, 662-756). METRIC is not supported (the CPU
 * backend rejects it too, gsx-cpu/render.c:1126-1154). */
enum {
    GSX_HIP_FORWARD_INFERENCE = 0,    /* image only; no state retained */
    GSX_HIP_FORWARD_TRAIN_BORROW = 1, /* borrow_train_state = true: the backward differentiates at
                                         the values the Gaussian arrays hold when it is called */
    GSX_HIP_FORWARD_TRAIN_CLONE = 2   /* borrow_train_state = false: the backward differentiates at
                                         the values of this forward, whatever the caller changes */
};

/* Forward render into out_rgb [3,H,W]. forward_type is a GSX_HIP_FORWARD_* value. A TRAIN forward
 * retains the state for one backward: it copies the Gaussian fields it reads into the context
 * (56 B per Gaussian at SH degree 0, 236 B at degree 3), and, if visible_counter is non-null,
 * adds 1 to it for every visible Gaussian (gsx-cpu/render.c:980-982). The Gaussian arrays are
 * borrowed for the call. One host synchronisation per forward reads the instance count (the GPU
 * keeps working on the depth order meanwhile); a count above 2^32 - 1 (tile, Gaussian)
 * instances fails with GSX_HIP_ERROR_OUT_OF_RANGE before anything is emitted.
 * Precondition: finite inputs (Gaussian fields, and grad_rgb in the backward). The blend kernels
 * evaluate an entry for the 64 pixels of a wave at once, and a pixel that does not take it adds
 * 0 x its colour (or its gradient term): with finite values that changes nothing, but a
 * non-finite colour or image gradient then turns the other pixels of those waves into NaN as
 * well, where the CPU backend leaves them finite. Every pixel the CPU renders finite and this
 * build renders finite is bit-identical. */
gsx_hip_status gsx_hip_render_forward(gsx_hip_render_context* context, const gsx_hip_camera* camera,
                                      const gsx_hip_gaussians* gaussians, int32_t forward_type, float* out_rgb,
                                      float* visible_counter, hipStream_t stream);

/* Backward of the retained TRAIN forward; consumes the state (a second call fails with
 * GSX_HIP_ERROR_INVALID_STATE, as gsx-cpu/render.c:1406-1408, 1973). After a TRAIN_BORROW forward
 * it first compares the caller's Gaussian arrays with the retained copy (one read of both and one
 * host synchronisation) and, if any bit changed, re-runs the forward on the current values before
 * differentiating (the reference CUDA backend re-runs it unconditionally,
 * gsx-cuda/render.c:1451). */
gsx_hip_status gsx_hip_render_backward(gsx_hip_render_context* context, const float* grad_rgb,
                                       const gsx_hip_gaussian_grads* grads, hipStream_t stream);

gsx_hip_status gsx_hip_render_context_get_stats(const gsx_hip_render_context* context,
                                                gsx_hip_render_stats* out_stats);
gsx_hip_status gsx_hip_render_context_get_buffers(const gsx_hip_render_context* context,
                                                  gsx_hip_render_buffers* out_buffers);

/* Per-stage device timing: set_timing(capacity > 0) allocates a ring of `capacity` HIP event
 * sets; each forward (and the following backward) records one set on its launch stream, so a
 * timed loop pays no synchronisation. get_timings synchronises on the recorded events and writes
 * the per-stage average over the recorded sets, in milliseconds, in this order: preprocess,
 * depth_order (depth-key sort, tile counts in depth order, their scan and the instance-count
 * readback), emit, sort, ranges, blend_forward, blend_backward, instance_reduce,
 * projection_backward. set_timing(0) disables timing. */
enum { GSX_HIP_RENDER_STAGE_COUNT = 9 };
gsx_hip_status gsx_hip_render_context_set_timing(gsx_hip_render_context* context, int32_t capacity);
gsx_hip_status gsx_hip_render_context_get_timings(gsx_hip_render_context* context, float* out_ms, int32_t capacity,
                                                  int32_t* out_written);

/* ---- sort / scan ------------------------------------------------------------------------------
 * Replace cub::DeviceScan::ExclusiveSum (fastgs/forward.cu:180-185) and
 * cub::DeviceRadixSort::SortPairs (fastgs/forward.cu:155-161, 214-220). */
size_t gsx_hip_scan_temp_bytes(int64_t n);
gsx_hip_status gsx_hip_scan_exclusive_u32(const uint32_t* in, uint32_t* out, int64_t n, void* temp,
                                          hipStream_t stream);
/* The exclusive scan above without allocation or workspace, for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc); it has no
 * counterpart in the reference. The partial sums live in a static device array of 256 KiB per
 * GPU (held until the process ends), so n may be at most 67,108,864 (2^26) elements; larger n
 * fails with GSX_HIP_ERROR_OUT_OF_RANGE. Every call on one GPU uses that GPU's array: calls that
 * overlap on one GPU (different streams or host threads) race and must be serialised by the
 * caller. Nothing needs clearing between calls (every partial is written before it is read). */
gsx_hip_status gsx_hip_scan_exclusive_u32_noalloc(const uint32_t* in, uint32_t* out, int64_t n, hipStream_t stream);
size_t gsx_hip_radix_sort_temp_bytes(int64_t n);
/* Stable LSD sort of (key, value) pairs on key bits [begin_bit, end_bit), 8 bits per pass. */
gsx_hip_status gsx_hip_radix_sort_pairs_u64(uint64_t* keys, uint32_t* values, uint64_t* keys_alt,
                                            uint32_t* values_alt, int64_t n, int begin_bit, int end_bit, void* temp,
                                            int* out_result_in_alt, hipStream_t stream);
/* Stable LSD sort of keys alone on bits [begin_bit, end_bit); the other bits travel with the key
 * (the render path packs the emission position below begin_bit). No counterpart in the CUDA
 * backend, which always sorts pairs. */
gsx_hip_status gsx_hip_radix_sort_keys_u64(uint64_t* keys, uint64_t* keys_alt, int64_t n, int begin_bit,
                                           int end_bit, void* temp, int* out_result_in_alt, hipStream_t stream);

/* ---- tensor operations -------------------------------------------------------------------------
 * The element-wise, random, reduce and image-conversion entries of gsx_backend_buffer_i
 * (gsx/src/gsx-impl.h:302-458) that the CUDA backend implements in gsx-cuda/buffer.c and
 * reduce-kernels.cu; semantics of the CPU backend (gsx/src/gsx-cpu/core.c:874-2019). Pointers are
 * device pointers; nothing here synchronises except where stated. */
enum { GSX_HIP_DTYPE_F32 = 0, GSX_HIP_DTYPE_U8 = 1, GSX_HIP_DTYPE_I32 = 2 };
enum {                                   /* gsx_impl_unary_op (gsx-impl.h:295-300) */
    GSX_HIP_UNARY_EXP = 0,
    GSX_HIP_UNARY_SIGMOID = 1,
    GSX_HIP_UNARY_SIGMOID_DERIVATIVE = 2,
    GSX_HIP_UNARY_ABS = 3
};
enum {                                   /* gsx_impl_unary/binary_reduce_op (gsx-impl.h:234-243) */
    GSX_HIP_REDUCE_SUM = 0,
    GSX_HIP_REDUCE_MEAN = 1,
    GSX_HIP_REDUCE_MAX = 2,
    GSX_HIP_REDUCE_MSE = 3,
    GSX_HIP_REDUCE_MAE = 4
};
/* Repeat a pattern of 1..64 bytes over `bytes` (memset_tensor / fill_tensor / set_zero). */
gsx_hip_status gsx_hip_fill_pattern(void* dst, size_t bytes, const void* pattern, size_t pattern_bytes,
                                    hipStream_t stream);
/* Element i = pcg32_next_float of draw i of the (state, inc) stream (fill_rand_tensor). */
gsx_hip_status gsx_hip_fill_rand_f32(float* dst, int64_t count, uint64_t state, uint64_t inc, hipStream_t stream);
/* Box-Muller pairs from draws 2k, 2k+1, times sigma (fill_randn_tensor); logf / cosf / sinf are
 * glibc's, bit for bit, so the fill equals the CPU backend's. */
gsx_hip_status gsx_hip_fill_randn_f32(float* dst, int64_t count, uint64_t state, uint64_t inc, float sigma,
                                      hipStream_t stream);
/* fill_randint_tensor: element i = the i-th draw that pcg32_next_uint_bound accepts, mod bound,
 * for u8 (element_bytes 1) or i32 (4) elements. `draws` >= count draws are examined (temp of
 * gsx_hip_fill_randint_temp_bytes(draws)); when out_accepted is non-null the call synchronises
 * the stream and stores how many were accepted (fewer than count: call again with more draws). */
size_t gsx_hip_fill_randint_temp_bytes(int64_t draws);
gsx_hip_status gsx_hip_fill_randint(void* dst, int64_t count, int32_t element_bytes, uint64_t state, uint64_t inc,
                                    uint32_t bound, int64_t draws, void* temp, int64_t* out_accepted,
                                    hipStream_t stream);
/* multinomial_tensor: sample i from draw i and the (non-decreasing, positive-ended) cdf. */
gsx_hip_status gsx_hip_multinomial_i32(int32_t* out, int64_t samples, const float* cdf, int64_t categories,
                                       uint64_t state, uint64_t inc, hipStream_t stream);
/* check_finite_tensor: sets *flag (a device word the caller cleared) to 1 on any inf or NaN. */
gsx_hip_status gsx_hip_check_finite_f32(const float* x, int64_t count, uint32_t* flag, hipStream_t stream);
/* unary_tensor / unary_tensor_inplace (x may equal out); exp through the glibc-exact expf. */
gsx_hip_status gsx_hip_unary_f32(const float* x, float* out, int64_t count, int32_t op, hipStream_t stream);
/* clamp_inplace_tensor for GSX_HIP_DTYPE_*; lo and hi are host pointers to one element. */
gsx_hip_status gsx_hip_clamp_inplace(void* x, int64_t count, int32_t data_type, const void* lo, const void* hi,
                                     hipStream_t stream);
/* unary_reduce_tensor (sum, mean, max over rows of `reduce` elements of x) and
 * binary_reduce_tensor (mse, mae of x - y); out[outer]. Sums run in double in a fixed order;
 * max keeps the CPU's first-occurrence and NaN rules. temp: gsx_hip_reduce_temp_bytes. */
size_t gsx_hip_reduce_temp_bytes(int64_t outer, int64_t reduce);
gsx_hip_status gsx_hip_reduce_f32(const float* x, const float* y, int64_t outer, int64_t reduce, int32_t op,
                                  float* out, void* temp, hipStream_t stream);
/* The dataloader's device layout step (replaces the HWC -> CHW kernels of
 * gsx/src/gsx-cuda/async_dl.cu:45-156): dst [channels, height, width] float32 from a tightly
 * packed HWC (channels 3) or HW (channels 1) payload of u8 (src_is_u8 != 0, values kept, not
 * scaled) or float32 already in device-visible memory. */
gsx_hip_status gsx_hip_dataloader_to_chw_f32(const void* src, int32_t src_is_u8, int64_t channels, int64_t height,
                                            int64_t width, float* dst, hipStream_t stream);
/* image_convert_colorspace (sRGB transfer curves with glibc's powf, bit for bit),
 * image_convert_storage_format (HWC <-> CHW for 1/2/4-byte elements) and
 * image_convert_data_type (f32 <-> u8), gsx/src/extra/gsx-image-impl.h:9-170. */
gsx_hip_status gsx_hip_image_colorspace_f32(const float* src, float* dst, int64_t count, int32_t src_srgb,
                                            int32_t dst_srgb, hipStream_t stream);
gsx_hip_status gsx_hip_image_storage_convert(const void* src, int32_t src_hwc, void* dst, int32_t dst_hwc,
                                             int64_t channels, int64_t height, int64_t width, int32_t element_bytes,
                                             hipStream_t stream);
gsx_hip_status gsx_hip_image_quantize_u8(const float* src, uint8_t* dst, int64_t count, hipStream_t stream);
gsx_hip_status gsx_hip_image_dequantize_u8(const uint8_t* src, float* dst, int64_t count, hipStream_t stream);

/* ---- losses -----------------------------------------------------------------------------------
 * Replace gsx_cuda_loss_*_kernel_launch (gsx/src/gsx-cuda/internal.h:312-369, CHW forms); semantics of
 * gsx/src/gsx-cpu/loss.c:316-709 (accumulate into loss_map / grad_prediction; grad_scale is
 * already normalised as gsx_loss_scale_grad, gsx-tensor-helpers.h:236-244). */
gsx_hip_status gsx_hip_loss_l1_f32_forward_kernel_launch(float* loss_map, const float* prediction,
                                                         const float* target, int64_t total_elements, float scale,
                                                         hipStream_t stream);
gsx_hip_status gsx_hip_loss_l1_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                          const float* target, int64_t total_elements,
                                                          float grad_scale, hipStream_t stream);
gsx_hip_status gsx_hip_loss_mse_f32_forward_kernel_launch(float* loss_map, const float* prediction,
                                                          const float* target, int64_t total_elements, float scale,
                                                          hipStream_t stream);
gsx_hip_status gsx_hip_loss_mse_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                           const float* target, int64_t total_elements,
                                                           float grad_scale, hipStream_t stream);
/* SSIM on [outer, channels, H, W] CHW images; ssim_workspace = 3 * outer*channels*H*W floats
 * written by the forward and read by the backward. fuse_l1 != 0 also applies an L1 term of
 * l1_scale (forward) / l1_grad_scale (backward) first, bit-identical to calling the L1
 * launcher before. These are not drop-in replacements of gsx_cuda_loss_ssim_* (gsx-cuda/
 * internal.h:346-369): those take two buffers (ssim_buffer_a/b) and no L1 term; here one
 * workspace holds the three window moments the backward needs. The gsx loss vtable of this
 * library (gsx_amd/plugin/hip_loss.c) owns that workspace per loss context. Limits: at most 65535
 * planes (outer_count * channels) and height * width <= UINT32_MAX, else
 * GSX_HIP_ERROR_OUT_OF_RANGE. */
gsx_hip_status gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(float* loss_map, const float* prediction,
                                                               const float* target, int64_t outer_count,
                                                               int32_t channels, int32_t height, int32_t width,
                                                               float scale, float* ssim_workspace, float l1_scale,
                                                               int fuse_l1, hipStream_t stream);
gsx_hip_status gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(float* grad_prediction, const float* prediction,
                                                                const float* target, int64_t outer_count,
                                                                int32_t channels, int32_t height, int32_t width,
                                                                float grad_scale, const float* ssim_workspace,
                                                                float l1_grad_scale, int fuse_l1,
                                                                hipStream_t stream);

/* ---- optimizer --------------------------------------------------------------------------------
 * Adam, element arithmetic of gsx/src/gsx-cpu/optim.c:712-780; bias corrections
 * 1 - beta^step are computed by the caller in float64 (as the CPU does with pow). */
#define GSX_HIP_ADAM_MAX_GROUPS 16
typedef struct gsx_hip_adam_group {
    float* parameter;
    const float* gradient;
    float* first_moment;
    float* second_moment;
    int64_t count;
    float beta1, beta2, learning_rate, weight_decay, epsilon, max_grad;
    double bias_correction1, bias_correction2;
} gsx_hip_adam_group;

/* Counterpart of gsx_cuda_adam_step_f32_kernel_launch (gsx/src/gsx-cuda/internal.h:296-311),
 * with one difference in the contract: this launcher takes the bias corrections themselves,
 * 1 - beta^step in float64, and divides the moments by them as the CPU backend does
 * (gsx-cpu/optim.c:740-757); the CUDA vtable passes their float inverses instead
 * (gsx-cuda/optim.c:792-793), so a caller ported from there must not pass inverses. The gsx
 * vtable of this library (gsx_amd/plugin/hip_optim.c) calls the multi-group launcher below. */
gsx_hip_status gsx_hip_adam_step_f32_kernel_launch(float* parameter, const float* gradient, float* first_moment,
                                                   float* second_moment, int64_t total_elements, float beta1,
                                                   float beta2, float learning_rate, float weight_decay,
                                                   float epsilon, float max_grad, double bias_correction1,
                                                   double bias_correction2, hipStream_t stream);
/* All groups of one optimizer step in a single launch (the CUDA backend issues one launch
 * per group, gsx/src/gsx-cuda/optim.c:757-796). Above 256 MiB of traffic (28 bytes per element
 * over all groups) the launch reads and writes with non-temporal accesses; the results are the
 * same bits either way. */
gsx_hip_status gsx_hip_adam_step_multi_launch(const gsx_hip_adam_group* groups, int32_t group_count,
                                              hipStream_t stream);

/* ---- adaptive density control -----------------------------------------------------------------
 * Replaces the CUDA thrust pipeline (gsx/src/gsx-cuda/adc.cu:757-927) with the semantics of
 * the CPU default/ABSGS refine and opacity reset (gsx/src/gsx-cpu/adc/default.c:160-527,
 * gsx/src/gsx-cpu/adc.c:48-80, 380-559): identical grow/split/prune decisions, row order and
 * rows (the split normals use glibc's logf / cosf bit for bit); split k draws the CPU's pcg32
 * stream advanced by 12 * k draws. */
#define GSX_HIP_ADC_MAX_FIELDS 16
typedef struct gsx_hip_adc_params {
    int32_t algorithm; /* 0 GSX_ADC_ALGORITHM_DEFAULT, 1 GSX_ADC_ALGORITHM_ABSGS */
    float pruning_opacity_threshold;
    float opacity_clamp_value;
    float max_world_scale;
    float max_screen_scale;
    float duplicate_grad_threshold;
    float duplicate_scale_threshold;
    float duplicate_absgrad_threshold;
    float scene_scale;
    int64_t refine_every, start_refine, end_refine, max_num_gaussians, reset_every;
    /* GSX_ADC_ALGORITHM_MCMC (algorithm 2): position noise scale, target growth ratio per
     * refine, and the optimizer's current mean3d learning rate (the noise is scaled by it) */
    float noise_strength;
    float grow_ratio;
    float mean3d_learning_rate;
} gsx_hip_adc_params;

/* Rows of a Gaussian set on the device (the gsx_gs fields, gsx/include/gsx/gsx-core.h:286-308)
 * plus the Adam moments of each parameter field, all nullable except mean3d..sh0. Moment index
 * k follows the field order mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3. */
typedef struct gsx_hip_gs_rows {
    int64_t count;
    int32_t sh_degree;
    float *mean3d, *rotation, *logscale, *opacity, *sh0, *sh1, *sh2, *sh3;
    float *grad_acc, *absgrad_acc, *visible_counter, *max_screen_radius;
    float *first_moment[8];
    float *second_moment[8];
} gsx_hip_gs_rows;

typedef struct gsx_hip_adc_context gsx_hip_adc_context;
/* The context owns the split RNG (pcg32 seeded (seed, seed), gsx/src/gsx-cpu/adc.c:466) and
 * the scratch buffers; the RNG advances across steps like the CPU adc object's. */
gsx_hip_status gsx_hip_adc_context_create(gsx_hip_adc_context** out_context, uint64_t seed);
gsx_hip_status gsx_hip_adc_context_destroy(gsx_hip_adc_context* context);
/* One gsx_adc_step at global_step. Growth appends rows in place, so every buffer of `rows` needs
 * `capacity` >= count + (max_num_gaussians - count) rows; when rows are pruned the compacted set
 * is written to `out` (same fields bound) and *out_result_in_out = 1, otherwise the result stays
 * in `rows`. The final count is stored in the result's `count`. out_counts[4] = pruned,
 * duplicated, grown (split), reset, as gsx_adc_result. Synchronises the stream twice per refine
 * (candidate and survivor counts).
 * MCMC (algorithm 2, gsx/src/gsx-cpu/adc/mcmc.c:345-766, dispatched as gsx-cpu/adc.c:515-547):
 * every step before end_refine moves each mean3d by opacity-gated noise shaped by its covariance
 * (6 draws per Gaussian); a refine relocates the rows whose sigmoid(opacity) <= the pruning
 * threshold onto live rows drawn in proportion to opacity and grows the set to
 * min(floor(count * (1 + grow_ratio)), max_num_gaussians) rows drawn the same way (appended in
 * place: `capacity` >= that count), with the opacity / scale correction of the relocated sources.
 * Rows are never removed, so the result stays in `rows`; out_counts = relocated (as pruned), 0,
 * relocated + appended (as grown), reset. The draw weights form their cumulative sums in float
 * on the host, in index order, as the CPU and Metal backends do (a sequential float sum has no
 * parallel equivalent with the same rounding); the stream synchronises twice per draw. */
gsx_hip_status gsx_hip_adc_step(gsx_hip_adc_context* context, const gsx_hip_adc_params* params, uint64_t global_step,
                                gsx_hip_gs_rows* rows, int64_t capacity, gsx_hip_gs_rows* out,
                                int32_t* out_result_in_out, int64_t* out_counts, hipStream_t stream);

/* Replaces gsx_cuda_gather_rows_kernel_launch (gsx/src/gsx-cuda/internal.h:396-405): out row r
 * = src row src_indices[r]; an index outside [0, src_row_count) sets *out_has_out_of_range
 * (a device int, may be null; the CPU returns GSX_ERROR_OUT_OF_RANGE, gsx-cpu/core.c:1322-1324).
 * No host synchronisation. */
gsx_hip_status gsx_hip_gather_rows_kernel_launch(const void* src, void* dst, int64_t row_bytes, int64_t row_count,
                                                 const int32_t* src_indices, int64_t src_row_count,
                                                 int* out_has_out_of_range, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GSX_HIP_H */
