/*
 * hip_backend.c - provider, backend, buffer-type and buffer vtables of the gsx HIP backend
 * (gsx/src/gsx-impl.h:229-458). Counterparts: gsx/src/gsx-cuda/backend.c, gsx-cuda/buffer.c,
 * with the CPU backend's operation semantics (gsx/src/gsx-cpu/core.c); every operation is queued
 * on the backend's major stream through libgsx_hip.so.
 */
#include "hip_backend.h"

#include <stdlib.h>
#include <string.h>

/* ---- errors ---------------------------------------------------------------------------------- */

gsx_error gsx_hip_plugin_error(gsx_hip_status status, const char *what)
{
    switch(status) {
    case GSX_HIP_SUCCESS:
        return gsx_make_error(GSX_ERROR_SUCCESS, NULL);
    case GSX_HIP_ERROR_INVALID_ARGUMENT:
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, what);
    case GSX_HIP_ERROR_INVALID_STATE:
        return gsx_make_error(GSX_ERROR_INVALID_STATE, what);
    case GSX_HIP_ERROR_OUT_OF_RANGE:
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, what);
    case GSX_HIP_ERROR_OUT_OF_MEMORY:
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, what);
    case GSX_HIP_ERROR_NOT_SUPPORTED:
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, what);
    case 2: /* hipErrorOutOfMemory */
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, what);
    default:
        return gsx_make_error(GSX_ERROR_UNKNOWN, what);
    }
}

#define HIP_TRY(expr, what)                                         \
    do {                                                            \
        gsx_hip_status st_ = (expr);                                \
        if(st_ != GSX_HIP_SUCCESS) return gsx_hip_plugin_error(st_, (what)); \
    } while(0)

#define GSX_TRY(expr)                                               \
    do {                                                            \
        gsx_error e_ = (expr);                                      \
        if(!gsx_error_is_success(e_)) return e_;                    \
    } while(0)

static gsx_error ok(void) { return gsx_make_error(GSX_ERROR_SUCCESS, NULL); }

/* ---- provider and devices -------------------------------------------------------------------- */

static gsx_error hip_discover_devices(gsx_backend_provider_t provider, gsx_builtin_registry_state *registry);
static gsx_error hip_create_backend(gsx_backend_device_t device, const gsx_backend_desc *desc, gsx_backend_t *out);

static const gsx_backend_provider_i hip_provider_iface = { hip_discover_devices, hip_create_backend };

#define HIP_MAX_DEVICES 64
static struct gsx_backend_provider hip_provider = { 0 };
static gsx_hip_plugin_device hip_devices[HIP_MAX_DEVICES];
static int32_t hip_device_count = 0;

static gsx_error hip_discover_devices(gsx_backend_provider_t provider, gsx_builtin_registry_state *registry)
{
    int32_t count = 0;
    int32_t i = 0;

    if(gsx_hip_device_count(&count) != GSX_HIP_SUCCESS || count <= 0) {
        hip_device_count = 0;
        return ok();
    }
    if(count > HIP_MAX_DEVICES) {
        count = HIP_MAX_DEVICES;
    }
    hip_device_count = 0;
    for(i = 0; i < count; ++i) {
        gsx_hip_plugin_device *dev = &hip_devices[hip_device_count];
        size_t total = 0;

        memset(dev, 0, sizeof(*dev));
        if(gsx_hip_device_name(i, dev->name, sizeof(dev->name)) != GSX_HIP_SUCCESS) {
            continue;
        }
        (void)gsx_hip_device_total_memory(i, &total);
        dev->base.provider = provider;
        dev->base.info.backend_type = GSX_HIP_BACKEND_TYPE;
        dev->base.info.backend_name = GSX_HIP_BACKEND_NAME;
        dev->base.info.device_index = hip_device_count;
        dev->base.info.name = dev->name;
        dev->base.info.total_memory_bytes = (gsx_size_t)total;
        dev->ordinal = i;
        GSX_TRY(gsx_builtin_registry_append_device(registry, &dev->base));
        hip_device_count += 1;
    }
    return ok();
}

gsx_error gsx_hip_backend_provider_bootstrap(gsx_builtin_registry_state *registry)
{
    int32_t count = 0;

    if(registry == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "registry must be non-null");
    }
    if(gsx_hip_device_count(&count) != GSX_HIP_SUCCESS || count <= 0) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "no HIP devices available");
    }
    hip_provider.iface = &hip_provider_iface;
    hip_provider.backend_type = GSX_HIP_BACKEND_TYPE;
    hip_provider.backend_name = GSX_HIP_BACKEND_NAME;
    GSX_TRY(hip_provider.iface->discover_devices(&hip_provider, registry));
    return gsx_builtin_registry_append_provider(registry, &hip_provider);
}

/* ---- backend ----------------------------------------------------------------------------------- */

static gsx_error hip_backend_free(gsx_backend_t backend);
static gsx_error hip_backend_get_info(gsx_backend_t backend, gsx_backend_info *out_info);
static gsx_error hip_backend_get_capabilities(gsx_backend_t backend, gsx_backend_capabilities *out);
static gsx_error hip_backend_get_major_stream(gsx_backend_t backend, void **out_stream);
static gsx_error hip_backend_major_stream_sync(gsx_backend_t backend);
static gsx_error hip_backend_count_buffer_types(gsx_backend_t backend, gsx_index_t *out_count);
static gsx_error hip_backend_get_buffer_type(gsx_backend_t backend, gsx_index_t index, gsx_backend_buffer_type_t *out);
static gsx_error hip_backend_find_buffer_type(gsx_backend_t backend, gsx_backend_buffer_type_class type,
    gsx_backend_buffer_type_t *out);
static gsx_error hip_query_unary_reduce_workspace(gsx_backend_t backend, gsx_backend_buffer_type_class ws_type,
    gsx_data_type data_type, gsx_index_t x_rank, const gsx_index_t *x_shape, gsx_index_t out_rank,
    const gsx_index_t *out_shape, gsx_index_t start_axis, gsx_impl_unary_reduce_op op, gsx_size_t *out_bytes,
    gsx_size_t *out_alignment);
static gsx_error hip_query_binary_reduce_workspace(gsx_backend_t backend, gsx_backend_buffer_type_class ws_type,
    gsx_data_type data_type, gsx_index_t lhs_rank, const gsx_index_t *lhs_shape, gsx_index_t rhs_rank,
    const gsx_index_t *rhs_shape, gsx_index_t out_rank, const gsx_index_t *out_shape, gsx_index_t start_axis,
    gsx_impl_binary_reduce_op op, gsx_size_t *out_bytes, gsx_size_t *out_alignment);

static const gsx_backend_i hip_backend_iface = {
    hip_backend_free,
    hip_backend_get_info,
    hip_backend_get_capabilities,
    hip_backend_get_major_stream,
    hip_backend_major_stream_sync,
    hip_backend_count_buffer_types,
    hip_backend_get_buffer_type,
    hip_backend_find_buffer_type,
    hip_query_unary_reduce_workspace,
    hip_query_binary_reduce_workspace,
    gsx_hip_plugin_create_renderer,
    gsx_hip_plugin_create_loss,
    gsx_hip_plugin_create_optim,
    gsx_hip_plugin_create_adc,
    gsx_hip_plugin_create_async_dl
};

static const gsx_backend_buffer_type_i hip_buffer_type_iface;

static void hip_init_buffer_type(gsx_hip_plugin_backend *b, gsx_hip_plugin_buffer_type *t,
    gsx_backend_buffer_type_class type, const char *name, gsx_size_t alignment)
{
    memset(t, 0, sizeof(*t));
    t->base.iface = &hip_buffer_type_iface;
    t->base.backend = &b->base;
    t->base.live_arena_count = 0;
    t->info.backend = &b->base;
    t->info.type = type;
    t->info.name = name;
    t->info.alignment_bytes = alignment;
    t->info.max_allocation_size_bytes = 0;
}

static gsx_error hip_create_backend(gsx_backend_device_t device, const gsx_backend_desc *desc, gsx_backend_t *out)
{
    gsx_hip_plugin_device *dev = (gsx_hip_plugin_device *)device;
    gsx_hip_plugin_backend *b = NULL;
    gsx_hip_status st = GSX_HIP_SUCCESS;

    if(desc == NULL || out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "desc and out_backend must be non-null");
    }
    if(desc->options_size_bytes != 0 && desc->options == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "non-zero options_size_bytes requires a non-null options pointer");
    }
    if(desc->options != NULL || desc->options_size_bytes != 0) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip backend has no backend-specific options");
    }
    *out = NULL;
    b = (gsx_hip_plugin_backend *)calloc(1, sizeof(*b));
    if(b == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip backend");
    }
    b->base.iface = &hip_backend_iface;
    b->base.provider = &hip_provider;
    b->base.device = device;
    b->ordinal = dev->ordinal;
    st = gsx_hip_set_device(dev->ordinal);
    if(st == GSX_HIP_SUCCESS) st = gsx_hip_stream_create(&b->stream);
    if(st == GSX_HIP_SUCCESS) st = gsx_hip_malloc((void **)&b->flag, sizeof(uint32_t));
    if(st == GSX_HIP_SUCCESS) st = gsx_hip_host_alloc((void **)&b->flag_host, sizeof(uint32_t));
    if(st != GSX_HIP_SUCCESS) {
        if(b->stream != NULL) (void)gsx_hip_stream_destroy(b->stream);
        if(b->flag != NULL) (void)gsx_hip_free(b->flag);
        if(b->flag_host != NULL) (void)gsx_hip_host_free(b->flag_host);
        free(b);
        return gsx_hip_plugin_error(st, "hip backend creation failed");
    }
    b->capabilities.supported_data_types = GSX_DATA_TYPE_FLAG_F32;
    b->capabilities.supports_async_prefetch = true;
    hip_init_buffer_type(b, &b->device_type, GSX_BACKEND_BUFFER_TYPE_DEVICE, "device", 256);
    hip_init_buffer_type(b, &b->pinned_type, GSX_BACKEND_BUFFER_TYPE_HOST_PINNED, "host_pinned", 64);
    *out = &b->base;
    return ok();
}

static gsx_error hip_backend_free(gsx_backend_t backend)
{
    gsx_hip_plugin_backend *b = gsx_hip_plugin_backend_of(backend);

    if(backend == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "backend must be non-null");
    }
    if(b->base.live_buffer_count > 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "backend has live buffers");
    }
    if(b->base.live_arena_count > 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "backend has live arenas");
    }
    if(b->base.live_renderer_count > 0 || b->base.live_loss_count > 0 || b->base.live_optim_count > 0
        || b->base.live_adc_count > 0 || b->base.live_async_dl_count > 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE,
            "backend has live renderers, losses, optimizers, adcs, or async dataloaders");
    }
    (void)gsx_hip_stream_synchronize(b->stream);
    (void)gsx_hip_stream_destroy(b->stream);
    (void)gsx_hip_free(b->flag);
    (void)gsx_hip_host_free(b->flag_host);
    free(b);
    return ok();
}

static gsx_error hip_backend_get_info(gsx_backend_t backend, gsx_backend_info *out_info)
{
    if(out_info == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_info must be non-null");
    }
    out_info->backend_type = GSX_HIP_BACKEND_TYPE;
    out_info->device = backend->device;
    return ok();
}

static gsx_error hip_backend_get_capabilities(gsx_backend_t backend, gsx_backend_capabilities *out)
{
    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_capabilities must be non-null");
    }
    *out = gsx_hip_plugin_backend_of(backend)->capabilities;
    return ok();
}

static gsx_error hip_backend_get_major_stream(gsx_backend_t backend, void **out_stream)
{
    if(out_stream == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_stream must be non-null");
    }
    *out_stream = (void *)gsx_hip_plugin_stream(backend);
    return ok();
}

static gsx_error hip_backend_major_stream_sync(gsx_backend_t backend)
{
    HIP_TRY(gsx_hip_stream_synchronize(gsx_hip_plugin_stream(backend)), "hipStreamSynchronize failed");
    return ok();
}

static gsx_error hip_backend_count_buffer_types(gsx_backend_t backend, gsx_index_t *out_count)
{
    (void)backend;
    if(out_count == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_count must be non-null");
    }
    *out_count = 2;
    return ok();
}

static gsx_error hip_backend_get_buffer_type(gsx_backend_t backend, gsx_index_t index, gsx_backend_buffer_type_t *out)
{
    gsx_hip_plugin_backend *b = gsx_hip_plugin_backend_of(backend);

    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_buffer_type must be non-null");
    }
    if(index < 0 || index >= 2) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "buffer type index out of range");
    }
    *out = index == 0 ? &b->device_type.base : &b->pinned_type.base;
    return ok();
}

static gsx_error hip_backend_find_buffer_type(gsx_backend_t backend, gsx_backend_buffer_type_class type,
    gsx_backend_buffer_type_t *out)
{
    gsx_hip_plugin_backend *b = gsx_hip_plugin_backend_of(backend);

    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_buffer_type must be non-null");
    }
    switch(type) {
    case GSX_BACKEND_BUFFER_TYPE_DEVICE:
        *out = &b->device_type.base;
        return ok();
    case GSX_BACKEND_BUFFER_TYPE_HOST_PINNED:
        *out = &b->pinned_type.base;
        return ok();
    case GSX_BACKEND_BUFFER_TYPE_HOST:
    case GSX_BACKEND_BUFFER_TYPE_UNIFIED:
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "buffer type not supported by the hip backend");
    }
    return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "invalid buffer type class");
}

/* rows before start_axis x elements from start_axis on */
static gsx_error hip_reduce_extents(gsx_index_t rank, const gsx_index_t *shape, gsx_index_t start_axis,
    gsx_size_t *out_outer, gsx_size_t *out_reduce)
{
    gsx_size_t outer = 1, reduce = 1;
    gsx_index_t d = 0;

    if(shape == NULL || rank < 1 || start_axis < 0 || start_axis >= rank) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "reduce shape metadata is invalid");
    }
    for(d = 0; d < rank; ++d) {
        gsx_size_t *acc = d < start_axis ? &outer : &reduce;

        if(shape[d] < 0 || gsx_size_mul_overflows(*acc, (gsx_size_t)shape[d], acc)) {
            return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "reduce extent overflows");
        }
    }
    *out_outer = outer;
    *out_reduce = reduce;
    return ok();
}

static gsx_error hip_query_unary_reduce_workspace(gsx_backend_t backend, gsx_backend_buffer_type_class ws_type,
    gsx_data_type data_type, gsx_index_t x_rank, const gsx_index_t *x_shape, gsx_index_t out_rank,
    const gsx_index_t *out_shape, gsx_index_t start_axis, gsx_impl_unary_reduce_op op, gsx_size_t *out_bytes,
    gsx_size_t *out_alignment)
{
    gsx_size_t outer = 0, reduce = 0;

    (void)backend;
    (void)out_rank;
    (void)out_shape;
    (void)op;
    if(out_bytes == NULL || out_alignment == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "workspace outputs must be non-null");
    }
    if(ws_type != GSX_BACKEND_BUFFER_TYPE_DEVICE) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip reduce workspace must be device memory");
    }
    if(data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip reduce supports float32 only");
    }
    GSX_TRY(hip_reduce_extents(x_rank, x_shape, start_axis, &outer, &reduce));
    *out_bytes = (gsx_size_t)gsx_hip_reduce_temp_bytes((int64_t)outer, (int64_t)(reduce > 0 ? reduce : 1));
    *out_alignment = 256;
    return ok();
}

static gsx_error hip_query_binary_reduce_workspace(gsx_backend_t backend, gsx_backend_buffer_type_class ws_type,
    gsx_data_type data_type, gsx_index_t lhs_rank, const gsx_index_t *lhs_shape, gsx_index_t rhs_rank,
    const gsx_index_t *rhs_shape, gsx_index_t out_rank, const gsx_index_t *out_shape, gsx_index_t start_axis,
    gsx_impl_binary_reduce_op op, gsx_size_t *out_bytes, gsx_size_t *out_alignment)
{
    (void)rhs_rank;
    (void)rhs_shape;
    return hip_query_unary_reduce_workspace(backend, ws_type, data_type, lhs_rank, lhs_shape, out_rank, out_shape,
        start_axis, (gsx_impl_unary_reduce_op)op, out_bytes, out_alignment);
}

bool gsx_hip_plugin_tensor_on_device(gsx_backend_t backend, gsx_tensor_t tensor)
{
    gsx_hip_plugin_backend *b = gsx_hip_plugin_backend_of(backend);

    return tensor != NULL && tensor->backing_buffer != NULL
        && tensor->backing_buffer->buffer_type == &b->device_type.base;
}

gsx_size_t gsx_hip_plugin_tensor_elements(gsx_tensor_t tensor)
{
    gsx_size_t n = 1;
    gsx_index_t d = 0;

    for(d = 0; d < tensor->rank; ++d) {
        n *= (gsx_size_t)tensor->shape[d];
    }
    return n;
}

/* ---- buffer types ---------------------------------------------------------------------------- */

static const gsx_backend_buffer_i hip_buffer_iface;

static gsx_error hip_buffer_type_get_info(gsx_backend_buffer_type_t buffer_type, gsx_backend_buffer_type_info *out)
{
    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_info must be non-null");
    }
    *out = ((gsx_hip_plugin_buffer_type *)buffer_type)->info;
    return ok();
}

static gsx_error hip_buffer_type_get_alloc_size(gsx_backend_buffer_type_t buffer_type, gsx_size_t requested,
    gsx_size_t *out)
{
    gsx_size_t align = ((gsx_hip_plugin_buffer_type *)buffer_type)->info.alignment_bytes;

    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_alloc_size_bytes must be non-null");
    }
    if(gsx_round_up_overflows(requested, align, out)) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "allocation size overflows");
    }
    return ok();
}

static gsx_error hip_buffer_type_init_buffer(gsx_backend_buffer_type_t buffer_type, const gsx_backend_buffer_desc *desc,
    gsx_backend_buffer_t *out)
{
    gsx_hip_plugin_buffer_type *t = (gsx_hip_plugin_buffer_type *)buffer_type;
    gsx_hip_plugin_buffer *buf = NULL;
    gsx_size_t align = 0, alloc = 0;
    gsx_hip_status st = GSX_HIP_SUCCESS;

    if(desc == NULL || out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "desc and out_buffer must be non-null");
    }
    *out = NULL;
    if(desc->size_bytes == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer size must be non-zero");
    }
    align = desc->alignment_bytes != 0 ? desc->alignment_bytes : t->info.alignment_bytes;
    if(!gsx_is_power_of_two(align)) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer alignment must be a power of two");
    }
    if(align > 256) {
        /* hipMalloc returns 256-byte aligned memory; larger alignments are not offered */
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip buffers are aligned to at most 256 bytes");
    }
    if(gsx_round_up_overflows(desc->size_bytes, t->info.alignment_bytes, &alloc)) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "buffer size overflows");
    }
    buf = (gsx_hip_plugin_buffer *)calloc(1, sizeof(*buf));
    if(buf == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip buffer object");
    }
    if(t->info.type == GSX_BACKEND_BUFFER_TYPE_DEVICE) {
        /* from the stream-ordered pool: gsx_gs_resize reallocates whole Gaussian sets on every
         * density-control commit (gsx-core.c:2811-2869) */
        st = gsx_hip_pool_malloc(&buf->ptr, (size_t)alloc, gsx_hip_plugin_stream(buffer_type->backend));
    } else {
        st = gsx_hip_host_alloc(&buf->host, (size_t)alloc);
        if(st == GSX_HIP_SUCCESS) st = gsx_hip_host_device_pointer(buf->host, &buf->ptr);
    }
    if(st != GSX_HIP_SUCCESS) {
        if(buf->host != NULL) (void)gsx_hip_host_free(buf->host);
        else if(buf->ptr != NULL) (void)gsx_hip_pool_free(buf->ptr, gsx_hip_plugin_stream(buffer_type->backend));
        free(buf);
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "hip buffer allocation failed");
    }
    buf->base.iface = &hip_buffer_iface;
    buf->base.buffer_type = buffer_type;
    buf->base.size_bytes = desc->size_bytes;
    buf->base.alignment_bytes = align;
    *out = &buf->base;
    return ok();
}

static const gsx_backend_buffer_type_i hip_buffer_type_iface = {
    hip_buffer_type_get_info,
    hip_buffer_type_get_alloc_size,
    hip_buffer_type_init_buffer
};

/* ---- buffers ----------------------------------------------------------------------------------- */

static gsx_hip_plugin_buffer *hb(gsx_backend_buffer_t buffer) { return (gsx_hip_plugin_buffer *)buffer; }

static hipStream_t hb_stream(gsx_backend_buffer_t buffer) { return gsx_hip_plugin_stream(buffer->buffer_type->backend); }

static gsx_error hb_check_range(gsx_backend_buffer_t buffer, gsx_size_t offset, gsx_size_t count)
{
    gsx_size_t end = 0;

    if(offset > buffer->size_bytes || gsx_size_add_overflows(offset, count, &end) || end > buffer->size_bytes) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "buffer byte range exceeds the logical buffer size");
    }
    return ok();
}

/* view of `buffer` that lies inside it (gsx-cpu/core.c:385-399) */
static gsx_error hb_check_view(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view)
{
    gsx_size_t end = 0;

    if(view == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor_view must be non-null");
    }
    if(view->buffer != buffer) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor_view must reference the provided buffer");
    }
    if(gsx_size_add_overflows(view->offset_bytes, view->size_bytes, &end) || end > buffer->size_bytes) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "tensor view exceeds the backing buffer");
    }
    return ok();
}

/* a view of any buffer of the same backend */
static gsx_error hb_check_foreign_view(gsx_backend_buffer_t dst, const gsx_backend_tensor_view *view)
{
    if(view == NULL || view->buffer == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor views must be non-null");
    }
    if(view->buffer->buffer_type->backend != dst->buffer_type->backend) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensors must belong to the same backend");
    }
    return hb_check_view(view->buffer, view);
}

static void *hb_view_ptr(const gsx_backend_tensor_view *view)
{
    return (unsigned char *)hb(view->buffer)->ptr + (size_t)view->offset_bytes;
}

static gsx_error hb_free(gsx_backend_buffer_t buffer)
{
    gsx_hip_plugin_buffer *b = hb(buffer);

    if(buffer == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer must be non-null");
    }
    if(b->host != NULL) {
        /* queued work may still read or write the buffer, and the host touches pinned memory
         * directly: wait for the stream before the memory goes */
        (void)gsx_hip_stream_synchronize(hb_stream(buffer));
        (void)gsx_hip_host_free(b->host);
    } else {
        /* device memory returns to the pool behind the queued work (no host wait) */
        (void)gsx_hip_pool_free(b->ptr, hb_stream(buffer));
    }
    free(b);
    return ok();
}

static gsx_error hb_get_info(gsx_backend_buffer_t buffer, gsx_backend_buffer_info *out)
{
    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_info must be non-null");
    }
    out->backend = buffer->buffer_type->backend;
    out->buffer_type = buffer->buffer_type;
    out->size_bytes = buffer->size_bytes;
    out->alignment_bytes = buffer->alignment_bytes;
    return ok();
}

static gsx_error hb_get_native_handle(gsx_backend_buffer_t buffer, void **out)
{
    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_handle must be non-null");
    }
    *out = hb(buffer)->host != NULL ? hb(buffer)->host : hb(buffer)->ptr;
    return ok();
}

/* host address of byte `offset` (pinned buffers) or device address (device buffers) */
static void *hb_copy_ptr(gsx_backend_buffer_t buffer, gsx_size_t offset)
{
    gsx_hip_plugin_buffer *b = hb(buffer);

    return (unsigned char *)(b->host != NULL ? b->host : b->ptr) + (size_t)offset;
}

static gsx_error hb_upload(gsx_backend_buffer_t buffer, gsx_size_t dst_offset, const void *src, gsx_size_t count)
{
    GSX_TRY(hb_check_range(buffer, dst_offset, count));
    if(count == 0) return ok();
    if(src == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "src_bytes must be non-null for non-zero byte_count");
    }
    HIP_TRY(gsx_hip_memcpy_async(hb_copy_ptr(buffer, dst_offset), src, (size_t)count, hb_stream(buffer)),
        "hip upload failed");
    return ok();
}

static gsx_error hb_download(gsx_backend_buffer_t buffer, gsx_size_t src_offset, void *dst, gsx_size_t count)
{
    GSX_TRY(hb_check_range(buffer, src_offset, count));
    if(count == 0) return ok();
    if(dst == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "dst_bytes must be non-null for non-zero byte_count");
    }
    HIP_TRY(gsx_hip_memcpy_async(dst, hb_copy_ptr(buffer, src_offset), (size_t)count, hb_stream(buffer)),
        "hip download failed");
    return ok();
}

static gsx_error hb_set_zero(gsx_backend_buffer_t buffer)
{
    const uint8_t zero = 0;

    HIP_TRY(gsx_hip_fill_pattern(hb(buffer)->ptr, (size_t)buffer->size_bytes, &zero, 1, hb_stream(buffer)),
        "hip set_zero failed");
    return ok();
}

static gsx_error hb_memset_tensor(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, uint8_t value,
    gsx_size_t offset, gsx_size_t size)
{
    gsx_size_t end = 0;

    GSX_TRY(hb_check_view(buffer, view));
    if(gsx_size_add_overflows(offset, size, &end) || end > view->size_bytes) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "tensor subrange exceeds the tensor size");
    }
    if(size == 0) return ok();
    HIP_TRY(gsx_hip_fill_pattern((unsigned char *)hb_view_ptr(view) + (size_t)offset, (size_t)size, &value, 1,
                hb_stream(buffer)), "hip memset failed");
    return ok();
}

static gsx_error hb_set_tensor(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, const void *src,
    gsx_size_t offset, gsx_size_t size)
{
    gsx_size_t abs = 0;

    if(view == NULL || view->buffer != buffer) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor_view must reference the provided buffer");
    }
    if(gsx_size_add_overflows(view->offset_bytes, offset, &abs)) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "tensor offset overflow");
    }
    return hb_upload(buffer, abs, src, size);
}

static gsx_error hb_get_tensor(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, void *dst,
    gsx_size_t offset, gsx_size_t size)
{
    gsx_size_t abs = 0;

    if(view == NULL || view->buffer != buffer) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor_view must reference the provided buffer");
    }
    if(gsx_size_add_overflows(view->offset_bytes, offset, &abs)) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "tensor offset overflow");
    }
    return hb_download(buffer, abs, dst, size);
}

/* gsx-cpu/core.c:874-931: same backend, equal sizes, identical or disjoint ranges */
static gsx_error hb_copy_tensor(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *src,
    const gsx_backend_tensor_view *dst)
{
    if(dst_buffer == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer and tensor views must be non-null");
    }
    GSX_TRY(hb_check_foreign_view(dst_buffer, src));
    GSX_TRY(hb_check_view(dst_buffer, dst));
    if(src->size_bytes != dst->size_bytes) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor copy requires equal source and destination sizes");
    }
    if(src->size_bytes == 0) return ok();
    if(src->buffer == dst_buffer) {
        gsx_size_t s0 = src->offset_bytes, s1 = s0 + src->size_bytes;
        gsx_size_t d0 = dst->offset_bytes, d1 = d0 + dst->size_bytes;

        if(s0 == d0 && s1 == d1) return ok();
        if(!(d1 <= s0 || s1 <= d0)) {
            return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor copy rejects overlapping source and destination ranges");
        }
    }
    HIP_TRY(gsx_hip_memcpy_async(hb_view_ptr(dst), hb_view_ptr(src), (size_t)src->size_bytes, hb_stream(dst_buffer)),
        "hip tensor copy failed");
    return ok();
}

static gsx_error hb_fill_tensor(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, const void *value,
    gsx_size_t value_size)
{
    if(value_size == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "value_size_bytes must be non-zero");
    }
    if(view == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor_view must be non-null");
    }
    if(view->size_bytes != 0 && value == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "value_bytes must be non-null when the tensor is non-empty");
    }
    if(view->size_bytes % value_size != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor byte size must be a multiple of value_size_bytes");
    }
    GSX_TRY(hb_check_view(buffer, view));
    if(view->size_bytes == 0) return ok();
    if(value_size > 64) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip fill supports values of at most 64 bytes");
    }
    HIP_TRY(gsx_hip_fill_pattern(hb_view_ptr(view), (size_t)view->size_bytes, value, (size_t)value_size,
                hb_stream(buffer)), "hip fill failed");
    return ok();
}

static gsx_error hb_require_f32_view(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, const char *what)
{
    GSX_TRY(hb_check_view(buffer, view));
    if(view->data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, what);
    }
    if(view->size_bytes % sizeof(float) != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "float32 tensor byte size must be divisible by sizeof(float)");
    }
    return ok();
}

static gsx_error hb_fill_rand(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, uint64_t state,
    uint64_t inc)
{
    GSX_TRY(hb_require_f32_view(buffer, view, "rand fill only supports float32 tensors"));
    HIP_TRY(gsx_hip_fill_rand_f32((float *)hb_view_ptr(view), (int64_t)(view->size_bytes / 4), state, inc,
                hb_stream(buffer)), "hip rand fill failed");
    return ok();
}

static gsx_error hb_fill_randn(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, uint64_t state,
    uint64_t inc, gsx_float_t sigma)
{
    GSX_TRY(hb_require_f32_view(buffer, view, "randn fill only supports float32 tensors"));
    HIP_TRY(gsx_hip_fill_randn_f32((float *)hb_view_ptr(view), (int64_t)(view->size_bytes / 4), state, inc, sigma,
                hb_stream(buffer)), "hip randn fill failed");
    return ok();
}

static gsx_error hb_fill_randint(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, uint64_t state,
    uint64_t inc, uint32_t bound)
{
    int32_t elem = 0;
    int64_t count = 0, draws = 0, accepted = 0;
    void *temp = NULL;
    gsx_hip_status st = GSX_HIP_SUCCESS;

    GSX_TRY(hb_check_view(buffer, view));
    if(view->data_type == GSX_DATA_TYPE_U8) {
        elem = 1;
    } else if(view->data_type == GSX_DATA_TYPE_I32) {
        elem = 4;
        if(view->size_bytes % 4 != 0) {
            return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "int32 tensor byte size must be divisible by sizeof(int32_t)");
        }
    } else {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "randint fill only supports uint8 and int32 tensors");
    }
    if(bound == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "bound must be non-zero");
    }
    count = (int64_t)(view->size_bytes / (gsx_size_t)elem);
    if(count == 0) return ok();
    /* rejections of pcg32_next_uint_bound are rare for small bounds and at most half the draws:
     * examine a margin of extra draws and widen it until enough were accepted */
    draws = count + count / 8 + 4096;
    for(;;) {
        size_t bytes = gsx_hip_fill_randint_temp_bytes(draws);

        HIP_TRY(gsx_hip_pool_malloc(&temp, bytes, hb_stream(buffer)), "hip randint workspace allocation failed");
        st = gsx_hip_fill_randint(hb_view_ptr(view), count, elem, state, inc, bound, draws, temp, &accepted,
            hb_stream(buffer));
        (void)gsx_hip_pool_free(temp, hb_stream(buffer));
        HIP_TRY(st, "hip randint fill failed");
        if(accepted >= count) break;
        if(draws > INT64_MAX / 4) {
            return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "randint fill rejected too many draws");
        }
        draws = 2 * draws + (count - accepted) * 4;
    }
    return ok();
}

static gsx_error hb_multinomial(gsx_backend_buffer_t out_buffer, const gsx_backend_tensor_view *out_view,
    const gsx_backend_tensor_view *cdf_view, uint64_t state, uint64_t inc)
{
    int64_t samples = 0, categories = 0;

    if(out_view == NULL || cdf_view == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "multinomial tensor views must be non-null");
    }
    GSX_TRY(hb_check_view(out_buffer, out_view));
    GSX_TRY(hb_check_foreign_view(out_buffer, cdf_view));
    if(out_view->data_type != GSX_DATA_TYPE_I32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "multinomial output only supports int32 tensors");
    }
    if(cdf_view->data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "multinomial cdf only supports float32 tensors");
    }
    if(out_view->size_bytes % 4 != 0 || cdf_view->size_bytes % 4 != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "multinomial tensor byte sizes must be multiples of 4");
    }
    samples = (int64_t)(out_view->size_bytes / 4);
    categories = (int64_t)(cdf_view->size_bytes / 4);
    if(samples == 0 || categories == 0) return ok();
    if(categories > (int64_t)INT32_MAX) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "multinomial category count exceeds int32 output range");
    }
    HIP_TRY(gsx_hip_multinomial_i32((int32_t *)hb_view_ptr(out_view), samples, (const float *)hb_view_ptr(cdf_view),
                categories, state, inc, hb_stream(out_buffer)), "hip multinomial failed");
    return ok();
}

/* One device word: cleared, written by a kernel, read back after the stream drains. */
static gsx_error hb_read_flag(gsx_hip_plugin_backend *b, uint32_t *out)
{
    HIP_TRY(gsx_hip_memcpy_async(b->flag_host, b->flag, sizeof(uint32_t), b->stream), "hip flag readback failed");
    HIP_TRY(gsx_hip_stream_synchronize(b->stream), "hip flag readback failed");
    *out = *(volatile uint32_t *)b->flag_host;
    return ok();
}

static gsx_error hb_clear_flag(gsx_hip_plugin_backend *b)
{
    const uint32_t zero = 0;

    HIP_TRY(gsx_hip_fill_pattern(b->flag, sizeof(uint32_t), &zero, sizeof(zero), b->stream), "hip flag clear failed");
    return ok();
}

static gsx_error hb_check_finite(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, bool *out)
{
    gsx_hip_plugin_backend *b = gsx_hip_plugin_backend_of(buffer->buffer_type->backend);
    uint32_t bad = 0;

    if(out == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_is_finite must be non-null");
    }
    *out = true;
    GSX_TRY(hb_require_f32_view(buffer, view, "finite check is only implemented for float32 tensors"));
    if(view->size_bytes == 0) return ok();
    GSX_TRY(hb_clear_flag(b));
    HIP_TRY(gsx_hip_check_finite_f32((const float *)hb_view_ptr(view), (int64_t)(view->size_bytes / 4), b->flag,
                b->stream), "hip finite check failed");
    GSX_TRY(hb_read_flag(b, &bad));
    *out = bad == 0;
    return ok();
}

/* gsx-cpu/core.c:1248-1333: rows of x by int32 index; an index out of range fails */
static gsx_error hb_gather(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *x_view,
    const gsx_backend_tensor_view *index_view, const gsx_backend_tensor_view *out_view, gsx_index_t x_rank,
    const gsx_index_t *x_shape, gsx_index_t out_rank, const gsx_index_t *out_shape)
{
    gsx_hip_plugin_backend *b = gsx_hip_plugin_backend_of(dst_buffer->buffer_type->backend);
    gsx_size_t rows = 0, row_bytes = 0, expect = 0;
    uint32_t bad = 0;

    if(x_shape == NULL || out_shape == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer, tensor views, and shapes must be non-null");
    }
    GSX_TRY(hb_check_foreign_view(dst_buffer, x_view));
    GSX_TRY(hb_check_foreign_view(dst_buffer, index_view));
    GSX_TRY(hb_check_view(dst_buffer, out_view));
    rows = (gsx_size_t)out_shape[0];
    if(rows == 0 || x_rank < 1 || out_rank < 1) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "gather shape metadata is invalid");
    }
    if(out_view->size_bytes % rows != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "gather output view byte size must be row-aligned");
    }
    row_bytes = out_view->size_bytes / rows;
    if(gsx_size_mul_overflows((gsx_size_t)x_shape[0], row_bytes, &expect) || expect != x_view->size_bytes) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "gather x view byte size is inconsistent with row metadata");
    }
    if(index_view->size_bytes != rows * sizeof(int32_t)) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "index view byte size must match out leading dimension");
    }
    GSX_TRY(hb_clear_flag(b));
    HIP_TRY(gsx_hip_gather_rows_kernel_launch(hb_view_ptr(x_view), hb_view_ptr(out_view), (int64_t)row_bytes,
                (int64_t)rows, (const int32_t *)hb_view_ptr(index_view), (int64_t)x_shape[0], (int *)b->flag,
                b->stream), "hip gather failed");
    GSX_TRY(hb_read_flag(b, &bad));
    if(bad != 0) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "gather index is out of range");
    }
    return ok();
}

static gsx_error hb_unary(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *x_view,
    const gsx_backend_tensor_view *out_view, gsx_index_t rank, const gsx_index_t *shape, gsx_impl_unary_op op)
{
    (void)rank;
    if(shape == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer, tensor views, and shape must be non-null");
    }
    GSX_TRY(hb_check_foreign_view(dst_buffer, x_view));
    GSX_TRY(hb_check_view(dst_buffer, out_view));
    if(x_view->size_bytes != out_view->size_bytes) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "x and out view byte sizes must match");
    }
    if(x_view->data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "unary tensor op only supports float32 tensors");
    }
    if(x_view->size_bytes % 4 != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "float32 tensor byte size must be divisible by sizeof(float)");
    }
    if((int)op < GSX_HIP_UNARY_EXP || (int)op > GSX_HIP_UNARY_ABS) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "unknown unary tensor op");
    }
    HIP_TRY(gsx_hip_unary_f32((const float *)hb_view_ptr(x_view), (float *)hb_view_ptr(out_view),
                (int64_t)(x_view->size_bytes / 4), (int32_t)op, hb_stream(dst_buffer)), "hip unary op failed");
    return ok();
}

static gsx_error hb_unary_inplace(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, gsx_impl_unary_op op)
{
    GSX_TRY(hb_require_f32_view(buffer, view, "unary tensor op only supports float32 tensors"));
    if((int)op < GSX_HIP_UNARY_EXP || (int)op > GSX_HIP_UNARY_ABS) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "unknown unary tensor op");
    }
    HIP_TRY(gsx_hip_unary_f32((const float *)hb_view_ptr(view), (float *)hb_view_ptr(view),
                (int64_t)(view->size_bytes / 4), (int32_t)op, hb_stream(buffer)), "hip unary op failed");
    return ok();
}

static gsx_error hb_reduce_common(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *x_view,
    const gsx_backend_tensor_view *y_view, const gsx_backend_tensor_view *out_view,
    const gsx_backend_tensor_view *workspace_view, gsx_index_t rank, const gsx_index_t *shape,
    gsx_index_t start_axis, int32_t op)
{
    gsx_size_t outer = 0, reduce = 0, need = 0;

    GSX_TRY(hb_check_foreign_view(dst_buffer, x_view));
    if(y_view != NULL) GSX_TRY(hb_check_foreign_view(dst_buffer, y_view));
    GSX_TRY(hb_check_view(dst_buffer, out_view));
    if(x_view->data_type != out_view->data_type || (y_view != NULL && y_view->data_type != x_view->data_type)) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "reduce tensor data_type must match");
    }
    if(x_view->data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip reduce only supports float32 tensors");
    }
    GSX_TRY(hip_reduce_extents(rank, shape, start_axis, &outer, &reduce));
    if(out_view->size_bytes != outer * 4 || x_view->size_bytes != outer * reduce * 4
        || (y_view != NULL && y_view->size_bytes != x_view->size_bytes)) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "reduce tensor views are inconsistent with dispatch metadata");
    }
    if(outer == 0) return ok();
    if(reduce == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "reduce over an empty extent");
    }
    need = (gsx_size_t)gsx_hip_reduce_temp_bytes((int64_t)outer, (int64_t)reduce);
    if(workspace_view == NULL || workspace_view->buffer == NULL || workspace_view->size_bytes < need) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "reduce workspace is missing or too small");
    }
    GSX_TRY(hb_check_foreign_view(dst_buffer, workspace_view));
    HIP_TRY(gsx_hip_reduce_f32((const float *)hb_view_ptr(x_view),
                y_view != NULL ? (const float *)hb_view_ptr(y_view) : NULL, (int64_t)outer, (int64_t)reduce, op,
                (float *)hb_view_ptr(out_view), hb_view_ptr(workspace_view), hb_stream(dst_buffer)),
        "hip reduce failed");
    return ok();
}

static gsx_error hb_unary_reduce(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *x_view,
    const gsx_backend_tensor_view *out_view, const gsx_backend_tensor_view *workspace_view, gsx_index_t x_rank,
    const gsx_index_t *x_shape, gsx_index_t out_rank, const gsx_index_t *out_shape, gsx_index_t start_axis,
    gsx_impl_unary_reduce_op op)
{
    int32_t hop = op == GSX_IMPL_UNARY_REDUCE_OP_SUM ? GSX_HIP_REDUCE_SUM
        : op == GSX_IMPL_UNARY_REDUCE_OP_MEAN ? GSX_HIP_REDUCE_MEAN
        : op == GSX_IMPL_UNARY_REDUCE_OP_MAX ? GSX_HIP_REDUCE_MAX : -1;

    (void)out_rank;
    if(out_shape == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "reduce buffers, views, and shapes must be non-null");
    }
    if(hop < 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "unknown unary_reduce op");
    }
    return hb_reduce_common(dst_buffer, x_view, NULL, out_view, workspace_view, x_rank, x_shape, start_axis, hop);
}

static gsx_error hb_binary_reduce(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *lhs_view,
    const gsx_backend_tensor_view *rhs_view, const gsx_backend_tensor_view *out_view,
    const gsx_backend_tensor_view *workspace_view, gsx_index_t lhs_rank, const gsx_index_t *lhs_shape,
    gsx_index_t rhs_rank, const gsx_index_t *rhs_shape, gsx_index_t out_rank, const gsx_index_t *out_shape,
    gsx_index_t start_axis, gsx_impl_binary_reduce_op op)
{
    int32_t hop = op == GSX_IMPL_BINARY_REDUCE_OP_MSE ? GSX_HIP_REDUCE_MSE
        : op == GSX_IMPL_BINARY_REDUCE_OP_MAE ? GSX_HIP_REDUCE_MAE : -1;

    (void)out_rank;
    if(rhs_shape == NULL || out_shape == NULL || rhs_view == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "binary_reduce buffers, views, and shapes must be non-null");
    }
    if(rhs_rank != lhs_rank) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "lhs_rank and rhs_rank must match");
    }
    if(hop < 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "unknown binary_reduce op");
    }
    return hb_reduce_common(dst_buffer, lhs_view, rhs_view, out_view, workspace_view, lhs_rank, lhs_shape, start_axis,
        hop);
}

static gsx_error hb_clamp(gsx_backend_buffer_t buffer, const gsx_backend_tensor_view *view, const void *lo,
    const void *hi)
{
    gsx_size_t elem = 0;
    int32_t dtype = 0;

    if(lo == NULL || hi == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "buffer, tensor_view, min_value, and max_value must be non-null");
    }
    GSX_TRY(hb_check_view(buffer, view));
    GSX_TRY(gsx_data_type_get_size_bytes(view->data_type, &elem));
    if(view->size_bytes % elem != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "tensor view byte size is not aligned to element size");
    }
    switch(view->data_type) {
    case GSX_DATA_TYPE_F32: dtype = GSX_HIP_DTYPE_F32; break;
    case GSX_DATA_TYPE_U8: dtype = GSX_HIP_DTYPE_U8; break;
    case GSX_DATA_TYPE_I32: dtype = GSX_HIP_DTYPE_I32; break;
    default:
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "clamp_inplace only supports f32, u8, and i32 tensors");
    }
    HIP_TRY(gsx_hip_clamp_inplace(hb_view_ptr(view), (int64_t)(view->size_bytes / elem), dtype, lo, hi,
                hb_stream(buffer)), "hip clamp failed");
    return ok();
}

static gsx_error hb_image_dims(gsx_index_t rank, const gsx_index_t *shape, gsx_storage_format format,
    gsx_index_t *c, gsx_index_t *h, gsx_index_t *w)
{
    if(shape == NULL || rank != 3) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "image tensor rank must be 3");
    }
    if(format == GSX_STORAGE_FORMAT_CHW) {
        *c = shape[0];
        *h = shape[1];
        *w = shape[2];
    } else if(format == GSX_STORAGE_FORMAT_HWC) {
        *c = shape[2];
        *h = shape[0];
        *w = shape[1];
    } else {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "image storage_format must be CHW or HWC");
    }
    return ok();
}

static gsx_error hb_image_colorspace(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *src_view,
    gsx_storage_format storage_format, gsx_index_t rank, const gsx_index_t *shape, gsx_image_colorspace src_cs,
    const gsx_backend_tensor_view *dst_view, gsx_image_colorspace dst_cs)
{
    (void)storage_format;
    (void)rank;
    if(shape == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "image colorspace conversion inputs must be non-null");
    }
    GSX_TRY(hb_check_foreign_view(dst_buffer, src_view));
    GSX_TRY(hb_check_view(dst_buffer, dst_view));
    if(src_view->data_type != GSX_DATA_TYPE_F32 || dst_view->data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip image colorspace conversion only supports float32 tensors");
    }
    if(src_view->size_bytes != dst_view->size_bytes) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "image colorspace conversion requires equal source and destination sizes");
    }
    HIP_TRY(gsx_hip_image_colorspace_f32((const float *)hb_view_ptr(src_view), (float *)hb_view_ptr(dst_view),
                (int64_t)(src_view->size_bytes / 4), src_cs == GSX_IMAGE_COLOR_SPACE_SRGB,
                dst_cs == GSX_IMAGE_COLOR_SPACE_SRGB, hb_stream(dst_buffer)), "hip colorspace conversion failed");
    return ok();
}

static gsx_error hb_image_storage(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *src_view,
    gsx_index_t src_rank, const gsx_index_t *src_shape, gsx_storage_format src_format,
    const gsx_backend_tensor_view *dst_view, gsx_index_t dst_rank, const gsx_index_t *dst_shape,
    gsx_storage_format dst_format)
{
    gsx_index_t sc = 0, sh = 0, sw = 0, dc = 0, dh = 0, dw = 0;
    gsx_size_t elem = 0;

    GSX_TRY(hb_check_foreign_view(dst_buffer, src_view));
    GSX_TRY(hb_check_view(dst_buffer, dst_view));
    if(src_view->data_type != dst_view->data_type) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "image storage conversion requires matching data types");
    }
    GSX_TRY(gsx_data_type_get_size_bytes(src_view->data_type, &elem));
    if(!gsx_error_is_success(hb_image_dims(src_rank, src_shape, src_format, &sc, &sh, &sw))
        || !gsx_error_is_success(hb_image_dims(dst_rank, dst_shape, dst_format, &dc, &dh, &dw))
        || sc != dc || sh != dh || sw != dw) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "image storage conversion requires matching logical extents");
    }
    if(src_view->size_bytes != (gsx_size_t)sc * (gsx_size_t)sh * (gsx_size_t)sw * elem
        || dst_view->size_bytes != src_view->size_bytes) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "image storage conversion views are inconsistent with their shapes");
    }
    HIP_TRY(gsx_hip_image_storage_convert(hb_view_ptr(src_view), src_format == GSX_STORAGE_FORMAT_HWC,
                hb_view_ptr(dst_view), dst_format == GSX_STORAGE_FORMAT_HWC, sc, sh, sw, (int32_t)elem,
                hb_stream(dst_buffer)), "hip storage conversion failed");
    return ok();
}

static gsx_error hb_image_data_type(gsx_backend_buffer_t dst_buffer, const gsx_backend_tensor_view *src_view,
    gsx_storage_format storage_format, gsx_index_t rank, const gsx_index_t *shape,
    const gsx_backend_tensor_view *dst_view)
{
    gsx_index_t c = 0, h = 0, w = 0;
    int64_t count = 0;

    GSX_TRY(hb_check_foreign_view(dst_buffer, src_view));
    GSX_TRY(hb_check_view(dst_buffer, dst_view));
    if(!((src_view->data_type == GSX_DATA_TYPE_F32 && dst_view->data_type == GSX_DATA_TYPE_U8)
            || (src_view->data_type == GSX_DATA_TYPE_U8 && dst_view->data_type == GSX_DATA_TYPE_F32))) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip image data type conversion only supports float32 and uint8");
    }
    GSX_TRY(hb_image_dims(rank, shape, storage_format, &c, &h, &w));
    count = (int64_t)c * h * w;
    if(src_view->size_bytes != (gsx_size_t)count * (src_view->data_type == GSX_DATA_TYPE_F32 ? 4u : 1u)
        || dst_view->size_bytes != (gsx_size_t)count * (dst_view->data_type == GSX_DATA_TYPE_F32 ? 4u : 1u)) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "image data type conversion views are inconsistent with their shapes");
    }
    if(src_view->data_type == GSX_DATA_TYPE_F32) {
        HIP_TRY(gsx_hip_image_quantize_u8((const float *)hb_view_ptr(src_view), (uint8_t *)hb_view_ptr(dst_view), count,
                    hb_stream(dst_buffer)), "hip image quantize failed");
    } else {
        HIP_TRY(gsx_hip_image_dequantize_u8((const uint8_t *)hb_view_ptr(src_view), (float *)hb_view_ptr(dst_view),
                    count, hb_stream(dst_buffer)), "hip image dequantize failed");
    }
    return ok();
}

static const gsx_backend_buffer_i hip_buffer_iface = {
    hb_free,
    hb_get_info,
    hb_get_native_handle,
    hb_upload,
    hb_download,
    hb_set_zero,
    hb_memset_tensor,
    hb_set_tensor,
    hb_get_tensor,
    hb_copy_tensor,
    hb_fill_tensor,
    hb_fill_rand,
    hb_fill_randn,
    hb_fill_randint,
    hb_multinomial,
    hb_check_finite,
    hb_gather,
    hb_unary,
    hb_unary_inplace,
    hb_unary_reduce,
    hb_binary_reduce,
    hb_clamp,
    hb_image_colorspace,
    hb_image_storage,
    hb_image_data_type
};
