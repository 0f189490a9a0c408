/*
 * hip_backend.h - internal types of the gsx HIP backend plugin (the MI355X backend registered in
 * gsx's backend registry). The plugin is gsx-side host C: it implements the vtables of
 * gsx/src/gsx-impl.h:229-533 and calls the C ABI of libgsx_hip.so (include/gsx_hip.h) for all
 * device work. Compiled against gsx's own headers (gsx/include, gsx/src).
 */
#ifndef GSX_HIP_PLUGIN_BACKEND_H
#define GSX_HIP_PLUGIN_BACKEND_H

#include "gsx-impl.h"
#include "gsx_hip.h"

#include <stdbool.h>
#include <stdint.h>

/* The registry slot the HIP provider registers under. gsx's registry accepts the backend types
 * of gsx/include/gsx/gsx-backend.h:8-12 only (gsx-backend.c:184-193); a gsx tree that adds
 * GSX_BACKEND_TYPE_HIP builds the plugin with -DGSX_HIP_BACKEND_TYPE=GSX_BACKEND_TYPE_HIP. Without
 * it the provider takes the GPU slot, so `--backend cuda` of the unmodified apps selects it. */
#ifndef GSX_HIP_BACKEND_TYPE
#define GSX_HIP_BACKEND_TYPE GSX_BACKEND_TYPE_CUDA
#endif

#define GSX_HIP_BACKEND_NAME "hip"

typedef struct gsx_hip_plugin_device {
    struct gsx_backend_device base;
    int32_t ordinal;
    char name[256];
} gsx_hip_plugin_device;

typedef struct gsx_hip_plugin_buffer_type {
    struct gsx_backend_buffer_type base;
    gsx_backend_buffer_type_info info;
} gsx_hip_plugin_buffer_type;

typedef struct gsx_hip_plugin_backend {
    struct gsx_backend base;
    gsx_backend_capabilities capabilities;
    hipStream_t stream; /* the major stream */
    int32_t ordinal;
    gsx_hip_plugin_buffer_type device_type;
    gsx_hip_plugin_buffer_type pinned_type;
    uint32_t *flag;      /* one device word for check_finite / gather range results */
    uint32_t *flag_host; /* pinned word it is read back into */
} gsx_hip_plugin_backend;

typedef struct gsx_hip_plugin_buffer {
    struct gsx_backend_buffer base;
    void *ptr;      /* device-accessible address of byte 0 (device or pinned host memory) */
    void *host;     /* host address for pinned buffers, NULL for device buffers */
} gsx_hip_plugin_buffer;

/* status of libgsx_hip.so -> gsx_error with a static message */
gsx_error gsx_hip_plugin_error(gsx_hip_status status, const char *what);

static inline gsx_hip_plugin_backend *gsx_hip_plugin_backend_of(gsx_backend_t backend)
{
    return (gsx_hip_plugin_backend *)backend;
}

static inline hipStream_t gsx_hip_plugin_stream(gsx_backend_t backend)
{
    return gsx_hip_plugin_backend_of(backend)->stream;
}

/* device address of a tensor's first byte */
static inline void *gsx_hip_plugin_tensor_ptr(gsx_tensor_t tensor)
{
    gsx_hip_plugin_buffer *b = (gsx_hip_plugin_buffer *)tensor->backing_buffer;

    return (unsigned char *)b->ptr + (size_t)tensor->offset_bytes;
}

static inline float *gsx_hip_plugin_tensor_f32(gsx_tensor_t tensor)
{
    return tensor != NULL ? (float *)gsx_hip_plugin_tensor_ptr(tensor) : NULL;
}

/* true when the tensor lives in a buffer of this backend's DEVICE type */
bool gsx_hip_plugin_tensor_on_device(gsx_backend_t backend, gsx_tensor_t tensor);

/* element count of a tensor (product of its shape) */
gsx_size_t gsx_hip_plugin_tensor_elements(gsx_tensor_t tensor);

/* Object constructors of the other plugin files (the gsx_backend_i create_* entries). */
gsx_error gsx_hip_plugin_create_renderer(gsx_backend_t backend, const gsx_renderer_desc *desc, gsx_renderer_t *out);
gsx_error gsx_hip_plugin_create_loss(gsx_backend_t backend, const gsx_loss_desc *desc, gsx_loss_t *out);
gsx_error gsx_hip_plugin_create_optim(gsx_backend_t backend, const gsx_optim_desc *desc, gsx_optim_t *out);
gsx_error gsx_hip_plugin_create_adc(gsx_backend_t backend, const gsx_adc_desc *desc, gsx_adc_t *out);
gsx_error gsx_hip_plugin_create_async_dl(gsx_backend_t backend, const gsx_async_dl_desc *desc, gsx_async_dl_t *out);

/* Registers the provider and one device per visible HIP GPU (gsx-backend.c:225-235 pattern);
 * GSX_ERROR_NOT_SUPPORTED when no device is present, so registry init still succeeds. */
gsx_error gsx_hip_backend_provider_bootstrap(gsx_builtin_registry_state *registry);

#endif /* GSX_HIP_PLUGIN_BACKEND_H */
