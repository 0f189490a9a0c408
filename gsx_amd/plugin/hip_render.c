/*
 * hip_render.c - renderer and render-context vtables of the gsx HIP backend
 * (gsx/src/gsx-impl.h:475-484), over the render context of libgsx_hip.so. Counterpart of
 * gsx/src/gsx-cuda/render.c:1314-1571, with the CPU renderer's semantics and feature set
 * (gsx/src/gsx-cpu/render.c:1126-1154, 1254-1365, 1396-1975): float32 RGB only, no METRIC mode,
 * no cov3d input, no alpha/inverse-depth outputs; TRAIN retains state for exactly one backward,
 * cloned or borrowed as the request asks; gradient sinks are overwritten.
 */
#include "hip_backend.h"

#include <stdlib.h>
#include <string.h>

typedef struct hip_renderer {
    struct gsx_renderer base;
} hip_renderer;

typedef struct hip_render_context {
    struct gsx_render_context base;
    gsx_hip_render_context *ctx;
    bool has_train_state;
    gsx_index_t sh_degree;
    gsx_index_t count; /* Gaussians of the retained TRAIN forward */
} hip_render_context;

static gsx_error hr_ok(void) { return gsx_make_error(GSX_ERROR_SUCCESS, NULL); }

static gsx_error hr_destroy(gsx_renderer_t renderer);
static gsx_error hr_create_context(gsx_renderer_t renderer, gsx_render_context_t *out_context);
static gsx_error hr_render(gsx_renderer_t renderer, gsx_render_context_t context, const gsx_render_forward_request *request);
static gsx_error hr_backward(gsx_renderer_t renderer, gsx_render_context_t context,
    const gsx_render_backward_request *request);
static gsx_error hrc_destroy(gsx_render_context_t context);

static const gsx_renderer_i hip_renderer_iface = { hr_destroy, hr_create_context, hr_render, hr_backward };
static const gsx_render_context_i hip_render_context_iface = { hrc_destroy };

gsx_error gsx_hip_plugin_create_renderer(gsx_backend_t backend, const gsx_renderer_desc *desc, gsx_renderer_t *out)
{
    hip_renderer *r = NULL;
    gsx_renderer_capabilities caps = { 0 };
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(out == NULL || desc == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_renderer and desc must be non-null");
    }
    *out = NULL;
    if(desc->output_data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip renderer only supports float32 output_data_type");
    }
    if((desc->feature_flags & GSX_RENDERER_FEATURE_ANTIALIASING) != 0) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip renderer antialiasing feature flag is not implemented");
    }
    if(desc->enable_alpha_output || desc->enable_invdepth_output) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip renderer only supports RGB outputs");
    }
    r = (hip_renderer *)calloc(1, sizeof(*r));
    if(r == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip renderer");
    }
    caps.supported_precisions = GSX_RENDER_PRECISION_FLAG_FLOAT32;
    error = gsx_renderer_base_init(&r->base, &hip_renderer_iface, backend, desc, &caps);
    if(!gsx_error_is_success(error)) {
        free(r);
        return error;
    }
    *out = &r->base;
    return hr_ok();
}

static gsx_error hr_destroy(gsx_renderer_t renderer)
{
    if(renderer == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "renderer must be non-null");
    }
    gsx_renderer_base_deinit(renderer);
    free(renderer);
    return hr_ok();
}

static gsx_error hr_create_context(gsx_renderer_t renderer, gsx_render_context_t *out_context)
{
    hip_render_context *c = NULL;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };
    gsx_hip_status st = GSX_HIP_SUCCESS;

    if(out_context == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_context must be non-null");
    }
    *out_context = NULL;
    c = (hip_render_context *)calloc(1, sizeof(*c));
    if(c == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip render context");
    }
    st = gsx_hip_render_context_create(&c->ctx);
    if(st != GSX_HIP_SUCCESS) {
        free(c);
        return gsx_hip_plugin_error(st, "hip render context creation failed");
    }
    error = gsx_render_context_base_init(&c->base, &hip_render_context_iface, renderer);
    if(!gsx_error_is_success(error)) {
        (void)gsx_hip_render_context_destroy(c->ctx);
        free(c);
        return error;
    }
    *out_context = &c->base;
    return hr_ok();
}

static gsx_error hrc_destroy(gsx_render_context_t context)
{
    hip_render_context *c = (hip_render_context *)context;
    gsx_backend_t backend = NULL;

    if(context == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "context must be non-null");
    }
    backend = context->renderer->backend;
    /* queued kernels may still use the context's buffers */
    (void)gsx_hip_stream_synchronize(gsx_hip_plugin_stream(backend));
    (void)gsx_hip_render_context_destroy(c->ctx);
    gsx_render_context_base_deinit(&c->base);
    free(c);
    return hr_ok();
}

static gsx_error hr_require_device(gsx_backend_t backend, gsx_tensor_t tensor, const char *what)
{
    if(tensor != NULL && !gsx_hip_plugin_tensor_on_device(backend, tensor)) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, what);
    }
    return hr_ok();
}

static gsx_error hr_render(gsx_renderer_t renderer, gsx_render_context_t context, const gsx_render_forward_request *request)
{
    hip_render_context *c = (hip_render_context *)context;
    gsx_backend_t backend = renderer->backend;
    gsx_hip_camera cam;
    gsx_hip_gaussians g;
    int32_t type = GSX_HIP_FORWARD_INFERENCE;
    gsx_hip_status st = GSX_HIP_SUCCESS;
    gsx_tensor_t inputs[9];
    int i = 0;

    /* features the CPU backend rejects too (gsx-cpu/render.c:1126-1144) */
    if(request->precision != GSX_RENDER_PRECISION_FLOAT32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "requested render precision is not supported");
    }
    if(request->forward_type == GSX_RENDER_FORWARD_TYPE_METRIC) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "metric render mode is not implemented");
    }
    if(request->out_alpha != NULL || request->out_invdepth != NULL) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "alpha and inverse-depth outputs are not implemented");
    }
    if(request->gs_cov3d != NULL) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "gs_cov3d input is not implemented");
    }
    if(request->metric_map != NULL || request->gs_metric_accumulator != NULL) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "metric render inputs are not implemented");
    }
    /* render tensors must be device-backed (gsx-render.h:63-64) */
    inputs[0] = request->gs_mean3d;
    inputs[1] = request->gs_rotation;
    inputs[2] = request->gs_logscale;
    inputs[3] = request->gs_opacity;
    inputs[4] = request->gs_sh0;
    inputs[5] = request->gs_sh1;
    inputs[6] = request->gs_sh2;
    inputs[7] = request->gs_sh3;
    inputs[8] = request->out_rgb;
    for(i = 0; i < 9; ++i) {
        gsx_error e = hr_require_device(backend, inputs[i], "hip render tensors must be device-backed");

        if(!gsx_error_is_success(e)) return e;
    }
    {
        gsx_error e = hr_require_device(backend, request->gs_visible_counter, "hip render tensors must be device-backed");

        if(!gsx_error_is_success(e)) return e;
    }

    memset(&cam, 0, sizeof(cam));
    cam.fx = request->intrinsics->fx;
    cam.fy = request->intrinsics->fy;
    cam.cx = request->intrinsics->cx;
    cam.cy = request->intrinsics->cy;
    cam.width = renderer->info.width;
    cam.height = renderer->info.height;
    cam.rot[0] = request->pose->rot.x;
    cam.rot[1] = request->pose->rot.y;
    cam.rot[2] = request->pose->rot.z;
    cam.rot[3] = request->pose->rot.w;
    cam.transl[0] = request->pose->transl.x;
    cam.transl[1] = request->pose->transl.y;
    cam.transl[2] = request->pose->transl.z;
    cam.near_plane = request->near_plane;
    cam.far_plane = request->far_plane;
    cam.background[0] = request->background_color.x;
    cam.background[1] = request->background_color.y;
    cam.background[2] = request->background_color.z;

    memset(&g, 0, sizeof(g));
    g.count = (int64_t)request->gs_mean3d->shape[0];
    g.sh_degree = (int32_t)request->sh_degree;
    g.mean3d = gsx_hip_plugin_tensor_f32(request->gs_mean3d);
    g.rotation = gsx_hip_plugin_tensor_f32(request->gs_rotation);
    g.logscale = gsx_hip_plugin_tensor_f32(request->gs_logscale);
    g.opacity = gsx_hip_plugin_tensor_f32(request->gs_opacity);
    g.sh0 = gsx_hip_plugin_tensor_f32(request->gs_sh0);
    g.sh1 = request->sh_degree >= 1 ? gsx_hip_plugin_tensor_f32(request->gs_sh1) : NULL;
    g.sh2 = request->sh_degree >= 2 ? gsx_hip_plugin_tensor_f32(request->gs_sh2) : NULL;
    g.sh3 = request->sh_degree >= 3 ? gsx_hip_plugin_tensor_f32(request->gs_sh3) : NULL;

    if(request->forward_type == GSX_RENDER_FORWARD_TYPE_TRAIN) {
        type = request->borrow_train_state ? GSX_HIP_FORWARD_TRAIN_BORROW : GSX_HIP_FORWARD_TRAIN_CLONE;
    }
    c->has_train_state = false;
    st = gsx_hip_render_forward(c->ctx, &cam, &g, type, gsx_hip_plugin_tensor_f32(request->out_rgb),
        type != GSX_HIP_FORWARD_INFERENCE ? gsx_hip_plugin_tensor_f32(request->gs_visible_counter) : NULL,
        gsx_hip_plugin_stream(backend));
    if(st != GSX_HIP_SUCCESS) {
        return gsx_hip_plugin_error(st, "hip render forward failed");
    }
    c->has_train_state = type != GSX_HIP_FORWARD_INFERENCE;
    c->sh_degree = request->sh_degree;
    c->count = request->gs_mean3d->shape[0];
    return hr_ok();
}

static gsx_error hr_backward(gsx_renderer_t renderer, gsx_render_context_t context,
    const gsx_render_backward_request *request)
{
    hip_render_context *c = (hip_render_context *)context;
    gsx_backend_t backend = renderer->backend;
    gsx_hip_gaussian_grads grads;
    gsx_hip_status st = GSX_HIP_SUCCESS;
    gsx_tensor_t sinks[10];
    int i = 0;

    if(request->grad_alpha != NULL || request->grad_invdepth != NULL || request->grad_gs_cov3d != NULL) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "only RGB backward is implemented");
    }
    if(!c->has_train_state) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "backward requires a retained TRAIN forward on the same context");
    }
    /* sinks up to the forward's SH degree, none above (gsx-cpu/render.c:1086-1121) */
    if((c->sh_degree >= 1) != (request->grad_gs_sh1 != NULL) || (c->sh_degree >= 2) != (request->grad_gs_sh2 != NULL)
        || (c->sh_degree >= 3) != (request->grad_gs_sh3 != NULL)) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "SH gradient sinks must match the forward's sh_degree");
    }
    /* the front-end checks the sinks against each other (gsx-render.c:247-341); the kernels
     * write one row per Gaussian of the forward */
    if(request->grad_gs_opacity->shape[0] != c->count) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "gradient sinks must have the forward's Gaussian count");
    }
    sinks[0] = request->grad_rgb;
    sinks[1] = request->grad_gs_mean3d;
    sinks[2] = request->grad_gs_rotation;
    sinks[3] = request->grad_gs_logscale;
    sinks[4] = request->grad_gs_opacity;
    sinks[5] = request->grad_gs_sh0;
    sinks[6] = request->grad_gs_sh1;
    sinks[7] = request->grad_gs_sh2;
    sinks[8] = request->grad_gs_sh3;
    sinks[9] = NULL;
    for(i = 0; i < 9; ++i) {
        gsx_error e = hr_require_device(backend, sinks[i], "hip render tensors must be device-backed");

        if(!gsx_error_is_success(e)) return e;
    }
    memset(&grads, 0, sizeof(grads));
    grads.mean3d = gsx_hip_plugin_tensor_f32(request->grad_gs_mean3d);
    grads.rotation = gsx_hip_plugin_tensor_f32(request->grad_gs_rotation);
    grads.logscale = gsx_hip_plugin_tensor_f32(request->grad_gs_logscale);
    grads.opacity = gsx_hip_plugin_tensor_f32(request->grad_gs_opacity);
    grads.sh0 = gsx_hip_plugin_tensor_f32(request->grad_gs_sh0);
    grads.sh1 = gsx_hip_plugin_tensor_f32(request->grad_gs_sh1);
    grads.sh2 = gsx_hip_plugin_tensor_f32(request->grad_gs_sh2);
    grads.sh3 = gsx_hip_plugin_tensor_f32(request->grad_gs_sh3);
    /* gs_grad_acc / gs_absgrad_acc are left untouched, as the CPU backend leaves them */
    c->has_train_state = false;
    st = gsx_hip_render_backward(c->ctx, gsx_hip_plugin_tensor_f32(request->grad_rgb), &grads,
        gsx_hip_plugin_stream(backend));
    if(st != GSX_HIP_SUCCESS) {
        return gsx_hip_plugin_error(st, "hip render backward failed");
    }
    return hr_ok();
}
