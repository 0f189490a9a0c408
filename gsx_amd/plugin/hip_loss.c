/*
 * hip_loss.c - loss and loss-context vtables of the gsx HIP backend (gsx/src/gsx-impl.h:486-495),
 * over the L1 / MSE / SSIM launchers of libgsx_hip.so. Counterpart of gsx/src/gsx-cuda/loss.c with
 * the CPU semantics (gsx/src/gsx-cpu/loss.c:200-395): the forward adds scale * loss into the loss
 * map, the backward adds the gradient scaled by gsx_loss_scale_grad into the accumulator; the
 * front end retains the prediction and target for exactly one backward (gsx-loss.c:438-502).
 * SSIM runs on float32 [C,H,W] or [B,C,H,W] images in CHW storage; its forward keeps the window
 * moments the backward reads in the context's workspace.
 */
#include "hip_backend.h"
#include "gsx-tensor-helpers.h"

#include <stdlib.h>
#include <string.h>

typedef struct hip_loss {
    struct gsx_loss base;
} hip_loss;

typedef struct hip_loss_context {
    struct gsx_loss_context base;
    float *workspace;       /* SSIM moments of the last train forward: 3 floats per element */
    gsx_size_t workspace_floats;
} hip_loss_context;

static gsx_error hl_ok(void) { return gsx_make_error(GSX_ERROR_SUCCESS, NULL); }

static gsx_error hl_destroy(gsx_loss_t loss);
static gsx_error hl_create_context(gsx_loss_t loss, gsx_loss_context_t *out_context);
static gsx_error hl_forward(gsx_loss_t loss, gsx_loss_context_t context, const gsx_loss_forward_request *request);
static gsx_error hl_backward(gsx_loss_t loss, gsx_loss_context_t context, const gsx_loss_backward_request *request);
static gsx_error hlc_destroy(gsx_loss_context_t context);

static const gsx_loss_i hip_loss_iface = { hl_destroy, hl_create_context, hl_forward, hl_backward };
static const gsx_loss_context_i hip_loss_context_iface = { hlc_destroy };

gsx_error gsx_hip_plugin_create_loss(gsx_backend_t backend, const gsx_loss_desc *desc, gsx_loss_t *out)
{
    hip_loss *l = NULL;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(out == NULL || desc == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_loss and desc must be non-null");
    }
    *out = NULL;
    l = (hip_loss *)calloc(1, sizeof(*l));
    if(l == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip loss");
    }
    error = gsx_loss_base_init(&l->base, &hip_loss_iface, backend, desc);
    if(!gsx_error_is_success(error)) {
        free(l);
        return error;
    }
    *out = &l->base;
    return hl_ok();
}

static gsx_error hl_destroy(gsx_loss_t loss)
{
    if(loss == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "loss must be non-null");
    }
    gsx_loss_base_deinit(loss);
    free(loss);
    return hl_ok();
}

static gsx_error hl_create_context(gsx_loss_t loss, gsx_loss_context_t *out_context)
{
    hip_loss_context *c = NULL;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(out_context == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_context must be non-null");
    }
    *out_context = NULL;
    c = (hip_loss_context *)calloc(1, sizeof(*c));
    if(c == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip loss context");
    }
    error = gsx_loss_context_base_init(&c->base, &hip_loss_context_iface, loss);
    if(!gsx_error_is_success(error)) {
        free(c);
        return error;
    }
    *out_context = &c->base;
    return hl_ok();
}

static gsx_error hlc_destroy(gsx_loss_context_t context)
{
    hip_loss_context *c = (hip_loss_context *)context;

    if(context == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "context must be non-null");
    }
    if(c->workspace != NULL) {
        (void)gsx_hip_pool_free(c->workspace, gsx_hip_plugin_stream(context->loss->backend));
    }
    gsx_loss_context_base_deinit(&c->base);
    free(c);
    return hl_ok();
}

static gsx_error hl_require_f32_device(gsx_backend_t backend, gsx_tensor_t t)
{
    if(t == NULL || t->data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip loss tensors must use float32 storage");
    }
    if(!gsx_hip_plugin_tensor_on_device(backend, t)) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "hip loss tensors must be device-backed");
    }
    return hl_ok();
}

/* [outer, C, H, W] of an image tensor in CHW storage */
static gsx_error hl_ssim_layout(gsx_tensor_t t, int64_t *outer, int32_t *c, int32_t *h, int32_t *w)
{
    if(t->storage_format != GSX_STORAGE_FORMAT_CHW) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip ssim supports CHW storage only");
    }
    if(t->rank == 3) {
        *outer = 1;
        *c = t->shape[0];
        *h = t->shape[1];
        *w = t->shape[2];
    } else if(t->rank == 4) {
        *outer = t->shape[0];
        *c = t->shape[1];
        *h = t->shape[2];
        *w = t->shape[3];
    } else {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "ssim expects [C,H,W] or [B,C,H,W] tensors");
    }
    return hl_ok();
}

static gsx_error hl_forward(gsx_loss_t loss, gsx_loss_context_t context, const gsx_loss_forward_request *request)
{
    hip_loss_context *c = (hip_loss_context *)context;
    gsx_backend_t backend = loss->backend;
    hipStream_t stream = gsx_hip_plugin_stream(backend);
    gsx_size_t n = 0;
    gsx_hip_status st = GSX_HIP_SUCCESS;
    gsx_error e = { GSX_ERROR_SUCCESS, NULL };

    e = hl_require_f32_device(backend, request->prediction);
    if(gsx_error_is_success(e)) e = hl_require_f32_device(backend, request->target);
    if(gsx_error_is_success(e)) e = hl_require_f32_device(backend, request->loss_map_accumulator);
    if(!gsx_error_is_success(e)) return e;
    n = request->prediction->size_bytes / sizeof(float);
    if(n == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "hip loss tensors must contain at least one element");
    }
    switch(loss->algorithm) {
    case GSX_LOSS_ALGORITHM_L1:
        st = gsx_hip_loss_l1_f32_forward_kernel_launch(gsx_hip_plugin_tensor_f32(request->loss_map_accumulator),
            gsx_hip_plugin_tensor_f32(request->prediction), gsx_hip_plugin_tensor_f32(request->target), (int64_t)n,
            request->scale, stream);
        break;
    case GSX_LOSS_ALGORITHM_MSE:
        st = gsx_hip_loss_mse_f32_forward_kernel_launch(gsx_hip_plugin_tensor_f32(request->loss_map_accumulator),
            gsx_hip_plugin_tensor_f32(request->prediction), gsx_hip_plugin_tensor_f32(request->target), (int64_t)n,
            request->scale, stream);
        break;
    case GSX_LOSS_ALGORITHM_SSIM: {
        int64_t outer = 0;
        int32_t ch = 0, h = 0, w = 0;

        e = hl_ssim_layout(request->prediction, &outer, &ch, &h, &w);
        if(!gsx_error_is_success(e)) return e;
        if(request->train && c->workspace_floats < 3 * n) {
            if(c->workspace != NULL) {
                (void)gsx_hip_pool_free(c->workspace, stream);
                c->workspace = NULL;
                c->workspace_floats = 0;
            }
            st = gsx_hip_pool_malloc((void **)&c->workspace, (size_t)(3 * n) * sizeof(float), stream);
            if(st != GSX_HIP_SUCCESS) {
                return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "hip ssim workspace allocation failed");
            }
            c->workspace_floats = 3 * n;
        }
        st = gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(gsx_hip_plugin_tensor_f32(request->loss_map_accumulator),
            gsx_hip_plugin_tensor_f32(request->prediction), gsx_hip_plugin_tensor_f32(request->target), outer, ch, h,
            w, request->scale, request->train ? c->workspace : NULL, 0.0f, 0, stream);
        break;
    }
    default:
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "loss algorithm is out of range");
    }
    if(st != GSX_HIP_SUCCESS) {
        return gsx_hip_plugin_error(st, "hip loss forward failed");
    }
    return hl_ok();
}

static gsx_error hl_backward(gsx_loss_t loss, gsx_loss_context_t context, const gsx_loss_backward_request *request)
{
    hip_loss_context *c = (hip_loss_context *)context;
    gsx_backend_t backend = loss->backend;
    hipStream_t stream = gsx_hip_plugin_stream(backend);
    gsx_tensor_t pred = context->retained_prediction, target = context->retained_target;
    gsx_size_t n = 0;
    float grad_scale = 0.0f;
    gsx_hip_status st = GSX_HIP_SUCCESS;
    gsx_error e = { GSX_ERROR_SUCCESS, NULL };

    e = hl_require_f32_device(backend, pred);
    if(gsx_error_is_success(e)) e = hl_require_f32_device(backend, target);
    if(gsx_error_is_success(e)) e = hl_require_f32_device(backend, request->grad_prediction_accumulator);
    if(!gsx_error_is_success(e)) return e;
    n = pred->size_bytes / sizeof(float);
    if(n == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "hip loss tensors must contain at least one element");
    }
    grad_scale = gsx_loss_scale_grad(loss, n, request->scale);
    switch(loss->algorithm) {
    case GSX_LOSS_ALGORITHM_L1:
        st = gsx_hip_loss_l1_f32_backward_kernel_launch(gsx_hip_plugin_tensor_f32(request->grad_prediction_accumulator),
            gsx_hip_plugin_tensor_f32(pred), gsx_hip_plugin_tensor_f32(target), (int64_t)n, grad_scale, stream);
        break;
    case GSX_LOSS_ALGORITHM_MSE:
        st = gsx_hip_loss_mse_f32_backward_kernel_launch(gsx_hip_plugin_tensor_f32(request->grad_prediction_accumulator),
            gsx_hip_plugin_tensor_f32(pred), gsx_hip_plugin_tensor_f32(target), (int64_t)n, grad_scale, stream);
        break;
    case GSX_LOSS_ALGORITHM_SSIM: {
        int64_t outer = 0;
        int32_t ch = 0, h = 0, w = 0;

        e = hl_ssim_layout(pred, &outer, &ch, &h, &w);
        if(!gsx_error_is_success(e)) return e;
        if(c->workspace == NULL || c->workspace_floats < 3 * n) {
            return gsx_make_error(GSX_ERROR_INVALID_STATE, "hip ssim backward requires a train forward on the context");
        }
        st = gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(
            gsx_hip_plugin_tensor_f32(request->grad_prediction_accumulator), gsx_hip_plugin_tensor_f32(pred),
            gsx_hip_plugin_tensor_f32(target), outer, ch, h, w, grad_scale, c->workspace, 0.0f, 0, stream);
        break;
    }
    default:
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "loss algorithm is out of range");
    }
    if(st != GSX_HIP_SUCCESS) {
        return gsx_hip_plugin_error(st, "hip loss backward failed");
    }
    return hl_ok();
}
