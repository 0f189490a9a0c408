/*
 * ref_driver.c - a thin driver over gsx's PUBLIC C API, linked against the unmodified
 * gsx core + CPU backend compiled from the reference sources (see oracle/Makefile).
 *
 * TEST INFRASTRUCTURE ONLY. It is loaded by tests/ and by bench.py's cpu_baseline leg
 * (ctypes, host memory in and out) and never by the product path.
 *
 * Every entry point takes plain host arrays, uploads them into CPU-backend tensors, runs
 * the reference code path through the public front-ends, and downloads the results:
 *   - gsxref_render       gsx_renderer_render          (gsx/src/gsx-render.c:799-826)
 *   - gsxref_render_grad  TRAIN render + gsx_renderer_backward (gsx-render.c:828-854)
 *   - gsxref_loss         gsx_loss_forward / gsx_loss_backward (gsx/src/gsx-loss.c)
 *   - gsxref_adam         gsx_optim_step               (gsx/src/gsx-optim.c:498)
 *   - gsxref_adc          gsx_adc_step                 (gsx/src/gsx-adc.c:231)
 *   - gsxref_train_step   one image-fit style step (render, L1+SSIM, backward, Adam) with
 *                         per-stage wall-clock timings, used as the CPU baseline; the render
 *                         backward can be skipped (Adam then steps on zero gradients) to time
 *                         the other stages on scenes whose backward exceeds the CPU backend's
 *                         int32 scratch limit.
 *   - gsxref_reduce / gsxref_elementwise / gsxref_gather / gsxref_random / gsxref_image
 *                         the tensor, random and image operations of gsx-core.h, gsx-random.h
 *                         and extra/gsx-image.h.
 * gsxref_use_backend selects the backend the entry points run on: the CPU backend, or the
 * registry's GPU slot in a build linked with the HIP backend plugin (libgsxref_hip.so).
 * Return value: 0 on success, otherwise the gsx_error_code; gsxref_last_error() gives the
 * reference's static message.
 */
#define _POSIX_C_SOURCE 200809L
#include "gsx/gsx.h"
#include "gsx/gsx-random.h"
#include "gsx/extra/gsx-image.h"
#ifdef GSXREF_HIP_TYPE
#include "gsx_hip_type.h" /* HIP as a backend type of its own (libgsxref_hiptype.so) */
#endif

#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static const char *g_last_message = NULL;

static double now_seconds(void);

/* Optional callback after each ADC step of gsxref_adc: the step's index and its wall-clock
 * seconds, the major stream drained before and after the step (NULL: no hook, no drains). */
typedef void (*gsxref_step_hook)(int step, double seconds);
static gsxref_step_hook g_step_hook = NULL;

void gsxref_set_step_hook(gsxref_step_hook hook) { g_step_hook = hook; }
/* One backend per registry slot, created on first use; gsxref_use_backend picks the slot the
 * entry points below run on (the CPU backend unless told otherwise). */
static gsx_backend_t g_backends[3] = { NULL, NULL, NULL };
static gsx_backend_buffer_type_t g_device_types[3] = { NULL, NULL, NULL };
static int g_which = 0;
static gsx_backend_t g_backend = NULL;
static gsx_backend_buffer_type_t g_device_type = NULL;

const char *gsxref_last_error(void) { return g_last_message != NULL ? g_last_message : ""; }

#define TRY(expr)                                                   \
    do {                                                            \
        gsx_error e_ = (expr);                                      \
        if(!gsx_error_is_success(e_)) {                             \
            g_last_message = e_.message;                            \
            rc = (int)e_.code != 0 ? (int)e_.code : -1;             \
            goto done;                                              \
        }                                                           \
    } while(0)

/* Downloads are asynchronous on a GPU backend's major stream (gsx-backend.h:114): every entry
 * point drains it before the caller reads its host arrays. */
#define FINISH() do { if(g_backend != NULL) (void)gsx_backend_major_stream_sync(g_backend); } while(0)

static int ensure_backend(void)
{
#ifdef GSX_BACKEND_TYPE_HIP
    /* built with gsx_hip_type.h: slot 2 is the HIP backend type of its own */
    static const gsx_backend_type types[3] = { GSX_BACKEND_TYPE_CPU, GSX_BACKEND_TYPE_CUDA, GSX_BACKEND_TYPE_HIP };
#else
    static const gsx_backend_type types[3] = { GSX_BACKEND_TYPE_CPU, GSX_BACKEND_TYPE_CUDA, GSX_BACKEND_TYPE_METAL };
#endif
    gsx_backend_device_t device = NULL;
    gsx_backend_desc desc = { 0 };
    gsx_error e;

    if(g_backends[g_which] == NULL) {
        e = gsx_backend_registry_init();
        if(!gsx_error_is_success(e)) { g_last_message = e.message; return (int)e.code; }
        e = gsx_get_backend_device_by_type(types[g_which], 0, &device);
        if(!gsx_error_is_success(e)) { g_last_message = e.message; return (int)e.code; }
        desc.device = device;
        e = gsx_backend_init(&g_backends[g_which], &desc);
        if(!gsx_error_is_success(e)) { g_last_message = e.message; return (int)e.code; }
        e = gsx_backend_find_buffer_type(g_backends[g_which], GSX_BACKEND_BUFFER_TYPE_DEVICE, &g_device_types[g_which]);
        if(!gsx_error_is_success(e)) { g_last_message = e.message; return (int)e.code; }
    }
    g_backend = g_backends[g_which];
    g_device_type = g_device_types[g_which];
    return 0;
}

/* which: 0 the CPU backend, 1 the registry's GPU slot (GSX_BACKEND_TYPE_CUDA: in a build linked
 * with the HIP backend plugin, the MI355X backend registers there), 2 GSX_BACKEND_TYPE_HIP (only
 * in a build with gsx_hip_type.h, where the plugin registers under that type). */
int gsxref_use_backend(int which)
{
#ifdef GSX_BACKEND_TYPE_HIP
    if(which < 0 || which > 2) return (int)GSX_ERROR_OUT_OF_RANGE;
#else
    if(which < 0 || which > 1) return (int)GSX_ERROR_OUT_OF_RANGE;
#endif
    g_which = which;
    return ensure_backend();
}

/* Number of registered devices of a backend type (gsx_count_backend_devices_by_type), or a
 * negative gsx error code. */
int gsxref_count_devices(int backend_type)
{
    gsx_index_t count = 0;
    gsx_error e = gsx_backend_registry_init();

    if(!gsx_error_is_success(e)) { g_last_message = e.message; return -(int)e.code; }
    e = gsx_count_backend_devices_by_type((gsx_backend_type)backend_type, &count);
    if(!gsx_error_is_success(e)) { g_last_message = e.message; return -(int)e.code; }
    return (int)count;
}

/* Backend type and family name of the device the selected backend runs on. */
int gsxref_backend_type(void)
{
    gsx_backend_info info;
    gsx_backend_device_info dinfo;

    if(ensure_backend() != 0) return -1;
    if(!gsx_error_is_success(gsx_backend_get_info(g_backend, &info))) return -1;
    if(!gsx_error_is_success(gsx_backend_device_get_info(info.device, &dinfo))) return -1;
    return (int)dinfo.backend_type;
}

const char *gsxref_backend_family_name(void)
{
    gsx_backend_info info;
    gsx_backend_device_info dinfo;

    if(ensure_backend() != 0) return "";
    if(!gsx_error_is_success(gsx_backend_get_info(g_backend, &info))) return "";
    if(!gsx_error_is_success(gsx_backend_device_get_info(info.device, &dinfo))) return "";
    return dinfo.backend_name != NULL ? dinfo.backend_name : "";
}

/* Name of the device the selected backend runs on. */
const char *gsxref_backend_device_name(void)
{
    gsx_backend_info info;
    gsx_backend_device_info dinfo;

    if(ensure_backend() != 0) return "";
    if(!gsx_error_is_success(gsx_backend_get_info(g_backend, &info))) return "";
    if(!gsx_error_is_success(gsx_backend_device_get_info(info.device, &dinfo))) return "";
    return dinfo.name;
}

static gsx_error make_tensor(gsx_arena_t arena, gsx_tensor_t *out, int rank, int d0, int d1, int d2, const void *src)
{
    gsx_tensor_desc desc = { 0 };
    gsx_error e;

    desc.rank = rank;
    desc.shape[0] = d0;
    desc.shape[1] = d1;
    desc.shape[2] = d2;
    desc.data_type = GSX_DATA_TYPE_F32;
    desc.storage_format = GSX_STORAGE_FORMAT_CHW;
    desc.arena = arena;
    e = gsx_tensor_init(out, &desc);
    if(!gsx_error_is_success(e)) {
        return e;
    }
    if(src != NULL) {
        size_t count = (size_t)d0 * (size_t)(rank > 1 ? d1 : 1) * (size_t)(rank > 2 ? d2 : 1);
        return gsx_tensor_upload(*out, src, count * sizeof(float));
    }
    return gsx_tensor_set_zero(*out);
}

/* camera[17] = fx, fy, cx, cy, width, height, qx, qy, qz, qw, tx, ty, tz, near, far, bg_r, bg_g, bg_b
 * (18 floats; width/height are carried as floats holding integers). */
static void unpack_camera(const float *camera, gsx_camera_intrinsics *intr, gsx_camera_pose *pose,
    float *near_plane, float *far_plane, gsx_vec3 *bg)
{
    memset(intr, 0, sizeof(*intr));
    memset(pose, 0, sizeof(*pose));
    intr->model = GSX_CAMERA_MODEL_PINHOLE;
    intr->fx = camera[0];
    intr->fy = camera[1];
    intr->cx = camera[2];
    intr->cy = camera[3];
    intr->width = (gsx_index_t)camera[4];
    intr->height = (gsx_index_t)camera[5];
    pose->rot.x = camera[6];
    pose->rot.y = camera[7];
    pose->rot.z = camera[8];
    pose->rot.w = camera[9];
    pose->transl.x = camera[10];
    pose->transl.y = camera[11];
    pose->transl.z = camera[12];
    *near_plane = camera[13];
    *far_plane = camera[14];
    bg->x = camera[15];
    bg->y = camera[16];
    bg->z = camera[17];
}

typedef struct ref_scene {
    gsx_arena_t arena;
    gsx_tensor_t mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3;
} ref_scene;

static gsx_error scene_upload(ref_scene *s, int n, gsx_size_t extra_bytes, int sh_degree, const float *mean3d, const float *rotation,
    const float *logscale, const float *opacity, const float *sh0, const float *sh1, const float *sh2, const float *sh3)
{
    gsx_arena_desc adesc = { 0 };
    gsx_error e;

    memset(s, 0, sizeof(*s));
    adesc.initial_capacity_bytes = (gsx_size_t)n * 512u + extra_bytes + 65536u;
    e = gsx_arena_init(&s->arena, g_device_type, &adesc);
    if(!gsx_error_is_success(e)) return e;
    e = make_tensor(s->arena, &s->mean3d, 2, n, 3, 0, mean3d);
    if(!gsx_error_is_success(e)) return e;
    e = make_tensor(s->arena, &s->rotation, 2, n, 4, 0, rotation);
    if(!gsx_error_is_success(e)) return e;
    e = make_tensor(s->arena, &s->logscale, 2, n, 3, 0, logscale);
    if(!gsx_error_is_success(e)) return e;
    e = make_tensor(s->arena, &s->opacity, 1, n, 0, 0, opacity);
    if(!gsx_error_is_success(e)) return e;
    e = make_tensor(s->arena, &s->sh0, 2, n, 3, 0, sh0);
    if(!gsx_error_is_success(e)) return e;
    if(sh_degree >= 1) {
        e = make_tensor(s->arena, &s->sh1, 3, n, 3, 3, sh1);
        if(!gsx_error_is_success(e)) return e;
    }
    if(sh_degree >= 2) {
        e = make_tensor(s->arena, &s->sh2, 3, n, 5, 3, sh2);
        if(!gsx_error_is_success(e)) return e;
    }
    if(sh_degree >= 3) {
        e = make_tensor(s->arena, &s->sh3, 3, n, 7, 3, sh3);
        if(!gsx_error_is_success(e)) return e;
    }
    {
        gsx_error ok = { GSX_ERROR_SUCCESS, NULL };
        return ok;
    }
}

static void scene_free(ref_scene *s)
{
    gsx_tensor_t *all[] = { &s->mean3d, &s->rotation, &s->logscale, &s->opacity, &s->sh0, &s->sh1, &s->sh2, &s->sh3 };
    size_t i;

    for(i = 0; i < sizeof(all) / sizeof(all[0]); ++i) {
        if(*all[i] != NULL) {
            (void)gsx_tensor_free(*all[i]);
            *all[i] = NULL;
        }
    }
    if(s->arena != NULL) {
        (void)gsx_arena_free(s->arena);
        s->arena = NULL;
    }
}

/* Forward render. forward_type: 0 inference, 1 train. visible_counter (nullable, [n]) is
 * read, bound as gs_visible_counter for TRAIN forwards, and written back. */
int gsxref_render(int n, int sh_degree, const float *mean3d, const float *rotation, const float *logscale,
    const float *opacity, const float *sh0, const float *sh1, const float *sh2, const float *sh3,
    const float *camera, int forward_type, float *out_rgb, float *visible_counter)
{
    int rc = 0;
    ref_scene s = { 0 };
    gsx_renderer_t renderer = NULL;
    gsx_render_context_t context = NULL;
    gsx_renderer_desc rdesc = { 0 };
    gsx_render_forward_request req = { 0 };
    gsx_camera_intrinsics intr;
    gsx_camera_pose pose;
    gsx_tensor_t out = NULL;
    gsx_tensor_t counter = NULL;
    float near_plane = 0.0f;
    float far_plane = 0.0f;
    gsx_vec3 bg;

    rc = ensure_backend();
    if(rc != 0) return rc;
    unpack_camera(camera, &intr, &pose, &near_plane, &far_plane, &bg);
    TRY(scene_upload(&s, n, (gsx_size_t)intr.width * (gsx_size_t)intr.height * 64u, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3));
    TRY(make_tensor(s.arena, &out, 3, 3, intr.height, intr.width, NULL));
    if(visible_counter != NULL) {
        TRY(make_tensor(s.arena, &counter, 1, n, 0, 0, visible_counter));
    }
    rdesc.width = intr.width;
    rdesc.height = intr.height;
    rdesc.output_data_type = GSX_DATA_TYPE_F32;
    TRY(gsx_renderer_init(&renderer, g_backend, &rdesc));
    TRY(gsx_render_context_init(&context, renderer));
    req.intrinsics = &intr;
    req.pose = &pose;
    req.near_plane = near_plane;
    req.far_plane = far_plane;
    req.background_color = bg;
    req.precision = GSX_RENDER_PRECISION_FLOAT32;
    req.sh_degree = sh_degree;
    req.forward_type = forward_type != 0 ? GSX_RENDER_FORWARD_TYPE_TRAIN : GSX_RENDER_FORWARD_TYPE_INFERENCE;
    req.borrow_train_state = true;
    req.gs_mean3d = s.mean3d;
    req.gs_rotation = s.rotation;
    req.gs_logscale = s.logscale;
    req.gs_opacity = s.opacity;
    req.gs_sh0 = s.sh0;
    req.gs_sh1 = s.sh1;
    req.gs_sh2 = s.sh2;
    req.gs_sh3 = s.sh3;
    req.out_rgb = out;
    req.gs_visible_counter = counter;
    TRY(gsx_renderer_render(renderer, context, &req));
    TRY(gsx_tensor_download(out, out_rgb, (gsx_size_t)3 * intr.height * intr.width * sizeof(float)));
    if(counter != NULL) {
        TRY(gsx_tensor_download(counter, visible_counter, (gsx_size_t)n * sizeof(float)));
    }
done:
    FINISH();
    if(context != NULL) (void)gsx_render_context_free(context);
    if(renderer != NULL) (void)gsx_renderer_free(renderer);
    if(out != NULL) (void)gsx_tensor_free(out);
    if(counter != NULL) (void)gsx_tensor_free(counter);
    scene_free(&s);
    return rc;
}

/* TRAIN forward + backward. grads: mean3d [n,3], rotation [n,4], logscale [n,3], opacity [n],
 * sh0 [n,3], sh1..sh3 per sh_degree (nullable otherwise). Sinks are overwritten, as in the
 * reference (gsx-cpu/render.c:1537-1550). out_rgb receives the forward image. */
int gsxref_render_grad(int n, int sh_degree, const float *mean3d, const float *rotation, const float *logscale,
    const float *opacity, const float *sh0, const float *sh1, const float *sh2, const float *sh3,
    const float *camera, const float *grad_rgb, float *out_rgb,
    float *g_mean3d, float *g_rotation, float *g_logscale, float *g_opacity, float *g_sh0,
    float *g_sh1, float *g_sh2, float *g_sh3)
{
    int rc = 0;
    ref_scene s = { 0 };
    gsx_renderer_t renderer = NULL;
    gsx_render_context_t context = NULL;
    gsx_renderer_desc rdesc = { 0 };
    gsx_render_forward_request req = { 0 };
    gsx_render_backward_request breq = { 0 };
    gsx_camera_intrinsics intr;
    gsx_camera_pose pose;
    gsx_tensor_t out = NULL, gout = NULL;
    gsx_tensor_t gm = NULL, gr = NULL, gl = NULL, go = NULL, gs0 = NULL, gs1 = NULL, gs2 = NULL, gs3 = NULL;
    float near_plane = 0.0f;
    float far_plane = 0.0f;
    gsx_vec3 bg;
    gsx_size_t img_bytes;

    rc = ensure_backend();
    if(rc != 0) return rc;
    unpack_camera(camera, &intr, &pose, &near_plane, &far_plane, &bg);
    img_bytes = (gsx_size_t)3 * intr.height * intr.width * sizeof(float);
    TRY(scene_upload(&s, n, (gsx_size_t)intr.width * (gsx_size_t)intr.height * 64u, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3));
    TRY(make_tensor(s.arena, &out, 3, 3, intr.height, intr.width, NULL));
    TRY(make_tensor(s.arena, &gout, 3, 3, intr.height, intr.width, grad_rgb));
    TRY(make_tensor(s.arena, &gm, 2, n, 3, 0, NULL));
    TRY(make_tensor(s.arena, &gr, 2, n, 4, 0, NULL));
    TRY(make_tensor(s.arena, &gl, 2, n, 3, 0, NULL));
    TRY(make_tensor(s.arena, &go, 1, n, 0, 0, NULL));
    TRY(make_tensor(s.arena, &gs0, 2, n, 3, 0, NULL));
    if(sh_degree >= 1) TRY(make_tensor(s.arena, &gs1, 3, n, 3, 3, NULL));
    if(sh_degree >= 2) TRY(make_tensor(s.arena, &gs2, 3, n, 5, 3, NULL));
    if(sh_degree >= 3) TRY(make_tensor(s.arena, &gs3, 3, n, 7, 3, NULL));
    rdesc.width = intr.width;
    rdesc.height = intr.height;
    rdesc.output_data_type = GSX_DATA_TYPE_F32;
    TRY(gsx_renderer_init(&renderer, g_backend, &rdesc));
    TRY(gsx_render_context_init(&context, renderer));
    req.intrinsics = &intr;
    req.pose = &pose;
    req.near_plane = near_plane;
    req.far_plane = far_plane;
    req.background_color = bg;
    req.precision = GSX_RENDER_PRECISION_FLOAT32;
    req.sh_degree = sh_degree;
    req.forward_type = GSX_RENDER_FORWARD_TYPE_TRAIN;
    req.borrow_train_state = true;
    req.gs_mean3d = s.mean3d;
    req.gs_rotation = s.rotation;
    req.gs_logscale = s.logscale;
    req.gs_opacity = s.opacity;
    req.gs_sh0 = s.sh0;
    req.gs_sh1 = s.sh1;
    req.gs_sh2 = s.sh2;
    req.gs_sh3 = s.sh3;
    req.out_rgb = out;
    TRY(gsx_renderer_render(renderer, context, &req));
    breq.grad_rgb = gout;
    breq.grad_gs_mean3d = gm;
    breq.grad_gs_rotation = gr;
    breq.grad_gs_logscale = gl;
    breq.grad_gs_opacity = go;
    breq.grad_gs_sh0 = gs0;
    breq.grad_gs_sh1 = gs1;
    breq.grad_gs_sh2 = gs2;
    breq.grad_gs_sh3 = gs3;
    TRY(gsx_renderer_backward(renderer, context, &breq));
    TRY(gsx_tensor_download(out, out_rgb, img_bytes));
    TRY(gsx_tensor_download(gm, g_mean3d, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_tensor_download(gr, g_rotation, (gsx_size_t)n * 4u * sizeof(float)));
    TRY(gsx_tensor_download(gl, g_logscale, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_tensor_download(go, g_opacity, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_tensor_download(gs0, g_sh0, (gsx_size_t)n * 3u * sizeof(float)));
    if(gs1 != NULL) TRY(gsx_tensor_download(gs1, g_sh1, (gsx_size_t)n * 9u * sizeof(float)));
    if(gs2 != NULL) TRY(gsx_tensor_download(gs2, g_sh2, (gsx_size_t)n * 15u * sizeof(float)));
    if(gs3 != NULL) TRY(gsx_tensor_download(gs3, g_sh3, (gsx_size_t)n * 21u * sizeof(float)));
done:
    FINISH();
    if(context != NULL) (void)gsx_render_context_free(context);
    if(renderer != NULL) (void)gsx_renderer_free(renderer);
    {
        gsx_tensor_t all[] = { out, gout, gm, gr, gl, go, gs0, gs1, gs2, gs3 };
        size_t i;
        for(i = 0; i < sizeof(all) / sizeof(all[0]); ++i) {
            if(all[i] != NULL) (void)gsx_tensor_free(all[i]);
        }
    }
    scene_free(&s);
    return rc;
}

/* Loss forward then backward on [outer, C, H, W] CHW images.
 * algorithm: 0 L1, 1 MSE, 2 SSIM (gsx_loss_algorithm). grad_norm: 0 MEAN, 1 SUM.
 * loss_map and grad are accumulators: read, accumulated into, written back. grad may be NULL
 * to skip the backward. */
int gsxref_loss(int algorithm, int grad_norm, int outer, int channels, int height, int width,
    const float *prediction, const float *target, float scale, float *loss_map, float *grad)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_desc desc = { 0 };
    gsx_tensor_t pred = NULL, tgt = NULL, map = NULL, g = NULL;
    gsx_loss_t loss = NULL;
    gsx_loss_context_t context = NULL;
    gsx_loss_desc ldesc = { 0 };
    gsx_loss_forward_request freq = { 0 };
    gsx_loss_backward_request breq = { 0 };
    gsx_size_t bytes = (gsx_size_t)outer * channels * height * width * sizeof(float);

    rc = ensure_backend();
    if(rc != 0) return rc;
    adesc.initial_capacity_bytes = bytes * 4u + 4096u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    desc.rank = outer > 1 ? 4 : 3;
    if(outer > 1) {
        desc.shape[0] = outer; desc.shape[1] = channels; desc.shape[2] = height; desc.shape[3] = width;
    } else {
        desc.shape[0] = channels; desc.shape[1] = height; desc.shape[2] = width;
    }
    desc.data_type = GSX_DATA_TYPE_F32;
    desc.storage_format = GSX_STORAGE_FORMAT_CHW;
    desc.arena = arena;
    TRY(gsx_tensor_init(&pred, &desc));
    TRY(gsx_tensor_init(&tgt, &desc));
    TRY(gsx_tensor_init(&map, &desc));
    TRY(gsx_tensor_init(&g, &desc));
    TRY(gsx_tensor_upload(pred, prediction, bytes));
    TRY(gsx_tensor_upload(tgt, target, bytes));
    TRY(gsx_tensor_upload(map, loss_map, bytes));
    if(grad != NULL) TRY(gsx_tensor_upload(g, grad, bytes));
    ldesc.algorithm = (gsx_loss_algorithm)algorithm;
    ldesc.grad_normalization = (gsx_loss_grad_normalization_type)grad_norm;
    TRY(gsx_loss_init(&loss, g_backend, &ldesc));
    TRY(gsx_loss_context_init(&context, loss));
    freq.prediction = pred;
    freq.target = tgt;
    freq.loss_map_accumulator = map;
    freq.train = grad != NULL;
    freq.scale = scale;
    TRY(gsx_loss_forward(loss, context, &freq));
    if(grad != NULL) {
        breq.grad_prediction_accumulator = g;
        breq.scale = scale;
        TRY(gsx_loss_backward(loss, context, &breq));
        TRY(gsx_tensor_download(g, grad, bytes));
    }
    TRY(gsx_tensor_download(map, loss_map, bytes));
done:
    FINISH();
    if(context != NULL) (void)gsx_loss_context_free(context);
    if(loss != NULL) (void)gsx_loss_free(loss);
    if(pred != NULL) (void)gsx_tensor_free(pred);
    if(tgt != NULL) (void)gsx_tensor_free(tgt);
    if(map != NULL) (void)gsx_tensor_free(map);
    if(g != NULL) (void)gsx_tensor_free(g);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* Adam over one parameter group of `count` floats for `steps` steps, with the same gradient
 * each step. hyper[6] = lr, beta1, beta2, weight_decay, epsilon, max_grad.
 * param is updated in place; m and v receive the final moments. */
int gsxref_adam(int count, int steps, float *param, const float *grad, const float *hyper, float *m, float *v)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t p = NULL, g = NULL;
    gsx_optim_t optim = NULL;
    gsx_optim_desc odesc = { 0 };
    gsx_optim_param_group_desc group = { 0 };
    gsx_optim_step_request sreq = { 0 };
    int i;

    (void)m;
    (void)v;
    rc = ensure_backend();
    if(rc != 0) return rc;
    adesc.initial_capacity_bytes = (gsx_size_t)count * 16u + 4096u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    TRY(make_tensor(arena, &p, 1, count, 0, 0, param));
    TRY(make_tensor(arena, &g, 1, count, 0, 0, grad));
    group.role = GSX_OPTIM_PARAM_ROLE_MEAN3D;
    group.label = "p";
    group.parameter = p;
    group.gradient = g;
    group.learning_rate = hyper[0];
    group.beta1 = hyper[1];
    group.beta2 = hyper[2];
    group.weight_decay = hyper[3];
    group.epsilon = hyper[4];
    group.max_grad = hyper[5];
    odesc.algorithm = GSX_OPTIM_ALGORITHM_ADAM;
    odesc.param_groups = &group;
    odesc.param_group_count = 1;
    TRY(gsx_optim_init(&optim, g_backend, &odesc));
    sreq.force_all = true;
    for(i = 0; i < steps; ++i) {
        TRY(gsx_optim_step(optim, &sreq));
    }
    TRY(gsx_tensor_download(p, param, (gsx_size_t)count * sizeof(float)));
done:
    FINISH();
    if(optim != NULL) (void)gsx_optim_free(optim);
    if(p != NULL) (void)gsx_tensor_free(p);
    if(g != NULL) (void)gsx_tensor_free(g);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* One Adam step of every group on gradients filled with pcg32 normals (seeded `seed`). */
static gsx_error adam_probe_step(gsx_gs_t gs, gsx_optim_t optim, uint64_t seed)
{
    const gsx_gs_field grads[5] = { GSX_GS_FIELD_GRAD_MEAN3D, GSX_GS_FIELD_GRAD_LOGSCALE, GSX_GS_FIELD_GRAD_ROTATION,
        GSX_GS_FIELD_GRAD_OPACITY, GSX_GS_FIELD_GRAD_SH0 };
    gsx_optim_step_request sreq = { 0 };
    gsx_pcg32_t pcg = NULL;
    gsx_tensor_t t = NULL;
    gsx_error e;
    int k;

    e = gsx_pcg32_init(&pcg, (gsx_pcg32_state_t)seed);
    if(!gsx_error_is_success(e)) return e;
    for(k = 0; k < 5; ++k) {
        e = gsx_gs_get_field(gs, grads[k], &t);
        if(gsx_error_is_success(e)) e = gsx_pcg32_fill_randn(pcg, t, 0.01f);
        if(!gsx_error_is_success(e)) {
            (void)gsx_pcg32_free(pcg);
            return e;
        }
    }
    (void)gsx_pcg32_free(pcg);
    sreq.force_all = true;
    return gsx_optim_step(optim, &sreq);
}

/* ADC steps (DEFAULT, ABSGS or MCMC) on a Gaussian set with SH0 only and an Adam optimizer over
 * the 5 built-in roles. params[10] = pruning_opacity_threshold, opacity_clamp_value,
 * max_world_scale, max_screen_scale, duplicate_grad_threshold, duplicate_scale_threshold,
 * duplicate_absgrad_threshold, scene_scale, noise_strength, grow_ratio.
 * iparams[10] = algorithm, refine_every, start_refine, end_refine, max_num_gaussians,
 * reset_every, global_step, seed, step_count (consecutive global steps from global_step; 0 or 1:
 * one), optim_probe (non-zero: one Adam step on pcg32 normal gradients before the ADC steps and
 * one after, so the rows' optimizer moments show in the returned parameters).
 * In: n rows of mean3d/rotation/logscale/opacity/sh0 + grad_acc, absgrad_acc, visible_counter.
 * Out: *out_n rows written to out_* (capacity out_capacity rows); counters[4] = pruned,
 * duplicated, grown, reset, summed over the steps. */
int gsxref_adc(int n, const float *mean3d, const float *rotation, const float *logscale, const float *opacity,
    const float *sh0, const float *grad_acc, const float *absgrad_acc, const float *visible_counter,
    const float *params, const int64_t *iparams, int out_capacity, int *out_n,
    float *o_mean3d, float *o_rotation, float *o_logscale, float *o_opacity, float *o_sh0, int64_t *counters)
{
    int rc = 0;
    gsx_gs_t gs = NULL;
    gsx_gs_desc gdesc = { 0 };
    gsx_tensor_t t = NULL;
    gsx_adc_t adc = NULL;
    gsx_adc_desc adesc = { 0 };
    gsx_adc_request areq = { 0 };
    gsx_adc_result ares = { 0 };
    gsx_optim_t optim = NULL;
    gsx_optim_desc odesc = { 0 };
    gsx_optim_param_group_desc groups[5];
    gsx_gs_info info = { 0 };
    gsx_renderer_t adc_renderer = NULL;
    const gsx_gs_field fields[5] = { GSX_GS_FIELD_MEAN3D, GSX_GS_FIELD_LOGSCALE, GSX_GS_FIELD_ROTATION,
        GSX_GS_FIELD_OPACITY, GSX_GS_FIELD_SH0 };
    const gsx_gs_field grad_fields[5] = { GSX_GS_FIELD_GRAD_MEAN3D, GSX_GS_FIELD_GRAD_LOGSCALE,
        GSX_GS_FIELD_GRAD_ROTATION, GSX_GS_FIELD_GRAD_OPACITY, GSX_GS_FIELD_GRAD_SH0 };
    const gsx_optim_param_role roles[5] = { GSX_OPTIM_PARAM_ROLE_MEAN3D, GSX_OPTIM_PARAM_ROLE_LOGSCALE,
        GSX_OPTIM_PARAM_ROLE_ROTATION, GSX_OPTIM_PARAM_ROLE_OPACITY, GSX_OPTIM_PARAM_ROLE_SH0 };
    int k;

    rc = ensure_backend();
    if(rc != 0) return rc;
    gdesc.buffer_type = g_device_type;
    gdesc.count = (gsx_size_t)n;
    gdesc.aux_flags = GSX_GS_AUX_VISIBLE_COUNTER | GSX_GS_AUX_GRAD_ACC | GSX_GS_AUX_ABSGRAD_ACC;
    TRY(gsx_gs_init(&gs, &gdesc));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &t));
    TRY(gsx_tensor_upload(t, mean3d, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &t));
    TRY(gsx_tensor_upload(t, rotation, (gsx_size_t)n * 4u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &t));
    TRY(gsx_tensor_upload(t, logscale, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &t));
    TRY(gsx_tensor_upload(t, opacity, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &t));
    TRY(gsx_tensor_upload(t, sh0, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_GRAD_ACC, &t));
    TRY(gsx_tensor_upload(t, grad_acc, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ABSGRAD_ACC, &t));
    TRY(gsx_tensor_upload(t, absgrad_acc, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_VISIBLE_COUNTER, &t));
    TRY(gsx_tensor_upload(t, visible_counter, (gsx_size_t)n * sizeof(float)));

    memset(groups, 0, sizeof(groups));
    for(k = 0; k < 5; ++k) {
        TRY(gsx_gs_get_field(gs, fields[k], &groups[k].parameter));
        TRY(gsx_gs_get_field(gs, grad_fields[k], &groups[k].gradient));
        groups[k].role = roles[k];
        groups[k].label = "g";
        groups[k].learning_rate = 1e-3f;
        groups[k].beta1 = 0.9f;
        groups[k].beta2 = 0.999f;
        groups[k].epsilon = 1e-8f;
    }
    odesc.algorithm = GSX_OPTIM_ALGORITHM_ADAM;
    odesc.param_groups = groups;
    odesc.param_group_count = 5;
    TRY(gsx_optim_init(&optim, g_backend, &odesc));

    adesc.algorithm = (gsx_adc_algorithm)iparams[0];
    adesc.pruning_opacity_threshold = params[0];
    adesc.opacity_clamp_value = params[1];
    adesc.max_world_scale = params[2];
    adesc.max_screen_scale = params[3];
    adesc.duplicate_grad_threshold = params[4];
    adesc.duplicate_scale_threshold = params[5];
    adesc.duplicate_absgrad_threshold = params[6];
    adesc.refine_every = (gsx_index_t)iparams[1];
    adesc.start_refine = (gsx_index_t)iparams[2];
    adesc.end_refine = (gsx_index_t)iparams[3];
    adesc.max_num_gaussians = (gsx_index_t)iparams[4];
    adesc.reset_every = (gsx_index_t)iparams[5];
    adesc.seed = (gsx_size_t)iparams[7];
    adesc.noise_strength = params[8];
    adesc.grow_ratio = params[9];
    TRY(gsx_adc_init(&adc, g_backend, &adesc));
    areq.gs = gs;
    areq.optim = optim;
    /* default/ABSGS never use the dataloader; the reference's own ADC tests pass a placeholder
     * the same way (tests/adc_runtime.cpp:457). The renderer must belong to the backend. */
    {
        gsx_renderer_desc rdesc = { 0 };

        rdesc.width = 1;
        rdesc.height = 1;
        rdesc.output_data_type = GSX_DATA_TYPE_F32;
        TRY(gsx_renderer_init(&adc_renderer, g_backend, &rdesc));
    }
    areq.dataloader = (gsx_dataloader_t)0x1;
    areq.renderer = adc_renderer;
    areq.scene_scale = params[7];
    if(iparams[9] != 0) TRY(adam_probe_step(gs, optim, 101u));
    counters[0] = counters[1] = counters[2] = counters[3] = 0;
    for(k = 0; k < (iparams[8] > 1 ? (int)iparams[8] : 1); ++k) {
        double t0 = 0.0;

        areq.global_step = (gsx_size_t)iparams[6] + (gsx_size_t)k;
        if(g_step_hook != NULL) {
            FINISH();
            t0 = now_seconds();
        }
        TRY(gsx_adc_step(adc, &areq, &ares));
        if(g_step_hook != NULL) {
            FINISH();
            g_step_hook(k, now_seconds() - t0);
        }
        counters[0] += (int64_t)ares.pruned_count;
        counters[1] += (int64_t)ares.duplicated_count;
        counters[2] += (int64_t)ares.grown_count;
        counters[3] += (int64_t)ares.reset_count;
    }
    if(iparams[9] != 0) TRY(adam_probe_step(gs, optim, 202u));
    TRY(gsx_gs_get_info(gs, &info));
    *out_n = (int)info.count;
    if((int)info.count > out_capacity) {
        g_last_message = "adc output exceeds out_capacity";
        rc = -2;
        goto done;
    }
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &t));
    TRY(gsx_tensor_download(t, o_mean3d, info.count * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &t));
    TRY(gsx_tensor_download(t, o_rotation, info.count * 4u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &t));
    TRY(gsx_tensor_download(t, o_logscale, info.count * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &t));
    TRY(gsx_tensor_download(t, o_opacity, info.count * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &t));
    TRY(gsx_tensor_download(t, o_sh0, info.count * 3u * sizeof(float)));
done:
    FINISH();
    if(adc_renderer != NULL) (void)gsx_renderer_free(adc_renderer);
    if(adc != NULL) (void)gsx_adc_free(adc);
    if(optim != NULL) (void)gsx_optim_free(optim);
    if(gs != NULL) (void)gsx_gs_free(gs);
    return rc;
}

static double now_seconds(void)
{
    struct timespec ts;

    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* `iters` image-fit style training steps on one camera: TRAIN render, L1 (scale w_l1) and
 * SSIM (scale w_ssim) forward + backward, render backward, Adam over the 5 SH0 roles.
 * hyper[2] = lr_mean3d, lr_other. stage_seconds[5] accumulates render fwd, loss fwd,
 * loss bwd, render bwd, Adam (wall clock, single thread). The scene arrays are updated. */
int gsxref_train_step(int n, int iters, float *mean3d, float *rotation, float *logscale, float *opacity,
    float *sh0, const float *camera, const float *target_rgb, float w_l1, float w_ssim, const float *hyper,
    int skip_render_backward, double *stage_seconds)
{
    int rc = 0;
    gsx_gs_t gs = NULL;
    gsx_gs_desc gdesc = { 0 };
    gsx_tensor_t t = NULL;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t out = NULL, tgt = NULL, map = NULL, gout = NULL;
    gsx_renderer_t renderer = NULL;
    gsx_render_context_t rctx = NULL;
    gsx_renderer_desc rdesc = { 0 };
    gsx_loss_t l1 = NULL, ssim = NULL;
    gsx_loss_context_t l1ctx = NULL, ssimctx = NULL;
    gsx_loss_desc ldesc = { 0 };
    gsx_optim_t optim = NULL;
    gsx_optim_desc odesc = { 0 };
    gsx_optim_param_group_desc groups[5];
    gsx_optim_step_request sreq = { 0 };
    gsx_camera_intrinsics intr;
    gsx_camera_pose pose;
    float near_plane, far_plane;
    gsx_vec3 bg;
    gsx_size_t img_bytes;
    const gsx_gs_field fields[5] = { GSX_GS_FIELD_MEAN3D, GSX_GS_FIELD_LOGSCALE, GSX_GS_FIELD_ROTATION,
        GSX_GS_FIELD_OPACITY, GSX_GS_FIELD_SH0 };
    const gsx_gs_field grad_fields[5] = { GSX_GS_FIELD_GRAD_MEAN3D, GSX_GS_FIELD_GRAD_LOGSCALE,
        GSX_GS_FIELD_GRAD_ROTATION, GSX_GS_FIELD_GRAD_OPACITY, GSX_GS_FIELD_GRAD_SH0 };
    const gsx_optim_param_role roles[5] = { GSX_OPTIM_PARAM_ROLE_MEAN3D, GSX_OPTIM_PARAM_ROLE_LOGSCALE,
        GSX_OPTIM_PARAM_ROLE_ROTATION, GSX_OPTIM_PARAM_ROLE_OPACITY, GSX_OPTIM_PARAM_ROLE_SH0 };
    int k, it;

    rc = ensure_backend();
    if(rc != 0) return rc;
    unpack_camera(camera, &intr, &pose, &near_plane, &far_plane, &bg);
    img_bytes = (gsx_size_t)3 * intr.height * intr.width * sizeof(float);
    gdesc.buffer_type = g_device_type;
    gdesc.count = (gsx_size_t)n;
    gdesc.aux_flags = GSX_GS_AUX_NONE;
    TRY(gsx_gs_init(&gs, &gdesc));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &t));
    TRY(gsx_tensor_upload(t, mean3d, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &t));
    TRY(gsx_tensor_upload(t, rotation, (gsx_size_t)n * 4u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &t));
    TRY(gsx_tensor_upload(t, logscale, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &t));
    TRY(gsx_tensor_upload(t, opacity, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &t));
    TRY(gsx_tensor_upload(t, sh0, (gsx_size_t)n * 3u * sizeof(float)));
    adesc.initial_capacity_bytes = img_bytes * 4u + 4096u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    TRY(make_tensor(arena, &out, 3, 3, intr.height, intr.width, NULL));
    TRY(make_tensor(arena, &tgt, 3, 3, intr.height, intr.width, target_rgb));
    TRY(make_tensor(arena, &map, 3, 3, intr.height, intr.width, NULL));
    TRY(make_tensor(arena, &gout, 3, 3, intr.height, intr.width, NULL));
    rdesc.width = intr.width;
    rdesc.height = intr.height;
    rdesc.output_data_type = GSX_DATA_TYPE_F32;
    TRY(gsx_renderer_init(&renderer, g_backend, &rdesc));
    TRY(gsx_render_context_init(&rctx, renderer));
    ldesc.grad_normalization = GSX_LOSS_GRAD_NORMALIZATION_TYPE_MEAN;
    ldesc.algorithm = GSX_LOSS_ALGORITHM_L1;
    TRY(gsx_loss_init(&l1, g_backend, &ldesc));
    TRY(gsx_loss_context_init(&l1ctx, l1));
    ldesc.algorithm = GSX_LOSS_ALGORITHM_SSIM;
    TRY(gsx_loss_init(&ssim, g_backend, &ldesc));
    TRY(gsx_loss_context_init(&ssimctx, ssim));
    memset(groups, 0, sizeof(groups));
    for(k = 0; k < 5; ++k) {
        TRY(gsx_gs_get_field(gs, fields[k], &groups[k].parameter));
        TRY(gsx_gs_get_field(gs, grad_fields[k], &groups[k].gradient));
        groups[k].role = roles[k];
        groups[k].label = "g";
        groups[k].learning_rate = k == 0 ? hyper[0] : hyper[1];
        groups[k].beta1 = 0.9f;
        groups[k].beta2 = 0.999f;
        groups[k].epsilon = 1e-8f;
    }
    odesc.algorithm = GSX_OPTIM_ALGORITHM_ADAM;
    odesc.param_groups = groups;
    odesc.param_group_count = 5;
    TRY(gsx_optim_init(&optim, g_backend, &odesc));
    sreq.force_all = true;
    for(it = 0; it < iters; ++it) {
        gsx_render_forward_request req = { 0 };
        gsx_render_backward_request breq = { 0 };
        gsx_loss_forward_request lf = { 0 };
        gsx_loss_backward_request lb = { 0 };
        double t0, t1, t2, t3, t4, t5;

        TRY(gsx_tensor_set_zero(map));
        TRY(gsx_tensor_set_zero(gout));
        TRY(gsx_gs_zero_gradients(gs));
        req.intrinsics = &intr;
        req.pose = &pose;
        req.near_plane = near_plane;
        req.far_plane = far_plane;
        req.background_color = bg;
        req.precision = GSX_RENDER_PRECISION_FLOAT32;
        req.sh_degree = 0;
        req.forward_type = GSX_RENDER_FORWARD_TYPE_TRAIN;
        req.borrow_train_state = true;
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &req.gs_mean3d));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &req.gs_rotation));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &req.gs_logscale));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &req.gs_opacity));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &req.gs_sh0));
        req.out_rgb = out;
        t0 = now_seconds();
        TRY(gsx_renderer_render(renderer, rctx, &req));
        t1 = now_seconds();
        lf.prediction = out;
        lf.target = tgt;
        lf.loss_map_accumulator = map;
        lf.train = true;
        lf.scale = w_l1;
        TRY(gsx_loss_forward(l1, l1ctx, &lf));
        lf.scale = w_ssim;
        TRY(gsx_loss_forward(ssim, ssimctx, &lf));
        t2 = now_seconds();
        lb.grad_prediction_accumulator = gout;
        lb.scale = w_l1;
        TRY(gsx_loss_backward(l1, l1ctx, &lb));
        lb.scale = w_ssim;
        TRY(gsx_loss_backward(ssim, ssimctx, &lb));
        t3 = now_seconds();
        breq.grad_rgb = gout;
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_GRAD_MEAN3D, &breq.grad_gs_mean3d));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_GRAD_ROTATION, &breq.grad_gs_rotation));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_GRAD_LOGSCALE, &breq.grad_gs_logscale));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_GRAD_OPACITY, &breq.grad_gs_opacity));
        TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_GRAD_SH0, &breq.grad_gs_sh0));
        if(!skip_render_backward) TRY(gsx_renderer_backward(renderer, rctx, &breq));
        t4 = now_seconds();
        TRY(gsx_optim_step(optim, &sreq));
        t5 = now_seconds();
        stage_seconds[0] += t1 - t0;
        stage_seconds[1] += t2 - t1;
        stage_seconds[2] += t3 - t2;
        stage_seconds[3] += t4 - t3;
        stage_seconds[4] += t5 - t4;
    }
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &t));
    TRY(gsx_tensor_download(t, mean3d, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &t));
    TRY(gsx_tensor_download(t, rotation, (gsx_size_t)n * 4u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &t));
    TRY(gsx_tensor_download(t, logscale, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &t));
    TRY(gsx_tensor_download(t, opacity, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &t));
    TRY(gsx_tensor_download(t, sh0, (gsx_size_t)n * 3u * sizeof(float)));
done:
    FINISH();
    if(optim != NULL) (void)gsx_optim_free(optim);
    if(l1ctx != NULL) (void)gsx_loss_context_free(l1ctx);
    if(ssimctx != NULL) (void)gsx_loss_context_free(ssimctx);
    if(l1 != NULL) (void)gsx_loss_free(l1);
    if(ssim != NULL) (void)gsx_loss_free(ssim);
    if(rctx != NULL) (void)gsx_render_context_free(rctx);
    if(renderer != NULL) (void)gsx_renderer_free(renderer);
    {
        gsx_tensor_t all[] = { out, tgt, map, gout };
        size_t i;
        for(i = 0; i < sizeof(all) / sizeof(all[0]); ++i) {
            if(all[i] != NULL) (void)gsx_tensor_free(all[i]);
        }
    }
    if(arena != NULL) (void)gsx_arena_free(arena);
    if(gs != NULL) (void)gsx_gs_free(gs);
    return rc;
}

/* ---- tensor operations through gsx's public API (gsx-core.h:221-270, gsx-random.h,
 * extra/gsx-image.h), on the selected backend: the buffer-vtable operations a backend supplies
 * (gsx-impl.h:302-458) run on byte-identical inputs on both backends. ---------------------------- */

static gsx_error make_typed(gsx_arena_t arena, gsx_tensor_t *out, int rank, const int *shape, gsx_data_type dt,
    gsx_storage_format fmt, const void *src, size_t bytes)
{
    gsx_tensor_desc desc = { 0 };
    gsx_error e;
    int d;

    desc.rank = rank;
    for(d = 0; d < rank; ++d) desc.shape[d] = shape[d];
    desc.data_type = dt;
    desc.storage_format = fmt;
    desc.arena = arena;
    e = gsx_tensor_init(out, &desc);
    if(!gsx_error_is_success(e)) return e;
    if(src != NULL) return gsx_tensor_upload(*out, src, bytes);
    return gsx_tensor_set_zero(*out);
}

static size_t shape_count(int rank, const int *shape)
{
    size_t n = 1;
    int d;

    for(d = 0; d < rank; ++d) n *= (size_t)shape[d];
    return n;
}

/* op: 0 sum, 1 mean, 2 max (of x), 3 mse, 4 mae (of x - y) over axes [start_axis, rank);
 * out has the leading extents. */
int gsxref_reduce(int op, int rank, const int *shape, int start_axis, const float *x, const float *y, float *out)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t tx = NULL, ty = NULL, to = NULL;
    /* the output keeps the leading extents and one unit axis (gsx-core.c:1503-1530) */
    int out_shape[4] = { 1, 1, 1, 1 };
    int out_rank = start_axis + 1;
    size_t n = shape_count(rank, shape);
    size_t n_out = 1;
    int d;

    rc = ensure_backend();
    if(rc != 0) return rc;
    for(d = 0; d < start_axis; ++d) {
        out_shape[d] = shape[d];
        n_out *= (size_t)shape[d];
    }
    adesc.initial_capacity_bytes = (gsx_size_t)(2 * n + n_out) * 4u + 65536u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    TRY(make_typed(arena, &tx, rank, shape, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, x, n * 4));
    if(op >= 3) TRY(make_typed(arena, &ty, rank, shape, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, y, n * 4));
    TRY(make_typed(arena, &to, out_rank, out_shape, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, NULL, 0));
    {
        /* the reduce front-ends take a workspace arena of the same backend */
        gsx_arena_t ws = NULL;
        gsx_arena_desc wdesc = { 0 };

        wdesc.initial_capacity_bytes = (gsx_size_t)n * 8u + 65536u;
        TRY(gsx_arena_init(&ws, g_device_type, &wdesc));
        gsx_error re = { GSX_ERROR_OUT_OF_RANGE, "unknown reduce op" };

        switch(op) {
        case 0: re = gsx_tensor_sum(ws, tx, to, start_axis); break;
        case 1: re = gsx_tensor_mean(ws, tx, to, start_axis); break;
        case 2: re = gsx_tensor_max(ws, tx, to, start_axis); break;
        case 3: re = gsx_tensor_mse(ws, tx, ty, to, start_axis); break;
        case 4: re = gsx_tensor_mae(ws, tx, ty, to, start_axis); break;
        default: break;
        }
        if(!gsx_error_is_success(re)) {
            g_last_message = re.message;
            rc = (int)re.code;
        }
        FINISH();
        (void)gsx_arena_free(ws);
        if(rc != 0) goto done;
    }
    TRY(gsx_tensor_download(to, out, n_out * 4));
done:
    FINISH();
    if(tx != NULL) (void)gsx_tensor_free(tx);
    if(ty != NULL) (void)gsx_tensor_free(ty);
    if(to != NULL) (void)gsx_tensor_free(to);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* op: 0 exp, 1 sigmoid, 2 sigmoid', 3 abs (out = f(x), or in place when inplace != 0);
 * 4 clamp in place to [params[0], params[1]]; 5 check_finite (out[0] = 1 when all finite). */
int gsxref_elementwise(int op, int inplace, int count, const float *x, const float *params, float *out)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t tx = NULL, to = NULL;
    int shape[1];

    rc = ensure_backend();
    if(rc != 0) return rc;
    shape[0] = count;
    adesc.initial_capacity_bytes = (gsx_size_t)count * 8u + 65536u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    TRY(make_typed(arena, &tx, 1, shape, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, x, (size_t)count * 4));
    if(op <= 3 && !inplace) {
        TRY(make_typed(arena, &to, 1, shape, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, NULL, 0));
        switch(op) {
        case 0: TRY(gsx_tensor_exp(tx, to)); break;
        case 1: TRY(gsx_tensor_sigmoid(tx, to)); break;
        case 2: TRY(gsx_tensor_sigmoid_derivative(tx, to)); break;
        default: TRY(gsx_tensor_abs(tx, to)); break;
        }
        TRY(gsx_tensor_download(to, out, (size_t)count * 4));
    } else if(op <= 4) {
        switch(op) {
        case 0: TRY(gsx_tensor_exp_inplace(tx)); break;
        case 1: TRY(gsx_tensor_sigmoid_inplace(tx)); break;
        case 2: TRY(gsx_tensor_sigmoid_derivative_inplace(tx)); break;
        case 3: TRY(gsx_tensor_abs_inplace(tx)); break;
        default: {
            float lo = params[0], hi = params[1];

            TRY(gsx_tensor_clamp_inplace(tx, &lo, &hi));
        }
        }
        TRY(gsx_tensor_download(tx, out, (size_t)count * 4));
    } else if(op == 5) {
        bool finite = false;

        TRY(gsx_tensor_check_finite(tx, &finite));
        out[0] = finite ? 1.0f : 0.0f;
    } else {
        rc = (int)GSX_ERROR_OUT_OF_RANGE;
    }
done:
    FINISH();
    if(tx != NULL) (void)gsx_tensor_free(tx);
    if(to != NULL) (void)gsx_tensor_free(to);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* out[r] = x[index[r]] for rows of `width` floats (gsx_tensor_gather). */
int gsxref_gather(int rows, int width, const float *x, int count, const int32_t *index, float *out)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t tx = NULL, ti = NULL, to = NULL;
    int xs[2], os[2], is[1];

    rc = ensure_backend();
    if(rc != 0) return rc;
    xs[0] = rows;
    xs[1] = width;
    os[0] = count;
    os[1] = width;
    is[0] = count;
    adesc.initial_capacity_bytes = (gsx_size_t)(rows + count) * (gsx_size_t)width * 4u + (gsx_size_t)count * 4u + 65536u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    TRY(make_typed(arena, &tx, 2, xs, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, x, (size_t)rows * width * 4));
    TRY(make_typed(arena, &ti, 1, is, GSX_DATA_TYPE_I32, GSX_STORAGE_FORMAT_CHW, index, (size_t)count * 4));
    TRY(make_typed(arena, &to, 2, os, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, NULL, 0));
    TRY(gsx_tensor_gather(tx, ti, to));
    TRY(gsx_tensor_download(to, out, (size_t)count * width * 4));
done:
    FINISH();
    if(tx != NULL) (void)gsx_tensor_free(tx);
    if(ti != NULL) (void)gsx_tensor_free(ti);
    if(to != NULL) (void)gsx_tensor_free(to);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* kind: 0 rand (float), 1 randn (float, sigma = param), 2 randint (int32, bound = (uint32)param),
 * 3 multinomial (int32 samples from cdf[categories]); pcg32 seeded with `seed`
 * (gsx_pcg32_init). out has `count` elements. */
int gsxref_random(int kind, uint64_t seed, int count, float param, const float *cdf, int categories, void *out)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t to = NULL, tc = NULL;
    gsx_pcg32_t pcg = NULL;
    int shape[1], cshape[1];

    rc = ensure_backend();
    if(rc != 0) return rc;
    shape[0] = count;
    cshape[0] = categories;
    adesc.initial_capacity_bytes = (gsx_size_t)count * 4u + (gsx_size_t)categories * 4u + 65536u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    TRY(gsx_pcg32_init(&pcg, (gsx_pcg32_state_t)seed));
    TRY(make_typed(arena, &to, 1, shape, kind >= 2 ? GSX_DATA_TYPE_I32 : GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW,
        NULL, 0));
    switch(kind) {
    case 0: TRY(gsx_pcg32_fill_rand(pcg, to)); break;
    case 1: TRY(gsx_pcg32_fill_randn(pcg, to, param)); break;
    case 2: TRY(gsx_pcg32_fill_randint(pcg, to, (uint32_t)param)); break;
    case 3:
        TRY(make_typed(arena, &tc, 1, cshape, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, cdf, (size_t)categories * 4));
        TRY(gsx_pcg32_multinomial(pcg, to, tc));
        break;
    default: rc = (int)GSX_ERROR_OUT_OF_RANGE; goto done;
    }
    TRY(gsx_tensor_download(to, out, (size_t)count * 4));
done:
    FINISH();
    if(pcg != NULL) (void)gsx_pcg32_free(pcg);
    if(to != NULL) (void)gsx_tensor_free(to);
    if(tc != NULL) (void)gsx_tensor_free(tc);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* kind: 0 linear -> sRGB, 1 sRGB -> linear (float32 CHW [3,h,w]); 2 HWC -> CHW, 3 CHW -> HWC
 * (float32, c channels); 4 float32 -> uint8, 5 uint8 -> float32 (CHW [c,h,w]). */
int gsxref_image(int kind, int c, int h, int w, const void *src, void *dst)
{
    int rc = 0;
    gsx_arena_t arena = NULL;
    gsx_arena_desc adesc = { 0 };
    gsx_tensor_t ts = NULL, td = NULL;
    int chw[3], hwc[3];
    size_t n = (size_t)c * h * w;

    rc = ensure_backend();
    if(rc != 0) return rc;
    chw[0] = c;
    chw[1] = h;
    chw[2] = w;
    hwc[0] = h;
    hwc[1] = w;
    hwc[2] = c;
    adesc.initial_capacity_bytes = (gsx_size_t)n * 8u + 65536u;
    TRY(gsx_arena_init(&arena, g_device_type, &adesc));
    switch(kind) {
    case 0:
    case 1:
        TRY(make_typed(arena, &ts, 3, chw, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, src, n * 4));
        TRY(make_typed(arena, &td, 3, chw, GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW, NULL, 0));
        TRY(gsx_tensor_image_convert_colorspace(td, kind == 0 ? GSX_IMAGE_COLOR_SPACE_SRGB : GSX_IMAGE_COLOR_SPACE_LINEAR,
            ts, kind == 0 ? GSX_IMAGE_COLOR_SPACE_LINEAR : GSX_IMAGE_COLOR_SPACE_SRGB));
        TRY(gsx_tensor_download(td, dst, n * 4));
        break;
    case 2:
    case 3:
        TRY(make_typed(arena, &ts, 3, kind == 2 ? hwc : chw, GSX_DATA_TYPE_F32,
            kind == 2 ? GSX_STORAGE_FORMAT_HWC : GSX_STORAGE_FORMAT_CHW, src, n * 4));
        TRY(make_typed(arena, &td, 3, kind == 2 ? chw : hwc, GSX_DATA_TYPE_F32,
            kind == 2 ? GSX_STORAGE_FORMAT_CHW : GSX_STORAGE_FORMAT_HWC, NULL, 0));
        TRY(gsx_tensor_image_convert_storage_format(td, ts));
        TRY(gsx_tensor_download(td, dst, n * 4));
        break;
    case 4:
    case 5:
        TRY(make_typed(arena, &ts, 3, chw, kind == 4 ? GSX_DATA_TYPE_F32 : GSX_DATA_TYPE_U8, GSX_STORAGE_FORMAT_CHW, src,
            n * (kind == 4 ? 4 : 1)));
        TRY(make_typed(arena, &td, 3, chw, kind == 4 ? GSX_DATA_TYPE_U8 : GSX_DATA_TYPE_F32, GSX_STORAGE_FORMAT_CHW,
            NULL, 0));
        TRY(gsx_tensor_image_convert_data_type(td, ts));
        TRY(gsx_tensor_download(td, dst, n * (kind == 4 ? 1 : 4)));
        break;
    default:
        rc = (int)GSX_ERROR_OUT_OF_RANGE;
        break;
    }
done:
    FINISH();
    if(ts != NULL) (void)gsx_tensor_free(ts);
    if(td != NULL) (void)gsx_tensor_free(td);
    if(arena != NULL) (void)gsx_arena_free(arena);
    return rc;
}

/* ---- dataloader (gsx-data.h) -------------------------------------------------------------------
 * A dataset of `count` host images, rgb [count, h, w, 3] HWC and optional alpha [count, h, w], of
 * u8 (is_u8) or float32 elements, iterated through gsx_dataloader on the selected backend:
 * prefetch > 0 turns on async prefetch with that depth (the backend's async loader), 0 the
 * synchronous path. `steps` results are downloaded: rgb CHW floats to out_rgb [steps, 3, h, w],
 * alpha to out_alpha [steps, h, w] (nullable), stable sample indices to out_index and epochs to
 * out_epoch; sample k's intrinsics carry fx = 100 + k so out_fx [steps] shows the pairing. */
typedef struct ref_images {
    int count, h, w, is_u8;
    const unsigned char *rgb, *alpha;
} ref_images;

static gsx_error ref_ok(void)
{
    gsx_error ok = { GSX_ERROR_SUCCESS, NULL };
    return ok;
}

static gsx_error ref_images_length(void *object, gsx_size_t *out_length)
{
    *out_length = (gsx_size_t)((ref_images *)object)->count;
    return ref_ok();
}

static gsx_error ref_images_sample(void *object, gsx_size_t index, gsx_dataset_cpu_sample *out)
{
    const ref_images *d = (const ref_images *)object;
    const size_t elem = d->is_u8 ? 1u : 4u;
    const size_t px = (size_t)d->h * (size_t)d->w;

    memset(out, 0, sizeof(*out));
    out->intrinsics.model = GSX_CAMERA_MODEL_PINHOLE;
    out->intrinsics.fx = 100.0f + (float)index;
    out->intrinsics.fy = 100.0f;
    out->intrinsics.cx = 0.5f * (float)d->w;
    out->intrinsics.cy = 0.5f * (float)d->h;
    out->intrinsics.width = d->w;
    out->intrinsics.height = d->h;
    out->pose.rot.w = 1.0f;
    out->rgb_data = d->rgb + index * px * 3u * elem;
    out->alpha_data = d->alpha != NULL ? d->alpha + index * px * elem : NULL;
    return ref_ok();
}

static void ref_images_release(void *object, gsx_dataset_cpu_sample *sample)
{
    (void)object;
    (void)sample;
}

int gsxref_dataloader(int count, int h, int w, int is_u8, const void *rgb, const void *alpha, int shuffle,
    uint64_t seed, int prefetch, int steps, float *out_rgb, float *out_alpha, int64_t *out_index, int64_t *out_epoch,
    float *out_fx)
{
    int rc = 0;
    ref_images images;
    gsx_dataset_desc ddesc = { 0 };
    gsx_dataset_t dataset = NULL;
    gsx_dataloader_desc ldesc = { 0 };
    gsx_dataloader_t loader = NULL;
    gsx_dataloader_result res;
    const size_t px = (size_t)h * (size_t)w;
    int s;

    rc = ensure_backend();
    if(rc != 0) return rc;
    images.count = count;
    images.h = h;
    images.w = w;
    images.is_u8 = is_u8;
    images.rgb = (const unsigned char *)rgb;
    images.alpha = (const unsigned char *)alpha;
    ddesc.name = "gsxref";
    ddesc.object = &images;
    ddesc.image_data_type = is_u8 ? GSX_DATA_TYPE_U8 : GSX_DATA_TYPE_F32;
    ddesc.width = w;
    ddesc.height = h;
    ddesc.has_rgb = true;
    ddesc.has_alpha = alpha != NULL;
    ddesc.get_length = ref_images_length;
    ddesc.get_sample = ref_images_sample;
    ddesc.release_sample = ref_images_release;
    TRY(gsx_dataset_init(&dataset, &ddesc));
    ldesc.shuffle_each_epoch = shuffle != 0;
    ldesc.enable_async_prefetch = prefetch > 0;
    ldesc.prefetch_count = prefetch > 0 ? (gsx_size_t)prefetch : 0u;
    ldesc.seed = (gsx_size_t)seed;
    ldesc.image_data_type = GSX_DATA_TYPE_F32;
    TRY(gsx_dataloader_init(&loader, g_backend, dataset, &ldesc));
    for(s = 0; s < steps; ++s) {
        TRY(gsx_dataloader_next_ex(loader, &res));
        TRY(gsx_tensor_download(res.rgb_image, out_rgb + (size_t)s * 3u * px, 3u * px * sizeof(float)));
        if(out_alpha != NULL && res.alpha_image != NULL) {
            TRY(gsx_tensor_download(res.alpha_image, out_alpha + (size_t)s * px, px * sizeof(float)));
        }
        FINISH();
        out_index[s] = (int64_t)res.stable_sample_index;
        out_epoch[s] = (int64_t)res.epoch_index;
        out_fx[s] = res.intrinsics.fx;
    }
done:
    FINISH();
    if(loader != NULL) (void)gsx_dataloader_free(loader);
    if(dataset != NULL) (void)gsx_dataset_free(dataset);
    return rc;
}

/* ---- the session path (gsx-runtime.h: gsx_session_step) -------------------------------------
 * `warmup` + `iters` steps of gsx_session_step on the selected backend, configured as
 * image-fit-demo configures its session (apps/image_fit_demo.c:1286-1330): a one-image dataset
 * served by gsx_dataloader (async prefetch of depth `prefetch` when > 0), L1 (w_l1) + SSIM
 * (w_ssim) loss items, Adam over the five SH0 roles (hyper[0] mean3d, hyper[1] the others),
 * borrowed train state, SH degree 0, no ADC, session-owned device workspace, and per-stage
 * timings collected only when collect_timings is set (each timed stage then synchronises,
 * gsx-runtime.c:629-684). target_hwc is the image as the dataset hands it over: [h, w, 3]
 * float32. out_seconds[0] = wall-clock seconds of the `iters` timed steps (the major stream is
 * drained before and after); out_stage_us[8] = the last step's report timings (dataloader,
 * render fwd, loss fwd, loss bwd, render bwd, optim, adc, total), zeros without timings. The
 * scene arrays are updated with the trained values. */
typedef struct ref_one_image {
    const float *camera;
    const float *rgb;
} ref_one_image;

static gsx_error ref_one_length(void *object, gsx_size_t *out_length)
{
    (void)object;
    *out_length = 1u;
    return ref_ok();
}

static gsx_error ref_one_sample(void *object, gsx_size_t index, gsx_dataset_cpu_sample *out)
{
    const ref_one_image *d = (const ref_one_image *)object;
    float near_plane, far_plane;
    gsx_vec3 bg;

    (void)index;
    memset(out, 0, sizeof(*out));
    unpack_camera(d->camera, &out->intrinsics, &out->pose, &near_plane, &far_plane, &bg);
    out->rgb_data = d->rgb;
    out->alpha_data = NULL;
    return ref_ok();
}

int gsxref_session_fit(int n, int warmup, int iters, float *mean3d, float *rotation, float *logscale, float *opacity,
    float *sh0, const float *camera, const float *target_hwc, float w_l1, float w_ssim, const float *hyper,
    int collect_timings, int prefetch, double *out_seconds, double *out_stage_us)
{
    int rc = 0;
    gsx_gs_t gs = NULL;
    gsx_gs_desc gdesc = { 0 };
    gsx_tensor_t t = NULL;
    gsx_renderer_t renderer = NULL;
    gsx_renderer_desc rdesc = { 0 };
    gsx_loss_t l1 = NULL, ssim = NULL;
    gsx_loss_context_t l1ctx = NULL, ssimctx = NULL;
    gsx_loss_desc ldesc = { 0 };
    gsx_optim_t optim = NULL;
    gsx_optim_desc odesc = { 0 };
    gsx_optim_param_group_desc groups[5];
    gsx_dataset_desc ddesc = { 0 };
    gsx_dataset_t dataset = NULL;
    gsx_dataloader_desc dl = { 0 };
    gsx_dataloader_t loader = NULL;
    gsx_session_desc sdesc;
    gsx_session_t session = NULL;
    gsx_loss_item items[2];
    gsx_session_step_report report;
    ref_one_image image;
    gsx_camera_intrinsics intr;
    gsx_camera_pose pose;
    float near_plane, far_plane;
    gsx_vec3 bg;
    const gsx_gs_field fields[5] = { GSX_GS_FIELD_MEAN3D, GSX_GS_FIELD_LOGSCALE, GSX_GS_FIELD_ROTATION,
        GSX_GS_FIELD_OPACITY, GSX_GS_FIELD_SH0 };
    const gsx_gs_field grad_fields[5] = { GSX_GS_FIELD_GRAD_MEAN3D, GSX_GS_FIELD_GRAD_LOGSCALE,
        GSX_GS_FIELD_GRAD_ROTATION, GSX_GS_FIELD_GRAD_OPACITY, GSX_GS_FIELD_GRAD_SH0 };
    const gsx_optim_param_role roles[5] = { GSX_OPTIM_PARAM_ROLE_MEAN3D, GSX_OPTIM_PARAM_ROLE_LOGSCALE,
        GSX_OPTIM_PARAM_ROLE_ROTATION, GSX_OPTIM_PARAM_ROLE_OPACITY, GSX_OPTIM_PARAM_ROLE_SH0 };
    double t0;
    int k, it;

    out_seconds[0] = 0.0;
    for(k = 0; k < 8; ++k) out_stage_us[k] = 0.0;
    rc = ensure_backend();
    if(rc != 0) return rc;
    unpack_camera(camera, &intr, &pose, &near_plane, &far_plane, &bg);
    gdesc.buffer_type = g_device_type;
    gdesc.count = (gsx_size_t)n;
    gdesc.aux_flags = GSX_GS_AUX_NONE;
    TRY(gsx_gs_init(&gs, &gdesc));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &t));
    TRY(gsx_tensor_upload(t, mean3d, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &t));
    TRY(gsx_tensor_upload(t, rotation, (gsx_size_t)n * 4u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &t));
    TRY(gsx_tensor_upload(t, logscale, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &t));
    TRY(gsx_tensor_upload(t, opacity, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &t));
    TRY(gsx_tensor_upload(t, sh0, (gsx_size_t)n * 3u * sizeof(float)));
    rdesc.width = intr.width;
    rdesc.height = intr.height;
    rdesc.output_data_type = GSX_DATA_TYPE_F32;
    TRY(gsx_renderer_init(&renderer, g_backend, &rdesc));
    ldesc.grad_normalization = GSX_LOSS_GRAD_NORMALIZATION_TYPE_MEAN;
    ldesc.algorithm = GSX_LOSS_ALGORITHM_L1;
    TRY(gsx_loss_init(&l1, g_backend, &ldesc));
    TRY(gsx_loss_context_init(&l1ctx, l1));
    ldesc.algorithm = GSX_LOSS_ALGORITHM_SSIM;
    TRY(gsx_loss_init(&ssim, g_backend, &ldesc));
    TRY(gsx_loss_context_init(&ssimctx, ssim));
    memset(groups, 0, sizeof(groups));
    for(k = 0; k < 5; ++k) {
        TRY(gsx_gs_get_field(gs, fields[k], &groups[k].parameter));
        TRY(gsx_gs_get_field(gs, grad_fields[k], &groups[k].gradient));
        groups[k].role = roles[k];
        groups[k].label = "g";
        groups[k].learning_rate = k == 0 ? hyper[0] : hyper[1];
        groups[k].beta1 = 0.9f;
        groups[k].beta2 = 0.999f;
        groups[k].epsilon = 1e-8f;
    }
    odesc.algorithm = GSX_OPTIM_ALGORITHM_ADAM;
    odesc.param_groups = groups;
    odesc.param_group_count = 5;
    TRY(gsx_optim_init(&optim, g_backend, &odesc));
    image.camera = camera;
    image.rgb = target_hwc;
    ddesc.name = "gsxref-session";
    ddesc.object = &image;
    ddesc.image_data_type = GSX_DATA_TYPE_F32;
    ddesc.width = intr.width;
    ddesc.height = intr.height;
    ddesc.has_rgb = true;
    ddesc.has_alpha = false;
    ddesc.get_length = ref_one_length;
    ddesc.get_sample = ref_one_sample;
    ddesc.release_sample = ref_images_release;
    TRY(gsx_dataset_init(&dataset, &ddesc));
    dl.shuffle_each_epoch = false;
    dl.enable_async_prefetch = prefetch > 0;
    dl.prefetch_count = prefetch > 0 ? (gsx_size_t)prefetch : 0u;
    dl.image_data_type = GSX_DATA_TYPE_F32;
    TRY(gsx_dataloader_init(&loader, g_backend, dataset, &dl));
    items[0].loss = l1;
    items[0].context = l1ctx;
    items[0].scale = w_l1;
    items[1].loss = ssim;
    items[1].context = ssimctx;
    items[1].scale = w_ssim;
    memset(&sdesc, 0, sizeof(sdesc));
    sdesc.backend = g_backend;
    sdesc.gs = gs;
    sdesc.optim = optim;
    sdesc.renderer = renderer;
    sdesc.train_dataloader = loader;
    sdesc.loss_count = 2;
    sdesc.loss_items = items;
    sdesc.render.near_plane = near_plane;
    sdesc.render.far_plane = far_plane;
    sdesc.render.background_color = bg;
    sdesc.render.precision = GSX_RENDER_PRECISION_FLOAT32;
    sdesc.render.sh_degree_mode = GSX_SESSION_SH_DEGREE_MODE_EXPLICIT;
    sdesc.render.sh_degree = 0;
    sdesc.render.borrow_train_state = true;
    sdesc.optim_step.force_all = true;
    sdesc.adc_step.enabled = false;
    sdesc.workspace.buffer_type_class = GSX_BACKEND_BUFFER_TYPE_DEVICE;
    sdesc.workspace.auto_plan = true;
    sdesc.reporting.collect_timings = collect_timings != 0;
    TRY(gsx_session_init(&session, &sdesc));
    for(it = 0; it < warmup; ++it) TRY(gsx_session_step(session));
    FINISH();
    t0 = now_seconds();
    for(it = 0; it < iters; ++it) TRY(gsx_session_step(session));
    FINISH();
    out_seconds[0] = now_seconds() - t0;
    memset(&report, 0, sizeof(report));
    TRY(gsx_session_get_last_step_report(session, &report));
    out_stage_us[0] = report.timings.dataloader_us;
    out_stage_us[1] = report.timings.render_forward_us;
    out_stage_us[2] = report.timings.loss_forward_us;
    out_stage_us[3] = report.timings.loss_backward_us;
    out_stage_us[4] = report.timings.render_backward_us;
    out_stage_us[5] = report.timings.optim_step_us;
    out_stage_us[6] = report.timings.adc_step_us;
    out_stage_us[7] = report.timings.total_step_us;
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_MEAN3D, &t));
    TRY(gsx_tensor_download(t, mean3d, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_ROTATION, &t));
    TRY(gsx_tensor_download(t, rotation, (gsx_size_t)n * 4u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_LOGSCALE, &t));
    TRY(gsx_tensor_download(t, logscale, (gsx_size_t)n * 3u * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_OPACITY, &t));
    TRY(gsx_tensor_download(t, opacity, (gsx_size_t)n * sizeof(float)));
    TRY(gsx_gs_get_field(gs, GSX_GS_FIELD_SH0, &t));
    TRY(gsx_tensor_download(t, sh0, (gsx_size_t)n * 3u * sizeof(float)));
done:
    FINISH();
    if(session != NULL) (void)gsx_session_free(session);
    if(loader != NULL) (void)gsx_dataloader_free(loader);
    if(dataset != NULL) (void)gsx_dataset_free(dataset);
    if(optim != NULL) (void)gsx_optim_free(optim);
    if(l1ctx != NULL) (void)gsx_loss_context_free(l1ctx);
    if(ssimctx != NULL) (void)gsx_loss_context_free(ssimctx);
    if(l1 != NULL) (void)gsx_loss_free(l1);
    if(ssim != NULL) (void)gsx_loss_free(ssim);
    if(renderer != NULL) (void)gsx_renderer_free(renderer);
    if(gs != NULL) (void)gsx_gs_free(gs);
    return rc;
}
