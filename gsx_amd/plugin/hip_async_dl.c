/*
 * hip_async_dl.c - the async dataloader of the gsx HIP backend (the gsx_async_dl_i entry of
 * gsx/src/gsx-impl.h:524-529; counterpart of gsx/src/gsx-cuda/async_dl.cu and the CPU
 * backend's gsx-cpu/async_dl.cpp).
 *
 * One helper thread per loader fetches samples through the dataset callbacks, copies each
 * payload into page-locked staging owned by the destination slot, and enqueues on a helper
 * stream: the DMA into a device staging buffer, then the layout kernel that writes the slot's CHW
 * float tensors (gsx_hip_dataloader_to_chw_f32, values kept as gsx-data-impl.h:173-268 packs
 * them). Streams are ordered by events, not by host synchronisation:
 *   - submit (caller's thread) records slot_free[s] on the major stream, so the helper stream
 *     writes slot s only after every kernel queued before the slot came back has run;
 *   - the helper records slot_ready[s] after the layout kernel, and wait() makes the major stream
 *     wait for it before returning the slot, so the consumer's kernels see the finished image;
 *   - before reusing slot s's staging the helper thread waits on the host for slot_ready[s] of
 *     the slot's previous load (long complete in steady state).
 * Requests complete in submission order (one helper thread, one FIFO), which gsx's dataloader
 * checks (gsx-data.c:994-996). A failure is kept and returned by the next submit or wait.
 */
#define _POSIX_C_SOURCE 200809L
#include "hip_backend.h"
#include "gsx-data-impl.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct hip_dl_slot {
    void *host;          /* page-locked staging: rgb | alpha | invdepth payloads */
    void *device;        /* device staging of the same bytes */
    gsx_size_t rgb_bytes, alpha_bytes, invdepth_bytes;
    hipEvent_t free_ev;  /* the major stream is done with the slot */
    hipEvent_t ready_ev; /* the slot's tensors hold the loaded sample */
} hip_dl_slot;

typedef struct hip_dl_request {
    gsx_size_t stable_sample_index;
    gsx_size_t slot_index;
} hip_dl_request;

typedef struct hip_async_dl {
    struct gsx_async_dl base;
    gsx_backend_t backend;
    gsx_async_dl_desc desc;
    int32_t ordinal;
    hipStream_t stream;
    hip_dl_slot *slots;
    /* FIFO rings, each with room for every slot */
    hip_dl_request *requests;
    gsx_async_dl_ready_item *ready;
    gsx_size_t req_head, req_count, ready_head, ready_count;
    gsx_size_t inflight;
    pthread_mutex_t mutex;
    pthread_cond_t cond;
    pthread_t worker;
    bool worker_started;
    bool closed;
    bool failed;
    gsx_error failure;
} hip_async_dl;

static gsx_error hdl_ok(void) { return gsx_make_error(GSX_ERROR_SUCCESS, NULL); }

static gsx_error hdl_destroy(gsx_async_dl_t async_dl);
static gsx_error hdl_submit(gsx_async_dl_t async_dl, gsx_size_t stable_sample_index, gsx_size_t slot_index);
static gsx_error hdl_wait(gsx_async_dl_t async_dl, gsx_async_dl_ready_item *out_item);
static gsx_error hdl_inflight_count(gsx_async_dl_t async_dl, gsx_size_t *out_count);

static const gsx_async_dl_i hip_async_dl_iface = { hdl_destroy, hdl_submit, hdl_wait, hdl_inflight_count };

/* keep the first failure, stop accepting work and wake every waiter */
static void hdl_fail(hip_async_dl *dl, gsx_error error)
{
    pthread_mutex_lock(&dl->mutex);
    if(!dl->failed) {
        dl->failed = true;
        dl->failure = error;
    }
    dl->closed = true;
    pthread_cond_broadcast(&dl->cond);
    pthread_mutex_unlock(&dl->mutex);
}

/* one sample into slot r->slot_index (gsx-cuda/async_dl.cu:182-270 with event ordering) */
static gsx_error hdl_load(hip_async_dl *dl, const hip_dl_request *r, gsx_async_dl_ready_item *out_item)
{
    const gsx_dataset_desc *ds = &dl->desc.dataset_desc;
    gsx_dataloader_slot *slot = NULL;
    hip_dl_slot *hs = NULL;
    gsx_dataset_cpu_sample sample;
    const int32_t is_u8 = ds->image_data_type == GSX_DATA_TYPE_U8;
    gsx_size_t off = 0;
    gsx_error error;

    if(r->slot_index >= dl->desc.slot_count) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader request slot index is out of range");
    }
    slot = &dl->desc.slots[r->slot_index];
    hs = &dl->slots[r->slot_index];
    /* the staging of this slot's previous load has been consumed by its DMA */
    if(gsx_hip_event_synchronize(hs->ready_ev) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader staging wait failed");
    }
    memset(&sample, 0, sizeof(sample));
    error = ds->get_sample(ds->object, r->stable_sample_index, &sample);
    if(!gsx_error_is_success(error)) {
        return error;
    }
    error = gsx_dataloader_validate_sample(ds, &sample);
    if(!gsx_error_is_success(error)) {
        ds->release_sample(ds->object, &sample);
        return error;
    }
    memcpy(hs->host, sample.rgb_data, (size_t)hs->rgb_bytes);
    off = hs->rgb_bytes;
    if(ds->has_alpha) {
        memcpy((unsigned char *)hs->host + off, sample.alpha_data, (size_t)hs->alpha_bytes);
        off += hs->alpha_bytes;
    }
    if(ds->has_invdepth) {
        memcpy((unsigned char *)hs->host + off, sample.invdepth_data, (size_t)hs->invdepth_bytes);
        off += hs->invdepth_bytes;
    }
    memset(out_item, 0, sizeof(*out_item));
    out_item->stable_sample_index = r->stable_sample_index;
    out_item->slot_index = r->slot_index;
    out_item->intrinsics = sample.intrinsics;
    out_item->pose = sample.pose;
    out_item->stable_sample_id = sample.stable_sample_id;
    out_item->has_stable_sample_id = sample.has_stable_sample_id;
    ds->release_sample(ds->object, &sample);

    if(gsx_hip_stream_wait_event(dl->stream, hs->free_ev) != GSX_HIP_SUCCESS
        || gsx_hip_memcpy_async(hs->device, hs->host, (size_t)off, dl->stream) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader staging upload failed");
    }
    off = 0;
    if(gsx_hip_dataloader_to_chw_f32(hs->device, is_u8, 3, ds->height, ds->width,
           gsx_hip_plugin_tensor_f32(slot->rgb_tensor), dl->stream) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader rgb layout conversion failed");
    }
    off += hs->rgb_bytes;
    if(ds->has_alpha
        && gsx_hip_dataloader_to_chw_f32((unsigned char *)hs->device + off, is_u8, 1, ds->height, ds->width,
               gsx_hip_plugin_tensor_f32(slot->alpha_tensor), dl->stream) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader alpha layout conversion failed");
    }
    if(ds->has_alpha) off += hs->alpha_bytes;
    if(ds->has_invdepth
        && gsx_hip_dataloader_to_chw_f32((unsigned char *)hs->device + off, is_u8, 1, ds->height, ds->width,
               gsx_hip_plugin_tensor_f32(slot->invdepth_tensor), dl->stream) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader inverse-depth layout conversion failed");
    }
    if(gsx_hip_event_record(hs->ready_ev, dl->stream) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader event record failed");
    }
    return hdl_ok();
}

static void *hdl_worker(void *arg)
{
    hip_async_dl *dl = (hip_async_dl *)arg;

    if(gsx_hip_set_device(dl->ordinal) != GSX_HIP_SUCCESS) {
        hdl_fail(dl, gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader could not select the device"));
        return NULL;
    }
    for(;;) {
        hip_dl_request r;
        gsx_async_dl_ready_item item;
        gsx_error error;

        pthread_mutex_lock(&dl->mutex);
        while(dl->req_count == 0 && !dl->closed) {
            pthread_cond_wait(&dl->cond, &dl->mutex);
        }
        if(dl->req_count == 0) {
            pthread_mutex_unlock(&dl->mutex);
            return NULL;
        }
        r = dl->requests[dl->req_head];
        dl->req_head = (dl->req_head + 1) % dl->desc.slot_count;
        dl->req_count -= 1;
        pthread_mutex_unlock(&dl->mutex);

        error = hdl_load(dl, &r, &item);
        if(!gsx_error_is_success(error)) {
            hdl_fail(dl, error);
            return NULL;
        }
        pthread_mutex_lock(&dl->mutex);
        dl->ready[(dl->ready_head + dl->ready_count) % dl->desc.slot_count] = item;
        dl->ready_count += 1;
        pthread_cond_broadcast(&dl->cond);
        pthread_mutex_unlock(&dl->mutex);
    }
}

static void hdl_release(hip_async_dl *dl)
{
    gsx_size_t i = 0;

    if(dl->stream != NULL) {
        (void)gsx_hip_stream_synchronize(dl->stream);
    }
    if(dl->slots != NULL) {
        for(i = 0; i < dl->desc.slot_count; ++i) {
            hip_dl_slot *hs = &dl->slots[i];

            if(hs->host != NULL) (void)gsx_hip_host_free(hs->host);
            if(hs->device != NULL) (void)gsx_hip_free(hs->device);
            if(hs->free_ev != NULL) (void)gsx_hip_event_destroy(hs->free_ev);
            if(hs->ready_ev != NULL) (void)gsx_hip_event_destroy(hs->ready_ev);
        }
    }
    if(dl->stream != NULL) {
        (void)gsx_hip_stream_destroy(dl->stream);
    }
    free(dl->slots);
    free(dl->requests);
    free(dl->ready);
    pthread_cond_destroy(&dl->cond);
    pthread_mutex_destroy(&dl->mutex);
    free(dl);
}

gsx_error gsx_hip_plugin_create_async_dl(gsx_backend_t backend, const gsx_async_dl_desc *desc, gsx_async_dl_t *out)
{
    hip_async_dl *dl = NULL;
    gsx_size_t i = 0, pixels = 0, elem = 0;
    const gsx_dataset_desc *ds = NULL;
    gsx_error error;

    if(out == NULL || desc == NULL || desc->slots == NULL || desc->slot_count == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader desc, slots and out must be non-null");
    }
    *out = NULL;
    ds = &desc->dataset_desc;
    if(desc->output_data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip async dataloader writes float32 tensors only");
    }
    if(ds->image_data_type != GSX_DATA_TYPE_U8 && ds->image_data_type != GSX_DATA_TYPE_F32) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip async dataloader reads u8 or float32 payloads");
    }
    error = gsx_dataloader_compute_element_count(ds->width, ds->height, 1, &pixels);
    if(!gsx_error_is_success(error)) {
        return error;
    }
    elem = ds->image_data_type == GSX_DATA_TYPE_U8 ? 1u : 4u;
    for(i = 0; i < desc->slot_count; ++i) {
        const gsx_dataloader_slot *s = &desc->slots[i];

        if(s->rgb_tensor == NULL || !gsx_hip_plugin_tensor_on_device(backend, s->rgb_tensor)
            || s->rgb_tensor->size_bytes != 3u * pixels * sizeof(float)
            || (ds->has_alpha && (s->alpha_tensor == NULL || !gsx_hip_plugin_tensor_on_device(backend, s->alpha_tensor)
                                     || s->alpha_tensor->size_bytes != pixels * sizeof(float)))
            || (ds->has_invdepth
                && (s->invdepth_tensor == NULL || !gsx_hip_plugin_tensor_on_device(backend, s->invdepth_tensor)
                    || s->invdepth_tensor->size_bytes != pixels * sizeof(float)))) {
            return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT,
                "hip async dataloader slots must be float32 CHW device tensors of the dataset size");
        }
    }
    dl = (hip_async_dl *)calloc(1, sizeof(*dl));
    if(dl == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip async dataloader");
    }
    pthread_mutex_init(&dl->mutex, NULL);
    pthread_cond_init(&dl->cond, NULL);
    dl->base.iface = &hip_async_dl_iface;
    dl->backend = backend;
    dl->desc = *desc;
    dl->ordinal = gsx_hip_plugin_backend_of(backend)->ordinal;
    dl->slots = (hip_dl_slot *)calloc((size_t)desc->slot_count, sizeof(*dl->slots));
    dl->requests = (hip_dl_request *)calloc((size_t)desc->slot_count, sizeof(*dl->requests));
    dl->ready = (gsx_async_dl_ready_item *)calloc((size_t)desc->slot_count, sizeof(*dl->ready));
    if(dl->slots == NULL || dl->requests == NULL || dl->ready == NULL
        || gsx_hip_stream_create(&dl->stream) != GSX_HIP_SUCCESS) {
        hdl_release(dl);
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip async dataloader state");
    }
    for(i = 0; i < desc->slot_count; ++i) {
        hip_dl_slot *hs = &dl->slots[i];
        gsx_size_t bytes = 0;

        hs->rgb_bytes = 3u * pixels * elem;
        hs->alpha_bytes = ds->has_alpha ? pixels * elem : 0u;
        hs->invdepth_bytes = ds->has_invdepth ? pixels * elem : 0u;
        bytes = hs->rgb_bytes + hs->alpha_bytes + hs->invdepth_bytes;
        if(gsx_hip_host_alloc(&hs->host, (size_t)bytes) != GSX_HIP_SUCCESS
            || gsx_hip_malloc(&hs->device, (size_t)bytes) != GSX_HIP_SUCCESS
            || gsx_hip_event_create(&hs->free_ev) != GSX_HIP_SUCCESS
            || gsx_hip_event_create(&hs->ready_ev) != GSX_HIP_SUCCESS) {
            hdl_release(dl);
            return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip async dataloader staging");
        }
    }
    if(pthread_create(&dl->worker, NULL, hdl_worker, dl) != 0) {
        hdl_release(dl);
        return gsx_make_error(GSX_ERROR_UNKNOWN, "failed to start the hip async dataloader thread");
    }
    dl->worker_started = true;
    backend->live_async_dl_count += 1;
    *out = &dl->base;
    return hdl_ok();
}

static gsx_error hdl_destroy(gsx_async_dl_t async_dl)
{
    hip_async_dl *dl = (hip_async_dl *)async_dl;
    gsx_backend_t backend = NULL;

    if(dl == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader must be non-null");
    }
    pthread_mutex_lock(&dl->mutex);
    dl->closed = true;
    pthread_cond_broadcast(&dl->cond);
    pthread_mutex_unlock(&dl->mutex);
    if(dl->worker_started) {
        (void)pthread_join(dl->worker, NULL);
    }
    backend = dl->backend;
    hdl_release(dl);
    if(backend->live_async_dl_count == 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "backend live_async_dl_count underflow in async dataloader free");
    }
    backend->live_async_dl_count -= 1;
    return hdl_ok();
}

static gsx_error hdl_submit(gsx_async_dl_t async_dl, gsx_size_t stable_sample_index, gsx_size_t slot_index)
{
    hip_async_dl *dl = (hip_async_dl *)async_dl;
    gsx_error error = hdl_ok();

    if(dl == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader must be non-null");
    }
    if(slot_index >= dl->desc.slot_count) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader request slot index is out of range");
    }
    /* the slot may be written once the major stream is past everything queued so far */
    if(gsx_hip_event_record(dl->slots[slot_index].free_ev, gsx_hip_plugin_stream(dl->backend)) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader event record failed");
    }
    pthread_mutex_lock(&dl->mutex);
    if(dl->failed) {
        error = dl->failure;
    } else if(dl->closed || dl->req_count == dl->desc.slot_count) {
        error = gsx_make_error(GSX_ERROR_INVALID_STATE, "async dataloader request queue closed or full");
    } else {
        dl->requests[(dl->req_head + dl->req_count) % dl->desc.slot_count].stable_sample_index = stable_sample_index;
        dl->requests[(dl->req_head + dl->req_count) % dl->desc.slot_count].slot_index = slot_index;
        dl->req_count += 1;
        dl->inflight += 1;
        pthread_cond_broadcast(&dl->cond);
    }
    pthread_mutex_unlock(&dl->mutex);
    return error;
}

static gsx_error hdl_wait(gsx_async_dl_t async_dl, gsx_async_dl_ready_item *out_item)
{
    hip_async_dl *dl = (hip_async_dl *)async_dl;
    gsx_error error = hdl_ok();
    bool have = false;

    if(dl == NULL || out_item == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader and out_item must be non-null");
    }
    pthread_mutex_lock(&dl->mutex);
    while(dl->ready_count == 0 && !dl->closed) {
        pthread_cond_wait(&dl->cond, &dl->mutex);
    }
    if(dl->ready_count > 0) {
        *out_item = dl->ready[dl->ready_head];
        dl->ready_head = (dl->ready_head + 1) % dl->desc.slot_count;
        dl->ready_count -= 1;
        dl->inflight -= 1;
        have = true;
    } else {
        error = dl->failed ? dl->failure : gsx_make_error(GSX_ERROR_INVALID_STATE, "async dataloader ready queue closed");
    }
    pthread_mutex_unlock(&dl->mutex);
    if(have && gsx_hip_stream_wait_event(gsx_hip_plugin_stream(dl->backend), dl->slots[out_item->slot_index].ready_ev)
            != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip async dataloader stream ordering failed");
    }
    return error;
}

static gsx_error hdl_inflight_count(gsx_async_dl_t async_dl, gsx_size_t *out_count)
{
    hip_async_dl *dl = (hip_async_dl *)async_dl;

    if(dl == NULL || out_count == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "async dataloader and out_count must be non-null");
    }
    pthread_mutex_lock(&dl->mutex);
    *out_count = dl->inflight;
    pthread_mutex_unlock(&dl->mutex);
    return hdl_ok();
}
