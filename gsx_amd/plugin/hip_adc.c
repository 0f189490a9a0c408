/*
 * hip_adc.c - adaptive density control vtable of the gsx HIP backend (gsx/src/gsx-impl.h:470-473).
 * Every policy runs as one gsx_hip_adc_step with the CPU semantics of gsx/src/gsx-cpu/adc.c:380-559:
 *   - DEFAULT / ABSGS (adc/default.c:160-527): grow candidates up to the budget, duplicate or
 *     split, prune, clear the statistics, reset opacity in a reset window;
 *   - MCMC (adc/mcmc.c:345-766): position noise on every step before end_refine, and in a refine
 *     window relocation of the dead rows plus growth by grow_ratio.
 * A refine or reset works on a working copy of the Gaussian rows and their Adam moments; the
 * result is written back through gsx_gs_resize and the optimizer's resize, so the set and the
 * optimizer stay count-aligned (gsx-impl.h:36-37). An MCMC step with noise only moves mean3d in
 * place.
 */
#include "hip_backend.h"

#include <stdlib.h>
#include <string.h>

gsx_error gsx_hip_plugin_optim_moments(gsx_optim_t optim, gsx_index_t group, float **out_m, float **out_v,
    gsx_size_t *out_rows);

typedef struct hip_adc {
    struct gsx_adc base;
    gsx_hip_adc_context *ctx;
} hip_adc;

static gsx_error ha_ok(void) { return gsx_make_error(GSX_ERROR_SUCCESS, NULL); }

static gsx_error ha_destroy(gsx_adc_t adc);
static gsx_error ha_step(gsx_adc_t adc, const gsx_adc_request *request, gsx_adc_result *out_result);

static const gsx_adc_i hip_adc_iface = { ha_destroy, ha_step };

gsx_error gsx_hip_plugin_create_adc(gsx_backend_t backend, const gsx_adc_desc *desc, gsx_adc_t *out)
{
    hip_adc *a = NULL;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };
    gsx_hip_status st = GSX_HIP_SUCCESS;

    if(out == NULL || desc == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_adc and desc must be non-null");
    }
    *out = NULL;
    if(desc->algorithm != GSX_ADC_ALGORITHM_DEFAULT && desc->algorithm != GSX_ADC_ALGORITHM_ABSGS
        && desc->algorithm != GSX_ADC_ALGORITHM_MCMC) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED,
            "hip adc supports GSX_ADC_ALGORITHM_DEFAULT, GSX_ADC_ALGORITHM_ABSGS and GSX_ADC_ALGORITHM_MCMC");
    }
    a = (hip_adc *)calloc(1, sizeof(*a));
    if(a == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip adc");
    }
    error = gsx_adc_base_init(&a->base, &hip_adc_iface, backend, desc);
    if(!gsx_error_is_success(error)) {
        free(a);
        return error;
    }
    /* the split stream: pcg32 seeded (seed, seed), as the CPU adc object (gsx-cpu/adc.c:466) */
    st = gsx_hip_adc_context_create(&a->ctx, (uint64_t)desc->seed);
    if(st != GSX_HIP_SUCCESS) {
        gsx_adc_base_deinit(&a->base);
        free(a);
        return gsx_hip_plugin_error(st, "hip adc context creation failed");
    }
    *out = &a->base;
    return ha_ok();
}

static gsx_error ha_destroy(gsx_adc_t adc)
{
    hip_adc *a = (hip_adc *)adc;

    if(adc == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "adc must be non-null");
    }
    (void)gsx_hip_stream_synchronize(gsx_hip_plugin_stream(adc->backend));
    (void)gsx_hip_adc_context_destroy(a->ctx);
    gsx_adc_base_deinit(&a->base);
    free(a);
    return ha_ok();
}

static gsx_size_t ha_nonneg(gsx_index_t v) { return v <= 0 ? 0 : (gsx_size_t)v; }

/* gsx-cpu/adc.c:48-80 */
static bool ha_in_refine_window(const gsx_adc_desc *d, gsx_size_t step)
{
    return d->refine_every != 0 && step % (gsx_size_t)d->refine_every == 0 && step >= ha_nonneg(d->start_refine)
        && step <= ha_nonneg(d->end_refine);
}

static bool ha_in_reset_window(const gsx_adc_desc *d, gsx_size_t step)
{
    return d->reset_every != 0 && step % (gsx_size_t)d->reset_every == 0 && step >= ha_nonneg(d->start_refine)
        && step < ha_nonneg(d->end_refine);
}

/* The Gaussian set's field arrays: parameters (field order of gsx_hip_gs_rows: mean3d, rotation,
 * logscale, opacity, sh0..sh3), then the statistics grad_acc, absgrad_acc, visible_counter,
 * max_screen_radius. */
#define HA_FIELDS 12
static const gsx_gs_field ha_gs_field[HA_FIELDS] = {
    GSX_GS_FIELD_MEAN3D, GSX_GS_FIELD_ROTATION, GSX_GS_FIELD_LOGSCALE, GSX_GS_FIELD_OPACITY, GSX_GS_FIELD_SH0,
    GSX_GS_FIELD_SH1, GSX_GS_FIELD_SH2, GSX_GS_FIELD_SH3, GSX_GS_FIELD_GRAD_ACC, GSX_GS_FIELD_ABSGRAD_ACC,
    GSX_GS_FIELD_VISIBLE_COUNTER, GSX_GS_FIELD_MAX_SCREEN_RADIUS
};
static const int ha_width[HA_FIELDS] = { 3, 4, 3, 1, 3, 9, 15, 21, 1, 1, 1, 1 };
/* optimizer role of parameter field k (gsx-optim.h:12-21) */
static const gsx_optim_param_role ha_role[8] = {
    GSX_OPTIM_PARAM_ROLE_MEAN3D, GSX_OPTIM_PARAM_ROLE_ROTATION, GSX_OPTIM_PARAM_ROLE_LOGSCALE,
    GSX_OPTIM_PARAM_ROLE_OPACITY, GSX_OPTIM_PARAM_ROLE_SH0, GSX_OPTIM_PARAM_ROLE_SH1, GSX_OPTIM_PARAM_ROLE_SH2,
    GSX_OPTIM_PARAM_ROLE_SH3
};

static float **ha_slot(gsx_hip_gs_rows *r, int k)
{
    float **slots[HA_FIELDS] = { &r->mean3d, &r->rotation, &r->logscale, &r->opacity, &r->sh0, &r->sh1, &r->sh2,
        &r->sh3, &r->grad_acc, &r->absgrad_acc, &r->visible_counter, &r->max_screen_radius };
    return slots[k];
}

typedef struct ha_work {
    void *block;               /* one device allocation for both row sets */
    gsx_hip_gs_rows rows, out;
    int32_t moment_group[8];   /* optimizer group of parameter field k, or -1 */
    bool present[HA_FIELDS];
} ha_work;

static void ha_params(const gsx_adc_desc *d, const gsx_adc_request *request, gsx_float_t lr_mean3d,
    gsx_hip_adc_params *p)
{
    memset(p, 0, sizeof(*p));
    p->algorithm = d->algorithm == GSX_ADC_ALGORITHM_MCMC ? 2 : (d->algorithm == GSX_ADC_ALGORITHM_ABSGS ? 1 : 0);
    p->pruning_opacity_threshold = d->pruning_opacity_threshold;
    p->opacity_clamp_value = d->opacity_clamp_value;
    p->max_world_scale = d->max_world_scale;
    p->max_screen_scale = d->max_screen_scale;
    p->duplicate_grad_threshold = d->duplicate_grad_threshold;
    p->duplicate_scale_threshold = d->duplicate_scale_threshold;
    p->duplicate_absgrad_threshold = d->duplicate_absgrad_threshold;
    p->scene_scale = request->scene_scale;
    p->refine_every = d->refine_every;
    p->start_refine = d->start_refine;
    p->end_refine = d->end_refine;
    p->max_num_gaussians = d->max_num_gaussians;
    p->reset_every = d->reset_every;
    p->noise_strength = d->noise_strength;
    p->grow_ratio = d->grow_ratio;
    p->mean3d_learning_rate = lr_mean3d;
}

static gsx_error ha_step(gsx_adc_t adc, const gsx_adc_request *request, gsx_adc_result *out_result)
{
    hip_adc *a = (hip_adc *)adc;
    gsx_backend_t backend = adc->backend;
    hipStream_t stream = gsx_hip_plugin_stream(backend);
    const gsx_adc_desc *d = &adc->desc;
    gsx_gs_info info;
    gsx_tensor_t src[HA_FIELDS];
    ha_work w;
    gsx_hip_adc_params p;
    gsx_size_t n = 0, capacity = 0, total_floats = 0, offset = 0;
    int64_t counts[4] = { 0, 0, 0, 0 };
    int32_t in_out = 0;
    int64_t new_count = 0;
    int k = 0, sh_degree = 0;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };
    gsx_hip_status st = GSX_HIP_SUCCESS;
    bool use_optim = request->optim != NULL && request->optim->iface != NULL;
    bool refine = false, reset = false, noise = false;
    gsx_size_t copies = 2;
    gsx_float_t lr_mean3d = 0.0f;

    memset(out_result, 0, sizeof(*out_result));
    memset(&w, 0, sizeof(w));
    error = gsx_gs_get_info(request->gs, &info);
    if(!gsx_error_is_success(error)) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip adc requires gs info/query support");
    }
    n = info.count;
    out_result->gaussians_before = n;
    out_result->gaussians_after = n;
    refine = ha_in_refine_window(d, request->global_step);
    reset = ha_in_reset_window(d, request->global_step);
    /* MCMC noise: every step before end_refine (gsx-cpu/adc/mcmc.c:357-364) */
    noise = d->algorithm == GSX_ADC_ALGORITHM_MCMC && d->noise_strength > 0.0f
        && !(ha_nonneg(d->end_refine) > 0 && request->global_step >= ha_nonneg(d->end_refine));
    if(!refine && !reset && !noise) {
        return ha_ok();
    }
    if(n == 0) {
        return ha_ok();
    }
    if(noise) {
        /* the noise is scaled by the optimizer's current mean3d rate (mcmc.c:375-380) */
        error = gsx_optim_get_learning_rate_by_role(request->optim, GSX_OPTIM_PARAM_ROLE_MEAN3D, &lr_mean3d);
        if(!gsx_error_is_success(error)) {
            return error;
        }
    }

    /* the fields and moments that exist, all device tensors of this backend */
    for(k = 0; k < HA_FIELDS; ++k) {
        src[k] = NULL;
        if(!gsx_error_is_success(gsx_gs_get_field(request->gs, ha_gs_field[k], &src[k])) || src[k] == NULL) {
            src[k] = NULL;
            if(k <= 4) {
                return gsx_make_error(GSX_ERROR_INVALID_STATE, "hip adc requires mean3d, rotation, logscale, opacity and sh0");
            }
            continue;
        }
        if(!gsx_hip_plugin_tensor_on_device(backend, src[k]) || src[k]->data_type != GSX_DATA_TYPE_F32
            || src[k]->size_bytes != n * (gsx_size_t)ha_width[k] * sizeof(float)) {
            return gsx_make_error(GSX_ERROR_INVALID_STATE, "hip adc fields must be float32 device tensors of the gs count");
        }
        w.present[k] = true;
    }
    sh_degree = w.present[7] ? 3 : (w.present[6] ? 2 : (w.present[5] ? 1 : 0));
    ha_params(d, request, lr_mean3d, &p);
    if(!refine && !reset) {
        /* MCMC noise only: the count stays, mean3d moves in place */
        gsx_hip_gs_rows rows, unused;

        memset(&rows, 0, sizeof(rows));
        memset(&unused, 0, sizeof(unused));
        rows.count = (int64_t)n;
        rows.sh_degree = sh_degree;
        for(k = 0; k < HA_FIELDS; ++k) {
            if(w.present[k]) *ha_slot(&rows, k) = gsx_hip_plugin_tensor_f32(src[k]);
        }
        st = gsx_hip_adc_step(a->ctx, &p, (uint64_t)request->global_step, &rows, (int64_t)n, &unused, &in_out, counts,
            stream);
        return st == GSX_HIP_SUCCESS ? ha_ok() : gsx_hip_plugin_error(st, "hip adc noise failed");
    }
    for(k = 0; k < 8; ++k) {
        w.moment_group[k] = -1;
        if(use_optim && w.present[k] && request->optim->role_to_index[ha_role[k]] >= 0) {
            float *m = NULL, *v = NULL;
            gsx_size_t rows = 0;
            gsx_index_t gi = request->optim->role_to_index[ha_role[k]];

            error = gsx_hip_plugin_optim_moments(request->optim, gi, &m, &v, &rows);
            if(!gsx_error_is_success(error)) return error;
            if(rows != n) {
                return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer state is not count-aligned with the gs");
            }
            w.moment_group[k] = (int32_t)gi;
        }
    }

    /* working rows: capacity for every grown row (gsx_hip_adc_step appends in place) */
    capacity = n;
    if(d->max_num_gaussians > 0 && (gsx_size_t)d->max_num_gaussians > capacity) {
        capacity = (gsx_size_t)d->max_num_gaussians;
    }
    /* MCMC never removes rows: its result stays in the one row set */
    copies = d->algorithm == GSX_ADC_ALGORITHM_MCMC ? 1u : 2u;
    for(k = 0; k < HA_FIELDS; ++k) {
        if(w.present[k]) total_floats += copies * capacity * (gsx_size_t)ha_width[k];
        if(k < 8 && w.moment_group[k] >= 0) total_floats += 2 * copies * capacity * (gsx_size_t)ha_width[k];
    }
    /* from the stream-ordered pool: returned behind the step's queued copies, no host wait */
    st = gsx_hip_pool_malloc(&w.block, (size_t)total_floats * sizeof(float), stream);
    if(st != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "hip adc working rows allocation failed");
    }
#define HA_TAKE(width) ((float *)w.block + (offset += capacity * (gsx_size_t)(width), offset - capacity * (gsx_size_t)(width)))
    w.rows.count = (int64_t)n;
    w.rows.sh_degree = sh_degree;
    w.out.sh_degree = sh_degree;
    for(k = 0; k < HA_FIELDS; ++k) {
        if(!w.present[k]) continue;
        *ha_slot(&w.rows, k) = HA_TAKE(ha_width[k]);
        if(copies == 2) *ha_slot(&w.out, k) = HA_TAKE(ha_width[k]);
        st = gsx_hip_memcpy_async(*ha_slot(&w.rows, k), gsx_hip_plugin_tensor_ptr(src[k]),
            (size_t)n * (size_t)ha_width[k] * sizeof(float), stream);
        if(st != GSX_HIP_SUCCESS) break;
        if(k < 8 && w.moment_group[k] >= 0) {
            float *m = NULL, *v = NULL;
            gsx_size_t rows = 0;

            (void)gsx_hip_plugin_optim_moments(request->optim, w.moment_group[k], &m, &v, &rows);
            w.rows.first_moment[k] = HA_TAKE(ha_width[k]);
            w.rows.second_moment[k] = HA_TAKE(ha_width[k]);
            if(copies == 2) {
                w.out.first_moment[k] = HA_TAKE(ha_width[k]);
                w.out.second_moment[k] = HA_TAKE(ha_width[k]);
            }
            st = gsx_hip_memcpy_async(w.rows.first_moment[k], m, (size_t)n * (size_t)ha_width[k] * sizeof(float), stream);
            if(st == GSX_HIP_SUCCESS) {
                st = gsx_hip_memcpy_async(w.rows.second_moment[k], v, (size_t)n * (size_t)ha_width[k] * sizeof(float),
                    stream);
            }
            if(st != GSX_HIP_SUCCESS) break;
        }
    }
#undef HA_TAKE
    if(st != GSX_HIP_SUCCESS) {
        (void)gsx_hip_pool_free(w.block, stream);
        return gsx_hip_plugin_error(st, "hip adc working copy failed");
    }

    st = gsx_hip_adc_step(a->ctx, &p, (uint64_t)request->global_step, &w.rows, (int64_t)capacity, &w.out, &in_out,
        counts, stream);
    if(st != GSX_HIP_SUCCESS) {
        (void)gsx_hip_pool_free(w.block, stream);
        return gsx_hip_plugin_error(st, "hip adc step failed");
    }
    new_count = in_out ? w.out.count : w.rows.count;

    /* commit: the set (and the optimizer's moments) take the new count, then the rows */
    if((gsx_size_t)new_count != n) {
        error = gsx_gs_resize(request->gs, (gsx_size_t)new_count);
        if(gsx_error_is_success(error) && use_optim) {
            error = gsx_optim_rebind_param_groups_from_gs(request->optim, request->gs);
            if(gsx_error_is_success(error)) error = gsx_optim_resize(request->optim, (gsx_size_t)new_count);
        }
        if(!gsx_error_is_success(error)) {
            (void)gsx_hip_pool_free(w.block, stream);
            return error;
        }
    }
    for(k = 0; k < HA_FIELDS && st == GSX_HIP_SUCCESS; ++k) {
        gsx_tensor_t dst = NULL;
        const gsx_hip_gs_rows *res = in_out ? &w.out : &w.rows;

        if(!w.present[k]) continue;
        if(!gsx_error_is_success(gsx_gs_get_field(request->gs, ha_gs_field[k], &dst)) || dst == NULL) {
            st = GSX_HIP_ERROR_INVALID_STATE;
            break;
        }
        st = gsx_hip_memcpy_async(gsx_hip_plugin_tensor_ptr(dst), *ha_slot((gsx_hip_gs_rows *)res, k),
            (size_t)new_count * (size_t)ha_width[k] * sizeof(float), stream);
        if(st == GSX_HIP_SUCCESS && k < 8 && w.moment_group[k] >= 0) {
            float *m = NULL, *v = NULL;
            gsx_size_t rows = 0;

            (void)gsx_hip_plugin_optim_moments(request->optim, w.moment_group[k], &m, &v, &rows);
            st = gsx_hip_memcpy_async(m, res->first_moment[k], (size_t)new_count * (size_t)ha_width[k] * sizeof(float),
                stream);
            if(st == GSX_HIP_SUCCESS) {
                st = gsx_hip_memcpy_async(v, res->second_moment[k],
                    (size_t)new_count * (size_t)ha_width[k] * sizeof(float), stream);
            }
        }
    }
    (void)gsx_hip_pool_free(w.block, stream);
    if(st != GSX_HIP_SUCCESS) {
        return gsx_hip_plugin_error(st, "hip adc commit failed");
    }
    if(counts[3] != 0 && use_optim) {
        /* the opacity group restarts with the clamp: moments and step count (default.c:306-311) */
        error = gsx_optim_reset_param_group_by_role(request->optim, GSX_OPTIM_PARAM_ROLE_OPACITY);
        if(!gsx_error_is_success(error)) {
            return error;
        }
    }
    out_result->gaussians_after = (gsx_size_t)new_count;
    out_result->pruned_count = (gsx_size_t)counts[0];
    out_result->duplicated_count = (gsx_size_t)counts[1];
    out_result->grown_count = (gsx_size_t)counts[2];
    out_result->reset_count = (gsx_size_t)counts[3];
    out_result->mutated = counts[0] != 0 || counts[1] != 0 || counts[2] != 0 || counts[3] != 0
        || (gsx_size_t)new_count != n;
    return ha_ok();
}
