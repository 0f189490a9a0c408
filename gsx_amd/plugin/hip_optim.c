/*
 * hip_optim.c - Adam optimizer vtable of the gsx HIP backend (gsx/src/gsx-impl.h:460-468).
 * Counterpart of gsx/src/gsx-cuda/optim.c with the CPU semantics of gsx/src/gsx-cpu/optim.c:
 * per-group step counters and bias corrections 1 - beta^t in double (optim.c:730-731), the
 * element update of optim.c:736-760 (one launch for all selected groups), moments that follow
 * the parameter rows through permute / gather / resize (optim.c:823-1085) and reset to zero.
 * The moments are optimizer-owned device arrays of the parameter's shape.
 */
#include "hip_backend.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct hip_optim {
    struct gsx_optim base;
    gsx_size_t *steps;
    float **m;
    float **v;
    gsx_size_t *rows;       /* leading extent of each group's moments */
    gsx_size_t *row_floats; /* floats per row */
} hip_optim;

static gsx_error ho_ok(void) { return gsx_make_error(GSX_ERROR_SUCCESS, NULL); }

static gsx_error ho_destroy(gsx_optim_t optim);
static gsx_error ho_step_selected(gsx_optim_t optim, const bool *selected);
static gsx_error ho_permute(gsx_optim_t optim, gsx_tensor_t permutation);
static gsx_error ho_gather(gsx_optim_t optim, gsx_tensor_t indices);
static gsx_error ho_resize(gsx_optim_t optim, gsx_size_t new_count);
static gsx_error ho_reset_all(gsx_optim_t optim);
static gsx_error ho_reset_by_index(gsx_optim_t optim, gsx_index_t index);

static const gsx_optim_i hip_optim_iface = {
    ho_destroy, ho_step_selected, ho_permute, ho_gather, ho_resize, ho_reset_all, ho_reset_by_index
};

static hipStream_t ho_stream(const hip_optim *o) { return gsx_hip_plugin_stream(o->base.backend); }

/* rows and floats per row of a parameter tensor (gsx-cpu/optim.c:525-543) */
static gsx_error ho_layout(gsx_tensor_t t, gsx_size_t *rows, gsx_size_t *row_floats)
{
    gsx_size_t n = 0;

    if(t == NULL || t->rank <= 0 || t->shape[0] <= 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer tensors must keep a positive leading extent");
    }
    n = t->size_bytes / sizeof(float);
    if(n % (gsx_size_t)t->shape[0] != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer tensor size must be divisible by the leading extent");
    }
    *rows = (gsx_size_t)t->shape[0];
    *row_floats = n / *rows;
    return ho_ok();
}

/* parameter and gradient still compatible device float32 tensors (gsx-cpu/optim.c:210-240) */
static gsx_error ho_check_group(const hip_optim *o, gsx_index_t i)
{
    const gsx_optim_param_group_desc *g = &o->base.param_groups[i];
    gsx_index_t d = 0;

    if(g->parameter == NULL || g->gradient == NULL || g->parameter->backing_buffer == NULL
        || g->gradient->backing_buffer == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer parameter and gradient tensors must remain live and accessible");
    }
    if(!gsx_hip_plugin_tensor_on_device(o->base.backend, g->parameter)
        || !gsx_hip_plugin_tensor_on_device(o->base.backend, g->gradient)) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer tensors must be device tensors of the owning backend");
    }
    if(g->parameter->rank != g->gradient->rank || g->parameter->data_type != g->gradient->data_type
        || g->parameter->size_bytes != g->gradient->size_bytes) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer parameter and gradient tensors are no longer compatible");
    }
    if(g->parameter->data_type != GSX_DATA_TYPE_F32 || g->parameter->size_bytes % sizeof(float) != 0) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer tensors must remain float32");
    }
    for(d = 0; d < g->parameter->rank; ++d) {
        if(g->parameter->shape[d] != g->gradient->shape[d]) {
            return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer parameter and gradient tensor shapes no longer match");
        }
    }
    return ho_ok();
}

static gsx_error ho_alloc_zero(hipStream_t stream, gsx_size_t floats, float **m, float **v)
{
    const uint8_t zero = 0;
    size_t bytes = (size_t)(floats > 0 ? floats : 1) * sizeof(float);

    *m = NULL;
    *v = NULL;
    if(gsx_hip_pool_malloc((void **)m, bytes, stream) != GSX_HIP_SUCCESS
        || gsx_hip_pool_malloc((void **)v, bytes, stream) != GSX_HIP_SUCCESS) {
        if(*m != NULL) (void)gsx_hip_pool_free(*m, stream);
        if(*v != NULL) (void)gsx_hip_pool_free(*v, stream);
        *m = NULL;
        *v = NULL;
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "hip optimizer moment allocation failed");
    }
    if(gsx_hip_fill_pattern(*m, bytes, &zero, 1, stream) != GSX_HIP_SUCCESS
        || gsx_hip_fill_pattern(*v, bytes, &zero, 1, stream) != GSX_HIP_SUCCESS) {
        return gsx_make_error(GSX_ERROR_UNKNOWN, "hip optimizer moment clear failed");
    }
    return ho_ok();
}

static void ho_free_arrays(hip_optim *o)
{
    gsx_index_t i = 0;

    /* the pool takes the moments back behind the major stream's queued work (no host wait) */
    for(i = 0; i < o->base.param_group_count; ++i) {
        if(o->m != NULL && o->m[i] != NULL) (void)gsx_hip_pool_free(o->m[i], ho_stream(o));
        if(o->v != NULL && o->v[i] != NULL) (void)gsx_hip_pool_free(o->v[i], ho_stream(o));
    }
    free(o->steps);
    free(o->m);
    free(o->v);
    free(o->rows);
    free(o->row_floats);
}

gsx_error gsx_hip_plugin_create_optim(gsx_backend_t backend, const gsx_optim_desc *desc, gsx_optim_t *out)
{
    hip_optim *o = NULL;
    gsx_index_t i = 0, n = 0;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(out == NULL || desc == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "out_optim and desc must be non-null");
    }
    *out = NULL;
    if(desc->state_buffer_type != NULL
        && desc->state_buffer_type != &gsx_hip_plugin_backend_of(backend)->device_type.base) {
        return gsx_make_error(GSX_ERROR_NOT_SUPPORTED, "hip optimizer state lives in device memory");
    }
    o = (hip_optim *)calloc(1, sizeof(*o));
    if(o == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip optimizer");
    }
    error = gsx_optim_base_init(&o->base, &hip_optim_iface, backend, desc);
    if(!gsx_error_is_success(error)) {
        free(o);
        return error;
    }
    n = o->base.param_group_count;
    o->steps = (gsx_size_t *)calloc((size_t)(n > 0 ? n : 1), sizeof(gsx_size_t));
    o->m = (float **)calloc((size_t)(n > 0 ? n : 1), sizeof(float *));
    o->v = (float **)calloc((size_t)(n > 0 ? n : 1), sizeof(float *));
    o->rows = (gsx_size_t *)calloc((size_t)(n > 0 ? n : 1), sizeof(gsx_size_t));
    o->row_floats = (gsx_size_t *)calloc((size_t)(n > 0 ? n : 1), sizeof(gsx_size_t));
    if(o->steps == NULL || o->m == NULL || o->v == NULL || o->rows == NULL || o->row_floats == NULL) {
        ho_free_arrays(o);
        gsx_optim_base_deinit(&o->base);
        free(o);
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate hip optimizer state arrays");
    }
    for(i = 0; i < n; ++i) {
        error = ho_check_group(o, i);
        if(gsx_error_is_success(error)) {
            error = ho_layout(o->base.param_groups[i].parameter, &o->rows[i], &o->row_floats[i]);
        }
        if(gsx_error_is_success(error)) {
            error = ho_alloc_zero(ho_stream(o), o->rows[i] * o->row_floats[i], &o->m[i], &o->v[i]);
        }
        if(!gsx_error_is_success(error)) {
            ho_free_arrays(o);
            gsx_optim_base_deinit(&o->base);
            free(o);
            return error;
        }
    }
    *out = &o->base;
    return ho_ok();
}

static gsx_error ho_destroy(gsx_optim_t optim)
{
    hip_optim *o = (hip_optim *)optim;

    if(optim == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optim must be non-null");
    }
    ho_free_arrays(o);
    gsx_optim_base_deinit(&o->base);
    free(o);
    return ho_ok();
}

/* moments that match the parameter exactly (gsx-cpu/optim.c:242-278) */
static gsx_error ho_check_exact(const hip_optim *o, gsx_index_t i)
{
    gsx_size_t rows = 0, width = 0;
    gsx_error error = ho_check_group(o, i);

    if(!gsx_error_is_success(error)) {
        return error;
    }
    if(!gsx_error_is_success(ho_layout(o->base.param_groups[i].parameter, &rows, &width))
        || rows != o->rows[i] || width != o->row_floats[i]) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer state tensors no longer match the parameter tensor layout");
    }
    return ho_ok();
}

static gsx_error ho_step_selected(gsx_optim_t optim, const bool *selected)
{
    hip_optim *o = (hip_optim *)optim;
    gsx_hip_adam_group batch[GSX_HIP_ADAM_MAX_GROUPS];
    int32_t used = 0;
    gsx_index_t i = 0;

    for(i = 0; i < o->base.param_group_count; ++i) {
        const gsx_optim_param_group_desc *g = &o->base.param_groups[i];
        gsx_hip_adam_group *a = NULL;
        gsx_error error = { GSX_ERROR_SUCCESS, NULL };

        if(selected != NULL && !selected[i]) {
            continue;
        }
        error = ho_check_exact(o, i);
        if(!gsx_error_is_success(error)) {
            return error;
        }
        if(o->steps[i] == UINT64_MAX) {
            return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "optimizer Adam step counter overflowed");
        }
        o->steps[i] += 1;
        a = &batch[used++];
        memset(a, 0, sizeof(*a));
        a->parameter = gsx_hip_plugin_tensor_f32(g->parameter);
        a->gradient = gsx_hip_plugin_tensor_f32(g->gradient);
        a->first_moment = o->m[i];
        a->second_moment = o->v[i];
        a->count = (int64_t)(o->rows[i] * o->row_floats[i]);
        a->beta1 = g->beta1;
        a->beta2 = g->beta2;
        a->learning_rate = o->base.learning_rates[i];
        a->weight_decay = g->weight_decay;
        a->epsilon = g->epsilon;
        a->max_grad = g->max_grad;
        a->bias_correction1 = 1.0 - pow((double)g->beta1, (double)o->steps[i]);
        a->bias_correction2 = 1.0 - pow((double)g->beta2, (double)o->steps[i]);
        if(used == GSX_HIP_ADAM_MAX_GROUPS) {
            gsx_hip_status st = gsx_hip_adam_step_multi_launch(batch, used, ho_stream(o));

            if(st != GSX_HIP_SUCCESS) return gsx_hip_plugin_error(st, "hip adam step failed");
            used = 0;
        }
    }
    if(used > 0) {
        gsx_hip_status st = gsx_hip_adam_step_multi_launch(batch, used, ho_stream(o));

        if(st != GSX_HIP_SUCCESS) return gsx_hip_plugin_error(st, "hip adam step failed");
    }
    return ho_ok();
}

static gsx_error ho_reset_by_index(gsx_optim_t optim, gsx_index_t index)
{
    hip_optim *o = (hip_optim *)optim;
    const uint8_t zero = 0;
    size_t bytes = 0;

    if(index < 0 || index >= o->base.param_group_count) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "optimizer param-group index is out of range");
    }
    if(o->m[index] == NULL || o->v[index] == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer state tensors are unavailable");
    }
    bytes = (size_t)(o->rows[index] * o->row_floats[index]) * sizeof(float);
    if(bytes > 0) {
        if(gsx_hip_fill_pattern(o->m[index], bytes, &zero, 1, ho_stream(o)) != GSX_HIP_SUCCESS
            || gsx_hip_fill_pattern(o->v[index], bytes, &zero, 1, ho_stream(o)) != GSX_HIP_SUCCESS) {
            return gsx_make_error(GSX_ERROR_UNKNOWN, "hip optimizer reset failed");
        }
    }
    o->steps[index] = 0;
    return ho_ok();
}

static gsx_error ho_reset_all(gsx_optim_t optim)
{
    gsx_index_t i = 0;

    for(i = 0; i < optim->param_group_count; ++i) {
        gsx_error error = ho_reset_by_index(optim, i);

        if(!gsx_error_is_success(error)) return error;
    }
    return ho_ok();
}

/* host copy of an int32 control tensor of this backend with `expect` entries */
static gsx_error ho_read_indices(const hip_optim *o, gsx_tensor_t t, gsx_size_t expect, const char *what, int32_t **out)
{
    int32_t *host = NULL;

    *out = NULL;
    if(t == NULL || t->backing_buffer == NULL) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer control tensors must be live and accessible");
    }
    if(t->backing_buffer->buffer_type->backend != o->base.backend) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer control tensors must belong to the optimizer backend");
    }
    if(t->data_type != GSX_DATA_TYPE_I32) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, what);
    }
    if(t->rank != 1 || (gsx_size_t)t->shape[0] != expect) {
        return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer control tensor has an incompatible rank or leading extent");
    }
    host = (int32_t *)malloc(sizeof(int32_t) * (size_t)(expect > 0 ? expect : 1));
    if(host == NULL) {
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate optimizer index staging");
    }
    if(expect > 0) {
        if(gsx_hip_memcpy_async(host, gsx_hip_plugin_tensor_ptr(t), (size_t)expect * sizeof(int32_t), ho_stream(o))
                != GSX_HIP_SUCCESS
            || gsx_hip_stream_synchronize(ho_stream(o)) != GSX_HIP_SUCCESS) {
            free(host);
            return gsx_make_error(GSX_ERROR_UNKNOWN, "hip optimizer index readback failed");
        }
    }
    *out = host;
    return ho_ok();
}

/* Rows of every group's moments re-laid by `index` (new row r = old row index[r]) into fresh
 * arrays of `new_rows` rows; rows at or past `copy_rows` of a resize are zero. */
static gsx_error ho_relayout(hip_optim *o, gsx_tensor_t index, gsx_size_t new_rows, gsx_size_t copy_rows)
{
    gsx_index_t i = 0;

    for(i = 0; i < o->base.param_group_count; ++i) {
        float *m = NULL, *v = NULL;
        size_t row_bytes = (size_t)o->row_floats[i] * sizeof(float);
        gsx_error error = ho_alloc_zero(ho_stream(o), new_rows * o->row_floats[i], &m, &v);

        if(!gsx_error_is_success(error)) return error;
        if(index != NULL && new_rows > 0) {
            if(gsx_hip_gather_rows_kernel_launch(o->m[i], m, (int64_t)row_bytes, (int64_t)new_rows,
                    (const int32_t *)gsx_hip_plugin_tensor_ptr(index), (int64_t)o->rows[i], NULL, ho_stream(o))
                    != GSX_HIP_SUCCESS
                || gsx_hip_gather_rows_kernel_launch(o->v[i], v, (int64_t)row_bytes, (int64_t)new_rows,
                    (const int32_t *)gsx_hip_plugin_tensor_ptr(index), (int64_t)o->rows[i], NULL, ho_stream(o))
                    != GSX_HIP_SUCCESS) {
                return gsx_make_error(GSX_ERROR_UNKNOWN, "hip optimizer gather failed");
            }
        } else if(copy_rows > 0) {
            if(gsx_hip_memcpy_async(m, o->m[i], (size_t)copy_rows * row_bytes, ho_stream(o)) != GSX_HIP_SUCCESS
                || gsx_hip_memcpy_async(v, o->v[i], (size_t)copy_rows * row_bytes, ho_stream(o)) != GSX_HIP_SUCCESS) {
                return gsx_make_error(GSX_ERROR_UNKNOWN, "hip optimizer resize copy failed");
            }
        }
        /* the old moments return to the pool behind the gathers queued above */
        (void)gsx_hip_pool_free(o->m[i], ho_stream(o));
        (void)gsx_hip_pool_free(o->v[i], ho_stream(o));
        o->m[i] = m;
        o->v[i] = v;
        o->rows[i] = new_rows;
    }
    return ho_ok();
}

/* every group's parameter has moved to `new_rows` rows of the moments' width; the moments all
 * have `old_rows` rows (gsx-cpu/optim.c:569-631) */
static gsx_error ho_check_transition(const hip_optim *o, gsx_size_t *old_rows, gsx_size_t *new_rows)
{
    gsx_index_t i = 0;

    for(i = 0; i < o->base.param_group_count; ++i) {
        gsx_size_t rows = 0, width = 0;
        gsx_error error = ho_check_group(o, i);

        if(gsx_error_is_success(error)) error = ho_layout(o->base.param_groups[i].parameter, &rows, &width);
        if(!gsx_error_is_success(error)) return error;
        if(width != o->row_floats[i]) {
            return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer state tensors no longer match the parameter row layout");
        }
        if(i == 0) {
            *old_rows = o->rows[i];
            *new_rows = rows;
        } else if(o->rows[i] != *old_rows || rows != *new_rows) {
            return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer param groups must share the same leading extents");
        }
    }
    return ho_ok();
}

static gsx_error ho_permute(gsx_optim_t optim, gsx_tensor_t permutation)
{
    hip_optim *o = (hip_optim *)optim;
    gsx_size_t count = 0, r = 0;
    int32_t *idx = NULL;
    bool *seen = NULL;
    gsx_index_t i = 0;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(o->base.param_group_count == 0) return ho_ok();
    for(i = 0; i < o->base.param_group_count; ++i) {
        error = ho_check_exact(o, i);
        if(!gsx_error_is_success(error)) return error;
        if(i == 0) count = o->rows[0];
        else if(o->rows[i] != count) {
            return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer param groups must share the same leading extent for permutation");
        }
    }
    error = ho_read_indices(o, permutation, count, "optimizer permutation tensor must be rank-1 int32", &idx);
    if(!gsx_error_is_success(error)) return error;
    seen = (bool *)calloc((size_t)(count > 0 ? count : 1), sizeof(bool));
    if(seen == NULL) {
        free(idx);
        return gsx_make_error(GSX_ERROR_OUT_OF_MEMORY, "failed to allocate optimizer permutation validation bitmap");
    }
    for(r = 0; r < count; ++r) {
        if(idx[r] < 0) {
            error = gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer permutation entries must be non-negative");
        } else if((gsx_size_t)idx[r] >= count) {
            error = gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer permutation entries must be in range");
        } else if(seen[idx[r]]) {
            error = gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer permutation entries must be unique");
        } else {
            seen[idx[r]] = true;
            continue;
        }
        break;
    }
    free(seen);
    free(idx);
    if(!gsx_error_is_success(error)) return error;
    return ho_relayout(o, permutation, count, 0);
}

static gsx_error ho_gather(gsx_optim_t optim, gsx_tensor_t indices)
{
    hip_optim *o = (hip_optim *)optim;
    gsx_size_t old_rows = 0, new_rows = 0, r = 0;
    int32_t *idx = NULL;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(o->base.param_group_count == 0) return ho_ok();
    error = ho_check_transition(o, &old_rows, &new_rows);
    if(!gsx_error_is_success(error)) return error;
    error = ho_read_indices(o, indices, new_rows, "optimizer indices tensor must be rank-1 int32", &idx);
    if(!gsx_error_is_success(error)) return error;
    for(r = 0; r < new_rows; ++r) {
        if(idx[r] < 0 || (gsx_size_t)idx[r] >= old_rows) {
            free(idx);
            return gsx_make_error(GSX_ERROR_INVALID_ARGUMENT, "optimizer gather indices must be in range");
        }
    }
    free(idx);
    return ho_relayout(o, indices, new_rows, 0);
}

static gsx_error ho_resize(gsx_optim_t optim, gsx_size_t new_count)
{
    hip_optim *o = (hip_optim *)optim;
    gsx_size_t old_rows = 0, new_rows = 0;
    gsx_error error = { GSX_ERROR_SUCCESS, NULL };

    if(o->base.param_group_count == 0) return ho_ok();
    error = ho_check_transition(o, &old_rows, &new_rows);
    if(!gsx_error_is_success(error)) return error;
    if(new_rows != new_count) {
        return gsx_make_error(GSX_ERROR_INVALID_STATE, "optimizer resize expects parameter tensors to already expose the target leading extent");
    }
    return ho_relayout(o, NULL, new_count, old_rows < new_count ? old_rows : new_count);
}

gsx_error gsx_hip_plugin_optim_moments(gsx_optim_t optim, gsx_index_t group, float **out_m, float **out_v,
    gsx_size_t *out_rows)
{
    hip_optim *o = (hip_optim *)optim;

    if(optim == NULL || group < 0 || group >= o->base.param_group_count) {
        return gsx_make_error(GSX_ERROR_OUT_OF_RANGE, "optimizer param-group index is out of range");
    }
    *out_m = o->m[group];
    *out_v = o->v[group];
    *out_rows = o->rows[group];
    return ho_ok();
}
