/*
 * gsx_oracle.c - CPU restatement of the gsx CPU backend algorithms on the training hot path.
 *
 * TEST INFRASTRUCTURE (see gsx_oracle.h): the checker for the gfx950 kernels, never part of
 * the product. Compiled like the reference (C11, -O3, no -march => no FMA contraction) so
 * that, on the same inputs, results are bit-identical to the reference CPU backend.
 *
 * Each function cites the reference lines whose arithmetic it restates, operation by
 * operation: the order of float operations is part of the contract (a reordered sum moves
 * alpha across the 1/255 threshold, gsx/src/gsx-cpu/render.c:106-111).
 */
#include "gsx_oracle.h"

#include "../gsx_amd/csrc/gsx_math.h"
#include "../gsx_amd/csrc/tile_cull.h"

#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------------------
 * Constants: gsx/src/gsx-cpu/render.c:85-111, loss.c:120-132.
 * ------------------------------------------------------------------------------------- */
#define SH_C0 0.28209479177387814f
#define SH_C1 0.4886025119029199f
static const float k_sh_c2[5] = { 1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
    -1.0925484305920792f, 0.5462742152960396f };
static const float k_sh_c3[7] = { -0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
    0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f, -0.5900435899266435f };
#define MIN_ABS_Z 1.0e-8f
#define MIN_QUAT_NORM_SQ 1.0e-20f
#define COV2D_DILATION 0.3f
#define POWER_THRESHOLD (-4.5f)
#define MIN_ALPHA (1.0f / 255.0f)
#define OPACITY_LOGIT_CULL (-5.537334267018537f)
#define MAX_FRAGMENT_ALPHA 0.999f
#define T_THRESHOLD 1.0e-4f

typedef struct v3 {
    float x, y, z;
} v3;

typedef struct m3 {
    float m[3][3];
} m3;

typedef struct cam {
    float fx, fy, cx, cy;
    int32_t width, height;
    float qx, qy, qz, qw;
    float tx, ty, tz;
    float near_plane, far_plane;
    float bg[3];
} cam;

static cam cam_from(const float *c)
{
    cam k;

    k.fx = c[0];
    k.fy = c[1];
    k.cx = c[2];
    k.cy = c[3];
    k.width = (int32_t)c[4];
    k.height = (int32_t)c[5];
    k.qx = c[6];
    k.qy = c[7];
    k.qz = c[8];
    k.qw = c[9];
    k.tx = c[10];
    k.ty = c[11];
    k.tz = c[12];
    k.near_plane = c[13];
    k.far_plane = c[14];
    k.bg[0] = c[15];
    k.bg[1] = c[16];
    k.bg[2] = c[17];
    return k;
}

static v3 mk3(float x, float y, float z)
{
    v3 v;

    v.x = x;
    v.y = y;
    v.z = z;
    return v;
}

/* render.c:397-407 */
static float sigmoid_render(float x)
{
    if(x >= 0.0f) {
        float z = expf(-x);
        return 1.0f / (1.0f + z);
    }
    {
        float z = expf(x);
        return z / (1.0f + z);
    }
}

/* render.c:421-451: normalised quaternion, identity below 1e-20 squared norm. */
static int quat_normalize(float qx, float qy, float qz, float qw, float *nx, float *ny, float *nz, float *nw)
{
    float norm_sq = qx * qx + qy * qy + qz * qz + qw * qw;
    float inv_norm;

    if(norm_sq <= MIN_QUAT_NORM_SQ) {
        *nx = 0.0f;
        *ny = 0.0f;
        *nz = 0.0f;
        *nw = 1.0f;
        return 0;
    }
    inv_norm = 1.0f / sqrtf(norm_sq);
    *nx = qx * inv_norm;
    *ny = qy * inv_norm;
    *nz = qz * inv_norm;
    *nw = qw * inv_norm;
    return 1;
}

/* render.c:543-559 (zero-initialised triple-loop product) */
static m3 m3_mul(m3 a, m3 b)
{
    m3 r;
    int i, j, k;

    for(i = 0; i < 3; ++i) {
        for(j = 0; j < 3; ++j) {
            r.m[i][j] = 0.0f;
            for(k = 0; k < 3; ++k) {
                r.m[i][j] += a.m[i][k] * b.m[k][j];
            }
        }
    }
    return r;
}

static m3 m3_t(m3 a)
{
    m3 r;
    int i, j;

    for(i = 0; i < 3; ++i) {
        for(j = 0; j < 3; ++j) {
            r.m[i][j] = a.m[j][i];
        }
    }
    return r;
}

static v3 m3_v(m3 a, v3 v)
{
    return mk3(a.m[0][0] * v.x + a.m[0][1] * v.y + a.m[0][2] * v.z,
        a.m[1][0] * v.x + a.m[1][1] * v.y + a.m[1][2] * v.z,
        a.m[2][0] * v.x + a.m[2][1] * v.y + a.m[2][2] * v.z);
}

/* render.c:561-581 */
static m3 rotation_from_xyzw(float qx_raw, float qy_raw, float qz_raw, float qw_raw)
{
    m3 r;
    float qx, qy, qz, qw;

    (void)quat_normalize(qx_raw, qy_raw, qz_raw, qw_raw, &qx, &qy, &qz, &qw);
    r.m[0][0] = 1.0f - 2.0f * (qy * qy + qz * qz);
    r.m[0][1] = 2.0f * (qx * qy - qw * qz);
    r.m[0][2] = 2.0f * (qx * qz + qw * qy);
    r.m[1][0] = 2.0f * (qx * qy + qw * qz);
    r.m[1][1] = 1.0f - 2.0f * (qx * qx + qz * qz);
    r.m[1][2] = 2.0f * (qy * qz - qw * qx);
    r.m[2][0] = 2.0f * (qx * qz - qw * qy);
    r.m[2][1] = 2.0f * (qy * qz + qw * qx);
    r.m[2][2] = 1.0f - 2.0f * (qx * qx + qy * qy);
    return r;
}

/* render.c:583-601: Sigma = (R S)(R S)^T, S = diag(exp(logscale)). */
static m3 cov3d_from(const float *q, const float *ls)
{
    m3 rs = rotation_from_xyzw(q[0], q[1], q[2], q[3]);
    float sx = expf(ls[0]);
    float sy = expf(ls[1]);
    float sz = expf(ls[2]);
    int row;

    for(row = 0; row < 3; ++row) {
        rs.m[row][0] *= sx;
        rs.m[row][1] *= sy;
        rs.m[row][2] *= sz;
    }
    return m3_mul(rs, m3_t(rs));
}

typedef struct projected {
    float mx, my, a, b, c, depth, xc, yc, zc;
} projected;

/* render.c:611-668: EWA projection without Jacobian clamp, +0.3 dilation. */
static int project(v3 mean, m3 cov3d, const cam *k, m3 w, projected *out)
{
    v3 mc = m3_v(w, mean);
    m3 cov_cam;
    float inv_z, inv_z2, j00, j02, j11, j12, jc00, jc01, jc02, jc11, jc12;

    mc = mk3(mc.x + k->tx, mc.y + k->ty, mc.z + k->tz);
    cov_cam = m3_mul(m3_mul(w, cov3d), m3_t(w));
    if(fabsf(mc.z) < MIN_ABS_Z) {
        memset(out, 0, sizeof(*out));
        return 0;
    }
    inv_z = 1.0f / mc.z;
    inv_z2 = inv_z * inv_z;
    j00 = k->fx * inv_z;
    j02 = -k->fx * mc.x * inv_z2;
    j11 = k->fy * inv_z;
    j12 = -k->fy * mc.y * inv_z2;
    jc00 = j00 * cov_cam.m[0][0] + j02 * cov_cam.m[2][0];
    jc01 = j00 * cov_cam.m[0][1] + j02 * cov_cam.m[2][1];
    jc02 = j00 * cov_cam.m[0][2] + j02 * cov_cam.m[2][2];
    jc11 = j11 * cov_cam.m[1][1] + j12 * cov_cam.m[2][1];
    jc12 = j11 * cov_cam.m[1][2] + j12 * cov_cam.m[2][2];
    out->mx = k->fx * mc.x * inv_z + k->cx;
    out->my = k->fy * mc.y * inv_z + k->cy;
    out->a = jc00 * j00 + jc02 * j02 + COV2D_DILATION;
    out->b = jc01 * j11 + jc02 * j12;
    out->c = jc11 * j11 + jc12 * j12 + COV2D_DILATION;
    out->depth = mc.z;
    out->xc = mc.x;
    out->yc = mc.y;
    out->zc = mc.z;
    return 1;
}

/* render.c:670-694: 3-sigma pixel box from the larger eigenvalue, clamped to the image. */
static void bbox_of(float a, float b, float c, float mx, float my, int32_t width, int32_t height, int32_t *bb)
{
    float trace = a + c;
    float det = a * c - b * b;
    float disc = sqrtf(fmaxf(0.0f, trace * trace * 0.25f - det));
    float l1 = trace * 0.5f + disc;
    float l2 = trace * 0.5f - disc;
    float radius = 3.0f * sqrtf(fmaxf(l1, l2));

    bb[0] = (int32_t)fmaxf(0.0f, floorf(mx - radius));
    bb[1] = (int32_t)fminf((float)(width - 1), ceilf(mx + radius));
    bb[2] = (int32_t)fmaxf(0.0f, floorf(my - radius));
    bb[3] = (int32_t)fminf((float)(height - 1), ceilf(my + radius));
}

static v3 sh_coeff(const float *sh, int64_t g, int count, int idx)
{
    const float *p = sh + ((size_t)g * (size_t)count + (size_t)idx) * 3u;

    return mk3(p[0], p[1], p[2]);
}

static v3 v3_add_scaled(v3 acc, v3 c, float s)
{
    return mk3(acc.x + c.x * s, acc.y + c.y * s, acc.z + c.z * s);
}

/* render.c:730-828: SH colour, clamped at max(c + 0.5, 0). */
static v3 eval_sh(int64_t g, int deg, v3 d, const float *sh0, const float *sh1, const float *sh2, const float *sh3)
{
    v3 r = mk3(SH_C0 * sh0[g * 3 + 0], SH_C0 * sh0[g * 3 + 1], SH_C0 * sh0[g * 3 + 2]);

    if(deg >= 1) {
        float x = d.x, y = d.y, z = d.z;

        r = v3_add_scaled(r, sh_coeff(sh1, g, 3, 0), -SH_C1 * y);
        r = v3_add_scaled(r, sh_coeff(sh1, g, 3, 1), SH_C1 * z);
        r = v3_add_scaled(r, sh_coeff(sh1, g, 3, 2), -SH_C1 * x);
        if(deg >= 2) {
            float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
            float basis2[5];
            int i;

            basis2[0] = k_sh_c2[0] * xy;
            basis2[1] = k_sh_c2[1] * yz;
            basis2[2] = k_sh_c2[2] * (2.0f * zz - xx - yy);
            basis2[3] = k_sh_c2[3] * xz;
            basis2[4] = k_sh_c2[4] * (xx - yy);
            for(i = 0; i < 5; ++i) {
                r = v3_add_scaled(r, sh_coeff(sh2, g, 5, i), basis2[i]);
            }
            if(deg >= 3) {
                float basis3[7];

                basis3[0] = k_sh_c3[0] * y * (3.0f * xx - yy);
                basis3[1] = k_sh_c3[1] * xy * z;
                basis3[2] = k_sh_c3[2] * y * (4.0f * zz - xx - yy);
                basis3[3] = k_sh_c3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
                basis3[4] = k_sh_c3[4] * x * (4.0f * zz - xx - yy);
                basis3[5] = k_sh_c3[5] * z * (xx - yy);
                basis3[6] = k_sh_c3[6] * x * (xx - 3.0f * yy);
                for(i = 0; i < 7; ++i) {
                    r = v3_add_scaled(r, sh_coeff(sh3, g, 7, i), basis3[i]);
                }
            }
        }
    }
    r.x = fmaxf(r.x + 0.5f, 0.0f);
    r.y = fmaxf(r.y + 0.5f, 0.0f);
    r.z = fmaxf(r.z + 0.5f, 0.0f);
    return r;
}

/* render.c:603-609 */
static v3 camera_centre(const cam *k, m3 w)
{
    v3 c = m3_v(m3_t(w), mk3(k->tx, k->ty, k->tz));

    return mk3(c.x * -1.0f, c.y * -1.0f, c.z * -1.0f);
}

typedef struct vis {
    int64_t g;
    int32_t bb[4];
    float rec[ORACLE_REC_FLOATS];
} vis;

/* render.c:850-1016 (count_visible + fill_visible in one pass): culls, projection, bbox,
 * sigmoid opacity and SH colour, in ascending Gaussian order. Returns the visible count. */
static int64_t collect_visible(int64_t n, int deg, const float *mean3d, const float *rot, const float *ls,
    const float *op, const float *sh0, const float *sh1, const float *sh2, const float *sh3, const cam *k,
    vis *out, float *visible_counter)
{
    m3 w = rotation_from_xyzw(k->qx, k->qy, k->qz, k->qw);
    v3 cc = camera_centre(k, w);
    int64_t count = 0;
    int64_t i;

    for(i = 0; i < n; ++i) {
        v3 mean = mk3(mean3d[i * 3 + 0], mean3d[i * 3 + 1], mean3d[i * 3 + 2]);
        m3 cov3d = cov3d_from(rot + i * 4, ls + i * 3);
        projected p;
        float det;
        int32_t bb[4];

        if(op[i] <= OPACITY_LOGIT_CULL) {
            continue;
        }
        if(!project(mean, cov3d, k, w, &p)) {
            continue;
        }
        det = p.a * p.c - p.b * p.b;
        if(p.depth < k->near_plane || p.depth > k->far_plane || det <= 0.0f) {
            continue;
        }
        bbox_of(p.a, p.b, p.c, p.mx, p.my, k->width, k->height, bb);
        if(bb[0] > bb[1] || bb[2] > bb[3]) {
            continue;
        }
        if(visible_counter != NULL) {
            visible_counter[i] += 1.0f;
        }
        if(out != NULL) {
            vis *v = &out[count];
            v3 d;
            v3 col;
            float len;

            v->g = i;
            memcpy(v->bb, bb, sizeof(bb));
            v->rec[ORACLE_REC_MEAN2D_X] = p.mx;
            v->rec[ORACLE_REC_MEAN2D_Y] = p.my;
            v->rec[ORACLE_REC_COV_A] = p.a;
            v->rec[ORACLE_REC_COV_B] = p.b;
            v->rec[ORACLE_REC_COV_C] = p.c;
            v->rec[ORACLE_REC_INV_DET] = 1.0f / det;
            v->rec[ORACLE_REC_DEPTH] = p.depth;
            v->rec[ORACLE_REC_X_CAM] = p.xc;
            v->rec[ORACLE_REC_Y_CAM] = p.yc;
            v->rec[ORACLE_REC_Z_CAM] = p.zc;
            v->rec[ORACLE_REC_RAW_OPACITY] = op[i];
            v->rec[ORACLE_REC_OPACITY] = sigmoid_render(op[i]);
            /* render.c:487-496 normalise(mean - camera centre) */
            d = mk3(mean.x - cc.x, mean.y - cc.y, mean.z - cc.z);
            len = sqrtf(d.x * d.x + d.y * d.y + d.z * d.z);
            if(len <= 0.0f) {
                d = mk3(0.0f, 0.0f, 0.0f);
            } else {
                float s = 1.0f / len;
                d = mk3(d.x * s, d.y * s, d.z * s);
            }
            col = eval_sh(i, deg, d, sh0, sh1, sh2, sh3);
            v->rec[ORACLE_REC_DIR_X] = d.x;
            v->rec[ORACLE_REC_DIR_Y] = d.y;
            v->rec[ORACLE_REC_DIR_Z] = d.z;
            v->rec[ORACLE_REC_COLOR_R] = col.x;
            v->rec[ORACLE_REC_COLOR_G] = col.y;
            v->rec[ORACLE_REC_COLOR_B] = col.z;
        }
        count += 1;
    }
    return count;
}

/* render.c:830-848: total order by (depth, Gaussian index). */
static int cmp_vis(const void *pa, const void *pb)
{
    const vis *a = (const vis *)pa;
    const vis *b = (const vis *)pb;

    if(a->rec[ORACLE_REC_DEPTH] < b->rec[ORACLE_REC_DEPTH]) return -1;
    if(a->rec[ORACLE_REC_DEPTH] > b->rec[ORACLE_REC_DEPTH]) return 1;
    if(a->g < b->g) return -1;
    if(a->g > b->g) return 1;
    return 0;
}

/* Per-visible preprocess output in Gaussian-index order (the order fill_visible emits).
 * out_index[v] = Gaussian index, out_rec[v*ORACLE_REC_FLOATS..], out_bbox[v*4..] =
 * x_min, x_max, y_min, y_max. Returns V. Buffers must hold n entries. */
int64_t oracle_preprocess(int64_t n, int sh_degree, const float *mean3d, const float *rotation,
    const float *logscale, const float *opacity, const float *sh0, const float *sh1, const float *sh2,
    const float *sh3, const float *camera, int64_t *out_index, float *out_rec, int32_t *out_bbox)
{
    cam k = cam_from(camera);
    vis *v = (vis *)malloc(sizeof(vis) * (size_t)(n > 0 ? n : 1));
    int64_t count, i;

    if(v == NULL) return -1;
    count = collect_visible(n, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, &k, v, NULL);
    for(i = 0; i < count; ++i) {
        out_index[i] = v[i].g;
        memcpy(out_rec + i * ORACLE_REC_FLOATS, v[i].rec, sizeof(v[i].rec));
        memcpy(out_bbox + i * 4, v[i].bb, sizeof(v[i].bb));
    }
    free(v);
    return count;
}

/* ---------------------------------------------------------------------------------------
 * Tile restatement (no CPU counterpart; the CPU rasterises per Gaussian bbox,
 * render.c:1035-1079). tiles(g) = { (tx,ty): x_min/T <= tx <= x_max/T, y_min/T <= ty <= y_max/T }
 * key = (ty * ceil(W/T) + tx) << 32 | float_bits(depth), value = Gaussian index, emitted in
 * ascending Gaussian order, then stably sorted by key. Since depth > near > 0, the float
 * bits order like the values, so each tile's list is the CPU (depth, index) order restricted
 * to the Gaussians whose bbox meets the tile.
 * ------------------------------------------------------------------------------------- */
typedef struct kv {
    uint64_t key;
    uint32_t value;
    uint64_t seq;
} kv;

static int cmp_kv(const void *pa, const void *pb)
{
    const kv *a = (const kv *)pa;
    const kv *b = (const kv *)pb;

    if(a->key < b->key) return -1;
    if(a->key > b->key) return 1;
    if(a->seq < b->seq) return -1;
    if(a->seq > b->seq) return 1;
    return 0;
}

/* The row-span constants of visible Gaussian v (gsx_amd/csrc/tile_cull.h), from its conic and
 * box as the kernels form them. */
static gsx_tile_span vis_span(const vis *v)
{
    const float inv_det = v->rec[ORACLE_REC_INV_DET];
    const float inv_a = v->rec[ORACLE_REC_COV_C] * inv_det;
    const float inv_b = -v->rec[ORACLE_REC_COV_B] * inv_det;
    const float inv_c = v->rec[ORACLE_REC_COV_A] * inv_det;

    return gsx_tile_span_make(v->rec[ORACLE_REC_MEAN2D_X], v->rec[ORACLE_REC_MEAN2D_Y], inv_a, inv_b, inv_c,
        v->rec[ORACLE_REC_OPACITY], v->bb[0], v->bb[1], v->bb[2], v->bb[3]);
}

/* The kept tiles [*txa, *txb] of tile row ty of visible Gaussian v (*txa > *txb when none): the
 * tiles holding a pixel column of the box where the row's band may receive a contribution
 * (tile_cull.h). Dropped instances are ones whose pixels all fail the power or alpha cut of
 * render.c:1055-1066, so the per-pixel lists lose only entries that are skipped. */
static void row_tiles(const vis *v, const gsx_tile_span *k, int32_t ty, int32_t tile_size, int32_t *txa, int32_t *txb)
{
    int32_t py0 = ty * tile_size, py1 = ty * tile_size + tile_size - 1;
    int xa, xb;

    if(py0 < v->bb[2]) py0 = v->bb[2];
    if(py1 > v->bb[3]) py1 = v->bb[3];
    gsx_tile_band_columns(k, v->bb[0], v->bb[1], py0, py1, &xa, &xb);
    if(xa > xb) {
        *txa = 1;
        *txb = 0;
    } else {
        *txa = xa / tile_size;
        *txb = xb / tile_size;
    }
}

/* Tile-key restatement (no CPU counterpart): visible Gaussians in Gaussian-index order, each
 * emitting key = tile << 32 | bits(depth) for the kept tiles of its box in row-major order,
 * then a stable sort by key. Per tile this is the CPU's (depth, index) order. Returns the
 * instance count I; writes sorted keys/values when capacity allows (else returns -I-1). */
int64_t oracle_tile_keys(int64_t n, int sh_degree, const float *mean3d, const float *rotation,
    const float *logscale, const float *opacity, const float *sh0, const float *sh1, const float *sh2,
    const float *sh3, const float *camera, int32_t tile_size, int64_t capacity, uint64_t *out_keys,
    uint32_t *out_values)
{
    cam k = cam_from(camera);
    vis *v = (vis *)malloc(sizeof(vis) * (size_t)(n > 0 ? n : 1));
    int64_t count, i, total = 0;
    int32_t tiles_x = (k.width + tile_size - 1) / tile_size;
    kv *pairs;
    int32_t tx, ty;

    if(v == NULL) return -1;
    count = collect_visible(n, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, &k, v, NULL);
    for(i = 0; i < count; ++i) {
        const gsx_tile_span sp = vis_span(&v[i]);
        int32_t txa, txb;

        for(ty = v[i].bb[2] / tile_size; ty <= v[i].bb[3] / tile_size; ++ty) {
            row_tiles(&v[i], &sp, ty, tile_size, &txa, &txb);
            if(txa <= txb) total += txb - txa + 1;
        }
    }
    if(total > capacity) {
        free(v);
        return -total - 1;
    }
    pairs = (kv *)malloc(sizeof(kv) * (size_t)(total > 0 ? total : 1));
    if(pairs == NULL) {
        free(v);
        return -1;
    }
    total = 0;
    for(i = 0; i < count; ++i) {
        uint32_t depth_bits = gsx_f32_bits(v[i].rec[ORACLE_REC_DEPTH]);
        const gsx_tile_span sp = vis_span(&v[i]);
        int32_t txa, txb;

        for(ty = v[i].bb[2] / tile_size; ty <= v[i].bb[3] / tile_size; ++ty) {
            row_tiles(&v[i], &sp, ty, tile_size, &txa, &txb);
            for(tx = txa; tx <= txb; ++tx) {
                uint64_t tile = (uint64_t)ty * (uint64_t)tiles_x + (uint64_t)tx;

                pairs[total].key = (tile << 32) | (uint64_t)depth_bits;
                pairs[total].value = (uint32_t)v[i].g;
                pairs[total].seq = (uint64_t)total;
                total += 1;
            }
        }
    }
    qsort(pairs, (size_t)total, sizeof(kv), cmp_kv);
    for(i = 0; i < total; ++i) {
        out_keys[i] = pairs[i].key;
        out_values[i] = pairs[i].value;
    }
    free(pairs);
    free(v);
    return total;
}

/* The tile test alone, for tests: 1 when the instance is kept. */
float oracle_tile_logf(float x) { return gsx_cull_logf(x); }

int oracle_tile_may_contribute(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity, int px0,
    int px1, int py0, int py1)
{
    return gsx_tile_may_contribute(mx, my, inv_a, inv_b, inv_c, opacity, px0, px1, py0, py1);
}

/* The band columns of tile_cull.h for the Gaussian with pixel box [x0, x1] x [y0, y1] and the
 * band of pixel rows [py0, py1]: out[0] = first, out[1] = last kept column (out[0] > out[1]
 * when none). */
void oracle_tile_band_columns(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity, int x0,
    int x1, int y0, int y1, int py0, int py1, int *out)
{
    const gsx_tile_span k = gsx_tile_span_make(mx, my, inv_a, inv_b, inv_c, opacity, x0, x1, y0, y1);

    gsx_tile_band_columns(&k, x0, x1, py0, py1, &out[0], &out[1]);
}

/* The contribution box of tile_cull.h (gsx_contribution_box) for the Gaussian with pixel box
 * [x0, x1] x [y0, y1]: out = xa, xb, ya, yb (empty when xa > xb or ya > yb). */
void oracle_contribution_box(float mx, float my, float inv_a, float inv_b, float inv_c, float opacity, int x0,
    int x1, int y0, int y1, int *out)
{
    gsx_contribution_box(mx, my, inv_a, inv_b, inv_c, opacity, x0, x1, y0, y1, &out[0], &out[1], &out[2], &out[3]);
}

/* [start, end) of every tile in the sorted key array; empty tiles get (0, 0). */
void oracle_tile_ranges(int64_t instance_count, const uint64_t *keys, int64_t tile_count, uint32_t *out_ranges)
{
    int64_t i;

    memset(out_ranges, 0, sizeof(uint32_t) * 2u * (size_t)tile_count);
    for(i = 0; i < instance_count; ++i) {
        uint64_t tile = keys[i] >> 32;

        if(i == 0 || (keys[i - 1] >> 32) != tile) {
            out_ranges[tile * 2 + 0] = (uint32_t)i;
        }
        if(i == instance_count - 1 || (keys[i + 1] >> 32) != tile) {
            out_ranges[tile * 2 + 1] = (uint32_t)(i + 1);
        }
    }
}

/* ---------------------------------------------------------------------------------------
 * Forward blend: render.c:1018-1088, 1254-1365.
 * out_rgb [3,H,W]; out_t (nullable) [H,W] final transmittance; visible_counter (nullable)
 * incremented as a TRAIN forward does (render.c:980-982).
 * ------------------------------------------------------------------------------------- */
int oracle_render_forward(int64_t n, int sh_degree, const float *mean3d, const float *rotation,
    const float *logscale, const float *opacity, const float *sh0, const float *sh1, const float *sh2,
    const float *sh3, const float *camera, float *out_rgb, float *out_t, float *visible_counter)
{
    cam k = cam_from(camera);
    size_t pixels = (size_t)k.width * (size_t)k.height;
    vis *v = (vis *)malloc(sizeof(vis) * (size_t)(n > 0 ? n : 1));
    float *t = (float *)malloc(sizeof(float) * (pixels > 0 ? pixels : 1));
    int64_t count, vi;
    size_t p;

    if(v == NULL || t == NULL) {
        free(v);
        free(t);
        return -1;
    }
    count = collect_visible(n, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, &k, v,
        visible_counter);
    memset(out_rgb, 0, sizeof(float) * 3u * pixels);
    for(p = 0; p < pixels; ++p) {
        t[p] = 1.0f;
    }
    qsort(v, (size_t)count, sizeof(vis), cmp_vis);
    for(vi = 0; vi < count; ++vi) {
        const float *r = v[vi].rec;
        float inv_a = r[ORACLE_REC_COV_C] * r[ORACLE_REC_INV_DET];
        float inv_b = -r[ORACLE_REC_COV_B] * r[ORACLE_REC_INV_DET];
        float inv_c = r[ORACLE_REC_COV_A] * r[ORACLE_REC_INV_DET];
        int32_t px, py;

        for(py = v[vi].bb[2]; py <= v[vi].bb[3]; ++py) {
            for(px = v[vi].bb[0]; px <= v[vi].bb[1]; ++px) {
                float dx = ((float)px + 0.5f) - r[ORACLE_REC_MEAN2D_X];
                float dy = ((float)py + 0.5f) - r[ORACLE_REC_MEAN2D_Y];
                float power = -0.5f * (inv_a * dx * dx + 2.0f * inv_b * dx * dy + inv_c * dy * dy);
                size_t pix = (size_t)py * (size_t)k.width + (size_t)px;
                float alpha, tb, wgt;

                if(power > 0.0f) power = 0.0f;
                if(power < POWER_THRESHOLD) continue;
                alpha = fminf(MAX_FRAGMENT_ALPHA, r[ORACLE_REC_OPACITY] * expf(power));
                if(alpha < MIN_ALPHA) continue;
                tb = t[pix];
                if(tb < T_THRESHOLD) continue;
                wgt = alpha * tb;
                out_rgb[0 * pixels + pix] += wgt * r[ORACLE_REC_COLOR_R];
                out_rgb[1 * pixels + pix] += wgt * r[ORACLE_REC_COLOR_G];
                out_rgb[2 * pixels + pix] += wgt * r[ORACLE_REC_COLOR_B];
                t[pix] = tb * (1.0f - alpha);
            }
        }
    }
    for(p = 0; p < pixels; ++p) {
        out_rgb[0 * pixels + p] += t[p] * k.bg[0];
        out_rgb[1 * pixels + p] += t[p] * k.bg[1];
        out_rgb[2 * pixels + p] += t[p] * k.bg[2];
    }
    if(out_t != NULL) {
        memcpy(out_t, t, sizeof(float) * pixels);
    }
    free(t);
    free(v);
    return 0;
}

/* ---------------------------------------------------------------------------------------
 * Backward: render.c:1367-1975. Gradient sinks are overwritten (zeroed, then accumulated,
 * render.c:1537-1550). Per-Gaussian accumulation runs back to front exactly as the CPU.
 * ------------------------------------------------------------------------------------- */
typedef struct contrib {
    int32_t pixel;
    float alpha;
    float t_before;
} contrib;

static void add_sh_grad(float *g, int64_t gi, int count, int idx, v3 d)
{
    float *p = g + ((size_t)gi * (size_t)count + (size_t)idx) * 3u;

    p[0] += d.x;
    p[1] += d.y;
    p[2] += d.z;
}

/* render.c:714-728 */
static void add_dir_grad(v3 *ddir, v3 dcol, v3 coeff, float bx, float by, float bz)
{
    float s = dcol.x * coeff.x + dcol.y * coeff.y + dcol.z * coeff.z;

    ddir->x += s * bx;
    ddir->y += s * by;
    ddir->z += s * bz;
}

static v3 v3_scale(v3 a, float s)
{
    return mk3(a.x * s, a.y * s, a.z * s);
}

/* The nine screen-space sums of one Gaussian's contributions (render.c:1603-1606): colour
 * (3), mean2d (2), cov2d (3), opacity. */
typedef struct screen_grad {
    float dc[3];
    float dm[2];
    float dcov[3];
    float dop;
} screen_grad;

/* Conic and d(conic)/d(cov2d) factors of one visible record (render.c:1590-1602). */
typedef struct conic_terms {
    float inv_a, inv_b, inv_c;
    float ca, cb, cc, inv_det2;
} conic_terms;

static conic_terms conic_of(const float *r)
{
    conic_terms c;
    float det;

    c.ca = r[ORACLE_REC_COV_A];
    c.cb = r[ORACLE_REC_COV_B];
    c.cc = r[ORACLE_REC_COV_C];
    c.inv_a = c.cc * r[ORACLE_REC_INV_DET];
    c.inv_b = -c.cb * r[ORACLE_REC_INV_DET];
    c.inv_c = c.ca * r[ORACLE_REC_INV_DET];
    det = c.ca * c.cc - c.cb * c.cb;
    c.inv_det2 = 1.0f / (det * det);
    return c;
}

/* One contribution's terms of the nine sums (render.c:1608-1656), in the CPU's float
 * expressions: out[0..2] colour, [3..4] mean2d, [5..7] cov2d, [8] opacity. Returns whether the
 * opacity term applies (op * G below the alpha cap, render.c:1631-1634). s = the pixel's suffix
 * (the colour behind this contribution). */
static int contrib_terms(const float *r, const conic_terms *c, int32_t px, int32_t py, float dox, float doy,
    float doz, float alpha, float tb, v3 s, float out[9])
{
    float dx = ((float)px + 0.5f) - r[ORACLE_REC_MEAN2D_X];
    float dy = ((float)py + 0.5f) - r[ORACLE_REC_MEAN2D_Y];
    float power = -0.5f * (c->inv_a * dx * dx + 2.0f * c->inv_b * dx * dy + c->inv_c * dy * dy);
    float gv = expf(power > 0.0f ? 0.0f : power);
    float wgt = alpha * tb;
    float dalpha = tb * (r[ORACLE_REC_COLOR_R] * dox + r[ORACLE_REC_COLOR_G] * doy + r[ORACLE_REC_COLOR_B] * doz);
    float dg = 0.0f, dpow, dia, dib, dic;
    int op_ok = 0;

    out[0] = wgt * dox;
    out[1] = wgt * doy;
    out[2] = wgt * doz;
    if(fabsf(1.0f - alpha) > 1.0e-6f) {
        dalpha -= (s.x * dox + s.y * doy + s.z * doz) / (1.0f - alpha);
    }
    out[8] = 0.0f;
    if(r[ORACLE_REC_OPACITY] * gv < MAX_FRAGMENT_ALPHA) {
        dg = dalpha * r[ORACLE_REC_OPACITY];
        out[8] = dalpha * gv;
        op_ok = 1;
    }
    dpow = dg * gv;
    out[3] = dpow * (c->inv_a * dx + c->inv_b * dy);
    out[4] = dpow * (c->inv_b * dx + c->inv_c * dy);
    dia = dpow * (-0.5f * dx * dx);
    dib = dpow * (-dx * dy);
    dic = dpow * (-0.5f * dy * dy);
    out[5] = dia * (-c->cc * c->cc * c->inv_det2) + dib * (c->cb * c->cc * c->inv_det2)
        + dic * (-c->cb * c->cb * c->inv_det2);
    out[6] = dia * (2.0f * c->cb * c->cc * c->inv_det2) + dib * (-(c->ca * c->cc + c->cb * c->cb) * c->inv_det2)
        + dic * (2.0f * c->ca * c->cb * c->inv_det2);
    out[7] = dia * (-c->cb * c->cb * c->inv_det2) + dib * (c->ca * c->cb * c->inv_det2)
        + dic * (-c->ca * c->ca * c->inv_det2);
    return op_ok;
}

/* Gradient sinks of a backward call. */
typedef struct grad_sinks {
    float *mean3d, *rotation, *logscale, *opacity, *sh0, *sh1, *sh2, *sh3;
} grad_sinks;

/* Parameter gradients of one visible Gaussian from its nine sums (render.c:1667-1969): colour
 * clamp mask, SH and view-direction terms, opacity through the sigmoid, mean through the
 * projection, cov2d -> cov3d -> scale and rotation (through the quaternion normalisation),
 * and the Jacobian's dependence on the camera-space mean. Adds into the sinks. */
static void project_grad_tail(const vis *e, const screen_grad *sg, int deg, const cam *kp, m3 w, v3 cc,
    const float *mean3d, const float *rotation, const float *logscale, const float *sh1, const float *sh2,
    const float *sh3, const grad_sinks *gs)
{
    const cam k = *kp;
    const float *r = e->rec;
    const int64_t gi = e->g;
    const float dcx = sg->dc[0], dcy = sg->dc[1], dcz = sg->dc[2], dmx = sg->dm[0], dmy = sg->dm[1];
    const float dca = sg->dcov[0], dcb = sg->dcov[1], dcc = sg->dcov[2], dop = sg->dop;
    const float *q = rotation + gi * 4;
    const float *ls = logscale + gi * 3;
    m3 cov3d = cov3d_from(q, ls);
    m3 rot = rotation_from_xyzw(q[0], q[1], q[2], q[3]);
    m3 srot = rot;
    m3 d_cov3d, d_rs, d_r, dsum;
    float sx = expf(ls[0]), sy = expf(ls[1]), sz = expf(ls[2]);
    float zc = r[ORACLE_REC_Z_CAM], xc = r[ORACLE_REC_X_CAM], yc = r[ORACLE_REC_Y_CAM];
    float j00 = k.fx / zc;
    float j02 = -k.fx * xc / (zc * zc);
    float j11 = k.fy / zc;
    float j12 = -k.fy * yc / (zc * zc);
    float mm[2][3];
    int row, col;
    float *g_mean3d = gs->mean3d, *g_rotation = gs->rotation, *g_logscale = gs->logscale;
    float *g_opacity = gs->opacity, *g_sh0 = gs->sh0, *g_sh1 = gs->sh1, *g_sh2 = gs->sh2, *g_sh3 = gs->sh3;

    /* render.c:1667-1828: colour clamp mask, SH and view-direction gradients. */
    {
        v3 dcol = mk3(dcx * (r[ORACLE_REC_COLOR_R] > 0.0f ? 1.0f : 0.0f),
            dcy * (r[ORACLE_REC_COLOR_G] > 0.0f ? 1.0f : 0.0f),
            dcz * (r[ORACLE_REC_COLOR_B] > 0.0f ? 1.0f : 0.0f));
        v3 ddir = mk3(0.0f, 0.0f, 0.0f);
        float x = r[ORACLE_REC_DIR_X], y = r[ORACLE_REC_DIR_Y], z = r[ORACLE_REC_DIR_Z];
        float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;

        g_sh0[gi * 3 + 0] += SH_C0 * dcol.x;
        g_sh0[gi * 3 + 1] += SH_C0 * dcol.y;
        g_sh0[gi * 3 + 2] += SH_C0 * dcol.z;
        if(deg >= 1 && g_sh1 != NULL) {
            add_sh_grad(g_sh1, gi, 3, 0, v3_scale(dcol, -SH_C1 * y));
            add_sh_grad(g_sh1, gi, 3, 1, v3_scale(dcol, SH_C1 * z));
            add_sh_grad(g_sh1, gi, 3, 2, v3_scale(dcol, -SH_C1 * x));
            add_dir_grad(&ddir, dcol, sh_coeff(sh1, gi, 3, 0), 0.0f, -SH_C1, 0.0f);
            add_dir_grad(&ddir, dcol, sh_coeff(sh1, gi, 3, 1), 0.0f, 0.0f, SH_C1);
            add_dir_grad(&ddir, dcol, sh_coeff(sh1, gi, 3, 2), -SH_C1, 0.0f, 0.0f);
        }
        if(deg >= 2 && g_sh2 != NULL) {
            add_sh_grad(g_sh2, gi, 5, 0, v3_scale(dcol, k_sh_c2[0] * xy));
            add_dir_grad(&ddir, dcol, sh_coeff(sh2, gi, 5, 0), k_sh_c2[0] * y, k_sh_c2[0] * x, 0.0f);
            add_sh_grad(g_sh2, gi, 5, 1, v3_scale(dcol, k_sh_c2[1] * yz));
            add_dir_grad(&ddir, dcol, sh_coeff(sh2, gi, 5, 1), 0.0f, k_sh_c2[1] * z, k_sh_c2[1] * y);
            add_sh_grad(g_sh2, gi, 5, 2, v3_scale(dcol, k_sh_c2[2] * (2.0f * zz - xx - yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh2, gi, 5, 2), -2.0f * k_sh_c2[2] * x, -2.0f * k_sh_c2[2] * y,
                4.0f * k_sh_c2[2] * z);
            add_sh_grad(g_sh2, gi, 5, 3, v3_scale(dcol, k_sh_c2[3] * xz));
            add_dir_grad(&ddir, dcol, sh_coeff(sh2, gi, 5, 3), k_sh_c2[3] * z, 0.0f, k_sh_c2[3] * x);
            add_sh_grad(g_sh2, gi, 5, 4, v3_scale(dcol, k_sh_c2[4] * (xx - yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh2, gi, 5, 4), 2.0f * k_sh_c2[4] * x, -2.0f * k_sh_c2[4] * y, 0.0f);
        }
        if(deg >= 3 && g_sh3 != NULL) {
            add_sh_grad(g_sh3, gi, 7, 0, v3_scale(dcol, k_sh_c3[0] * y * (3.0f * xx - yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 0), 6.0f * k_sh_c3[0] * x * y,
                3.0f * k_sh_c3[0] * (xx - yy), 0.0f);
            add_sh_grad(g_sh3, gi, 7, 1, v3_scale(dcol, k_sh_c3[1] * xy * z));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 1), k_sh_c3[1] * y * z, k_sh_c3[1] * x * z,
                k_sh_c3[1] * xy);
            add_sh_grad(g_sh3, gi, 7, 2, v3_scale(dcol, k_sh_c3[2] * y * (4.0f * zz - xx - yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 2), -2.0f * k_sh_c3[2] * x * y,
                k_sh_c3[2] * (4.0f * zz - xx - 3.0f * yy), 8.0f * k_sh_c3[2] * y * z);
            add_sh_grad(g_sh3, gi, 7, 3, v3_scale(dcol, k_sh_c3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 3), -6.0f * k_sh_c3[3] * x * z,
                -6.0f * k_sh_c3[3] * y * z, k_sh_c3[3] * (6.0f * zz - 3.0f * xx - 3.0f * yy));
            add_sh_grad(g_sh3, gi, 7, 4, v3_scale(dcol, k_sh_c3[4] * x * (4.0f * zz - xx - yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 4), k_sh_c3[4] * (4.0f * zz - 3.0f * xx - yy),
                -2.0f * k_sh_c3[4] * x * y, 8.0f * k_sh_c3[4] * x * z);
            add_sh_grad(g_sh3, gi, 7, 5, v3_scale(dcol, k_sh_c3[5] * z * (xx - yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 5), 2.0f * k_sh_c3[5] * x * z,
                -2.0f * k_sh_c3[5] * y * z, k_sh_c3[5] * (xx - yy));
            add_sh_grad(g_sh3, gi, 7, 6, v3_scale(dcol, k_sh_c3[6] * x * (xx - 3.0f * yy)));
            add_dir_grad(&ddir, dcol, sh_coeff(sh3, gi, 7, 6), 3.0f * k_sh_c3[6] * (xx - yy),
                -6.0f * k_sh_c3[6] * x * y, 0.0f);
        }
        if(deg >= 1) {
            v3 view = mk3(mean3d[gi * 3 + 0] - cc.x, mean3d[gi * 3 + 1] - cc.y, mean3d[gi * 3 + 2] - cc.z);
            float vn = sqrtf(view.x * view.x + view.y * view.y + view.z * view.z);

            if(vn > 0.0f) {
                float dd = ddir.x * x + ddir.y * y + ddir.z * z;
                v3 dv = mk3(ddir.x - x * dd, ddir.y - y * dd, ddir.z - z * dd);
                float s = 1.0f / vn;

                g_mean3d[gi * 3 + 0] += dv.x * s;
                g_mean3d[gi * 3 + 1] += dv.y * s;
                g_mean3d[gi * 3 + 2] += dv.z * s;
            }
        }
    }
    /* render.c:1830 */
    {
        float sg = sigmoid_render(r[ORACLE_REC_RAW_OPACITY]);

        g_opacity[gi] += dop * (sg * (1.0f - sg));
    }
    /* render.c:1832-1845 */
    {
        float inv_z = 1.0f / zc;
        float inv_z2 = inv_z * inv_z;
        v3 dmc = mk3(dmx * k.fx * inv_z, dmy * k.fy * inv_z,
            dmx * (-k.fx * xc * inv_z2) + dmy * (-k.fy * yc * inv_z2));
        v3 dmw = m3_v(m3_t(w), dmc);

        g_mean3d[gi * 3 + 0] += dmw.x;
        g_mean3d[gi * 3 + 1] += dmw.y;
        g_mean3d[gi * 3 + 2] += dmw.z;
    }
    /* render.c:1847-1875 */
    for(col = 0; col < 3; ++col) {
        mm[0][col] = j00 * w.m[0][col] + j02 * w.m[2][col];
        mm[1][col] = j11 * w.m[1][col] + j12 * w.m[2][col];
    }
    for(row = 0; row < 3; ++row) {
        for(col = 0; col < 3; ++col) {
            d_cov3d.m[row][col] = mm[0][row] * (dca * mm[0][col] + 0.5f * dcb * mm[1][col])
                + mm[1][row] * (0.5f * dcb * mm[0][col] + dcc * mm[1][col]);
        }
    }
    for(row = 0; row < 3; ++row) {
        srot.m[row][0] *= sx;
        srot.m[row][1] *= sy;
        srot.m[row][2] *= sz;
    }
    for(row = 0; row < 3; ++row) {
        for(col = 0; col < 3; ++col) {
            dsum.m[row][col] = d_cov3d.m[row][col] + d_cov3d.m[col][row];
        }
    }
    d_rs = m3_mul(dsum, srot);
    g_logscale[gi * 3 + 0] += (d_rs.m[0][0] * rot.m[0][0] + d_rs.m[1][0] * rot.m[1][0] + d_rs.m[2][0] * rot.m[2][0]) * sx;
    g_logscale[gi * 3 + 1] += (d_rs.m[0][1] * rot.m[0][1] + d_rs.m[1][1] * rot.m[1][1] + d_rs.m[2][1] * rot.m[2][1]) * sy;
    g_logscale[gi * 3 + 2] += (d_rs.m[0][2] * rot.m[0][2] + d_rs.m[1][2] * rot.m[1][2] + d_rs.m[2][2] * rot.m[2][2]) * sz;
    for(row = 0; row < 3; ++row) {
        d_r.m[row][0] = d_rs.m[row][0] * sx;
        d_r.m[row][1] = d_rs.m[row][1] * sy;
        d_r.m[row][2] = d_rs.m[row][2] * sz;
    }
    /* render.c:1877-1937: through the quaternion normalisation. */
    {
        float nx, ny, nz, nw;

        if(quat_normalize(q[0], q[1], q[2], q[3], &nx, &ny, &nz, &nw)) {
            float inv_norm = 1.0f / sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
            float dqw = 0.0f, dqx = 0.0f, dqy = 0.0f, dqz = 0.0f, dot;

            dqw += d_r.m[0][1] * (-2.0f * nz);
            dqw += d_r.m[0][2] * (2.0f * ny);
            dqw += d_r.m[1][0] * (2.0f * nz);
            dqw += d_r.m[1][2] * (-2.0f * nx);
            dqw += d_r.m[2][0] * (-2.0f * ny);
            dqw += d_r.m[2][1] * (2.0f * nx);

            dqx += d_r.m[0][1] * (2.0f * ny);
            dqx += d_r.m[0][2] * (2.0f * nz);
            dqx += d_r.m[1][0] * (2.0f * ny);
            dqx += d_r.m[1][1] * (-4.0f * nx);
            dqx += d_r.m[1][2] * (-2.0f * nw);
            dqx += d_r.m[2][0] * (2.0f * nz);
            dqx += d_r.m[2][1] * (2.0f * nw);
            dqx += d_r.m[2][2] * (-4.0f * nx);

            dqy += d_r.m[0][0] * (-4.0f * ny);
            dqy += d_r.m[0][1] * (2.0f * nx);
            dqy += d_r.m[0][2] * (2.0f * nw);
            dqy += d_r.m[1][0] * (2.0f * nx);
            dqy += d_r.m[1][2] * (2.0f * nz);
            dqy += d_r.m[2][0] * (-2.0f * nw);
            dqy += d_r.m[2][1] * (2.0f * nz);
            dqy += d_r.m[2][2] * (-4.0f * ny);

            dqz += d_r.m[0][0] * (-4.0f * nz);
            dqz += d_r.m[0][1] * (-2.0f * nw);
            dqz += d_r.m[0][2] * (2.0f * nx);
            dqz += d_r.m[1][0] * (2.0f * nw);
            dqz += d_r.m[1][1] * (-4.0f * nz);
            dqz += d_r.m[1][2] * (2.0f * ny);
            dqz += d_r.m[2][0] * (2.0f * nx);
            dqz += d_r.m[2][1] * (2.0f * ny);

            dot = nx * dqx + ny * dqy + nz * dqz + nw * dqw;
            g_rotation[gi * 4 + 0] += (dqx - nx * dot) * inv_norm;
            g_rotation[gi * 4 + 1] += (dqy - ny * dot) * inv_norm;
            g_rotation[gi * 4 + 2] += (dqz - nz * dot) * inv_norm;
            g_rotation[gi * 4 + 3] += (dqw - nw * dot) * inv_norm;
        }
    }
    /* render.c:1939-1969: the Jacobian's dependence on the camera-space mean. */
    {
        m3 cov_cam = m3_mul(m3_mul(w, cov3d), m3_t(w));
        float dj[2][3];
        float inv_z = 1.0f / zc;
        float inv_z2 = inv_z * inv_z;
        float inv_z3 = inv_z2 * inv_z;
        v3 dmj, dmwj;

        for(col = 0; col < 3; ++col) {
            dj[0][col] = 2.0f * dca * (j00 * cov_cam.m[0][col] + j02 * cov_cam.m[2][col])
                + dcb * (j11 * cov_cam.m[1][col] + j12 * cov_cam.m[2][col]);
            dj[1][col] = dcb * (j00 * cov_cam.m[0][col] + j02 * cov_cam.m[2][col])
                + 2.0f * dcc * (j11 * cov_cam.m[1][col] + j12 * cov_cam.m[2][col]);
        }
        dmj.x = dj[0][2] * (-k.fx * inv_z2);
        dmj.y = dj[1][2] * (-k.fy * inv_z2);
        dmj.z = dj[0][0] * (-k.fx * inv_z2) + dj[0][2] * (2.0f * k.fx * xc * inv_z3)
            + dj[1][1] * (-k.fy * inv_z2) + dj[1][2] * (2.0f * k.fy * yc * inv_z3);
        dmwj = m3_v(m3_t(w), dmj);
        g_mean3d[gi * 3 + 0] += dmwj.x;
        g_mean3d[gi * 3 + 1] += dmwj.y;
        g_mean3d[gi * 3 + 2] += dmwj.z;
    }
}

int oracle_render_backward(int64_t n, int deg, const float *mean3d, const float *rotation, const float *logscale,
    const float *opacity, const float *sh0, const float *sh1, const float *sh2, const float *sh3,
    const float *camera, const float *grad_rgb, float *g_mean3d, float *g_rotation, float *g_logscale,
    float *g_opacity, float *g_sh0, float *g_sh1, float *g_sh2, float *g_sh3)
{
    cam k = cam_from(camera);
    m3 w = rotation_from_xyzw(k.qx, k.qy, k.qz, k.qw);
    v3 cc = camera_centre(&k, w);
    size_t pixels = (size_t)k.width * (size_t)k.height;
    vis *v = (vis *)malloc(sizeof(vis) * (size_t)(n > 0 ? n : 1));
    float *t = (float *)malloc(sizeof(float) * (pixels > 0 ? pixels : 1));
    v3 *suffix = (v3 *)malloc(sizeof(v3) * (pixels > 0 ? pixels : 1));
    int64_t *offsets = NULL;
    contrib *contribs = NULL;
    int64_t count, vi, capacity = 0, total = 0;
    size_t p;
    const grad_sinks gs = { g_mean3d, g_rotation, g_logscale, g_opacity, g_sh0, g_sh1, g_sh2, g_sh3 };

    if(v == NULL || t == NULL || suffix == NULL) {
        free(v);
        free(t);
        free(suffix);
        return -1;
    }
    count = collect_visible(n, deg, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, &k, v, NULL);
    for(vi = 0; vi < count; ++vi) {
        capacity += (int64_t)(v[vi].bb[1] - v[vi].bb[0] + 1) * (int64_t)(v[vi].bb[3] - v[vi].bb[2] + 1);
    }
    offsets = (int64_t *)malloc(sizeof(int64_t) * (size_t)(count + 1));
    contribs = (contrib *)malloc(sizeof(contrib) * (size_t)(capacity > 0 ? capacity : 1));
    if(offsets == NULL || contribs == NULL) {
        free(v);
        free(t);
        free(suffix);
        free(offsets);
        free(contribs);
        return -1;
    }
    qsort(v, (size_t)count, sizeof(vis), cmp_vis);
    for(p = 0; p < pixels; ++p) {
        t[p] = 1.0f;
    }
    /* render.c:1476-1515: re-raster, recording (alpha, T_before) per contribution. */
    for(vi = 0; vi < count; ++vi) {
        const float *r = v[vi].rec;
        float inv_a = r[ORACLE_REC_COV_C] * r[ORACLE_REC_INV_DET];
        float inv_b = -r[ORACLE_REC_COV_B] * r[ORACLE_REC_INV_DET];
        float inv_c = r[ORACLE_REC_COV_A] * r[ORACLE_REC_INV_DET];
        int32_t px, py;

        offsets[vi] = total;
        for(py = v[vi].bb[2]; py <= v[vi].bb[3]; ++py) {
            for(px = v[vi].bb[0]; px <= v[vi].bb[1]; ++px) {
                float dx = ((float)px + 0.5f) - r[ORACLE_REC_MEAN2D_X];
                float dy = ((float)py + 0.5f) - r[ORACLE_REC_MEAN2D_Y];
                float power = -0.5f * (inv_a * dx * dx + 2.0f * inv_b * dx * dy + inv_c * dy * dy);
                size_t pix = (size_t)py * (size_t)k.width + (size_t)px;
                float tb = t[pix];
                float alpha;

                if(power > 0.0f) power = 0.0f;
                if(power < POWER_THRESHOLD) continue;
                alpha = fminf(MAX_FRAGMENT_ALPHA, r[ORACLE_REC_OPACITY] * expf(power));
                if(alpha < MIN_ALPHA || tb < T_THRESHOLD) continue;
                contribs[total].pixel = (int32_t)pix;
                contribs[total].alpha = alpha;
                contribs[total].t_before = tb;
                total += 1;
                t[pix] = tb * (1.0f - alpha);
            }
        }
    }
    offsets[count] = total;

    memset(g_mean3d, 0, sizeof(float) * 3u * (size_t)n);
    memset(g_rotation, 0, sizeof(float) * 4u * (size_t)n);
    memset(g_logscale, 0, sizeof(float) * 3u * (size_t)n);
    memset(g_sh0, 0, sizeof(float) * 3u * (size_t)n);
    memset(g_opacity, 0, sizeof(float) * (size_t)n);
    if(deg >= 1 && g_sh1 != NULL) memset(g_sh1, 0, sizeof(float) * 9u * (size_t)n);
    if(deg >= 2 && g_sh2 != NULL) memset(g_sh2, 0, sizeof(float) * 15u * (size_t)n);
    if(deg >= 3 && g_sh3 != NULL) memset(g_sh3, 0, sizeof(float) * 21u * (size_t)n);
    for(p = 0; p < pixels; ++p) {
        suffix[p] = mk3(t[p] * k.bg[0], t[p] * k.bg[1], t[p] * k.bg[2]);
    }

    for(vi = count; vi > 0; --vi) {
        const vis *e = &v[vi - 1];
        const float *r = e->rec;
        const conic_terms ct = conic_of(r);
        screen_grad sg;
        int64_t ci;

        memset(&sg, 0, sizeof(sg));
        /* render.c:1608-1656 */
        for(ci = offsets[vi - 1]; ci < offsets[vi]; ++ci) {
            const contrib *c = &contribs[ci];
            size_t pix = (size_t)c->pixel;
            float t9[9];

            if(contrib_terms(r, &ct, c->pixel % k.width, c->pixel / k.width, grad_rgb[0 * pixels + pix],
                   grad_rgb[1 * pixels + pix], grad_rgb[2 * pixels + pix], c->alpha, c->t_before, suffix[pix], t9)) {
                sg.dop += t9[8];
            }
            sg.dc[0] += t9[0];
            sg.dc[1] += t9[1];
            sg.dc[2] += t9[2];
            sg.dm[0] += t9[3];
            sg.dm[1] += t9[4];
            sg.dcov[0] += t9[5];
            sg.dcov[1] += t9[6];
            sg.dcov[2] += t9[7];
        }
        /* render.c:1658-1665 */
        for(ci = offsets[vi - 1]; ci < offsets[vi]; ++ci) {
            size_t pix = (size_t)contribs[ci].pixel;
            float wgt = contribs[ci].alpha * contribs[ci].t_before;

            suffix[pix].x += wgt * r[ORACLE_REC_COLOR_R];
            suffix[pix].y += wgt * r[ORACLE_REC_COLOR_G];
            suffix[pix].z += wgt * r[ORACLE_REC_COLOR_B];
        }
        project_grad_tail(e, &sg, deg, &k, w, cc, mean3d, rotation, logscale, sh1, sh2, sh3, &gs);
    }
    free(contribs);
    free(offsets);
    free(suffix);
    free(t);
    free(v);
    return 0;
}

/* ---------------------------------------------------------------------------------------
 * Losses: gsx/src/gsx-cpu/loss.c:316-709, gradient scale gsx-tensor-helpers.h:236-244.
 * Images are [outer, C, H, W] CHW float32; map and grad are accumulators.
 * ------------------------------------------------------------------------------------- */
void oracle_loss_l1(int64_t count, const float *pred, const float *target, float scale, float grad_scale,
    float *loss_map, float *grad)
{
    int64_t i;

    for(i = 0; i < count; ++i) {
        float d = pred[i] - target[i];

        if(loss_map != NULL) {
            loss_map[i] += scale * fabsf(d);
        }
        if(grad != NULL) {
            float s = 0.0f;

            if(d > 0.0f) s = 1.0f;
            else if(d < 0.0f) s = -1.0f;
            grad[i] += s * grad_scale;
        }
    }
}

void oracle_loss_mse(int64_t count, const float *pred, const float *target, float scale, float grad_scale,
    float *loss_map, float *grad)
{
    int64_t i;

    for(i = 0; i < count; ++i) {
        float d = pred[i] - target[i];

        if(loss_map != NULL) {
            loss_map[i] += scale * (d * d);
        }
        if(grad != NULL) {
            grad[i] += 2.0f * d * grad_scale;
        }
    }
}

static const double k_ssim_w[11] = { 0.001028380123898387, 0.0075987582094967365, 0.036000773310661316,
    0.10936068743467331, 0.21300552785396576, 0.26601171493530273, 0.21300552785396576, 0.10936068743467331,
    0.036000773310661316, 0.0075987582094967365, 0.001028380123898387 };

/* loss.c:397-556 and :632-709: direct 2D 11x11 window in float64 with zero padding;
 * C1 = 0.01^2, C2 = 0.03^2; 5-pixel boundary set to 0 in the map; dm/dmu1, dm/dsigma1^2,
 * dm/dsigma12 convolved again for the gradient. grad_scale is already normalised. */
int oracle_loss_ssim(int64_t outer, int64_t channels, int64_t height, int64_t width, const float *pred,
    const float *target, float scale, float grad_scale, float *loss_map, float *grad)
{
    int64_t plane = height * width;
    int64_t total = outer * channels * plane;
    double *dmu = NULL, *ds1 = NULL, *ds12 = NULL;
    int64_t o, y, x;
    const double ls = (double)scale;
    const double gs = (double)grad_scale;

    if(grad != NULL) {
        dmu = (double *)calloc((size_t)total, sizeof(double));
        ds1 = (double *)calloc((size_t)total, sizeof(double));
        ds12 = (double *)calloc((size_t)total, sizeof(double));
        if(dmu == NULL || ds1 == NULL || ds12 == NULL) {
            free(dmu);
            free(ds1);
            free(ds12);
            return -1;
        }
    }
    for(o = 0; o < outer * channels; ++o) {
        const float *pp = pred + o * plane;
        const float *tp = target + o * plane;

        for(y = 0; y < height; ++y) {
            for(x = 0; x < width; ++x) {
                double mu1 = 0.0, mu2 = 0.0, ex2 = 0.0, ey2 = 0.0, exy = 0.0;
                int64_t ky, kx, idx = o * plane + y * width + x;
                double m1s, m2s, s1, s2, s12, a, b, ct, dt, ssim;
                int boundary = y < 5 || y >= height - 5 || x < 5 || x >= width - 5;

                for(ky = -5; ky <= 5; ++ky) {
                    double wy = k_ssim_w[ky + 5];

                    for(kx = -5; kx <= 5; ++kx) {
                        double wgt = wy * k_ssim_w[kx + 5];
                        int64_t yy = y + ky, xx = x + kx;
                        double ps = 0.0, ts = 0.0;

                        if(yy >= 0 && xx >= 0 && yy < height && xx < width) {
                            ps = (double)pp[yy * width + xx];
                            ts = (double)tp[yy * width + xx];
                        }
                        mu1 += ps * wgt;
                        mu2 += ts * wgt;
                        ex2 += ps * ps * wgt;
                        ey2 += ts * ts * wgt;
                        exy += ps * ts * wgt;
                    }
                }
                m1s = mu1 * mu1;
                m2s = mu2 * mu2;
                s1 = ex2 - m1s;
                s2 = ey2 - m2s;
                s12 = exy - mu1 * mu2;
                a = m1s + m2s + 0.01 * 0.01;
                b = s1 + s2 + 0.03 * 0.03;
                ct = 2.0 * mu1 * mu2 + 0.01 * 0.01;
                dt = 2.0 * s12 + 0.03 * 0.03;
                ssim = (a * b) == 0.0 ? 1.0 : (ct * dt) / (a * b);
                if(loss_map != NULL) {
                    if(boundary) {
                        loss_map[idx] = 0.0f;
                    } else {
                        loss_map[idx] += (float)((1.0 - ssim) * ls);
                    }
                }
                if(grad != NULL) {
                    if(boundary || a == 0.0 || b == 0.0) {
                        dmu[idx] = 0.0;
                        ds1[idx] = 0.0;
                        ds12[idx] = 0.0;
                    } else {
                        double ab = a * b, aab = a * ab, abb = ab * b;

                        dmu[idx] = (2.0 * mu2 * dt) / ab - (2.0 * mu2 * ct) / ab - (2.0 * mu1 * ct * dt) / aab
                            + (2.0 * mu1 * ct * dt) / abb;
                        ds1[idx] = -(ct * dt) / abb;
                        ds12[idx] = (2.0 * ct) / ab;
                    }
                }
            }
        }
    }
    if(grad != NULL) {
        for(o = 0; o < outer * channels; ++o) {
            for(y = 0; y < height; ++y) {
                for(x = 0; x < width; ++x) {
                    double cm = 0.0, c1 = 0.0, c12 = 0.0;
                    int64_t ky, kx, idx = o * plane + y * width + x;

                    for(ky = -5; ky <= 5; ++ky) {
                        double wy = k_ssim_w[ky + 5];

                        for(kx = -5; kx <= 5; ++kx) {
                            double wgt = wy * k_ssim_w[kx + 5];
                            int64_t yy = y + ky, xx = x + kx;
                            double a = 0.0, b = 0.0, c = 0.0;

                            if(yy >= 0 && xx >= 0 && yy < height && xx < width) {
                                int64_t j = o * plane + yy * width + xx;

                                a = dmu[j];
                                b = ds1[j];
                                c = ds12[j];
                            }
                            cm += a * wgt;
                            c1 += b * wgt;
                            c12 += c * wgt;
                        }
                    }
                    grad[idx] += (float)(-(cm + 2.0 * (double)pred[idx] * c1 + (double)target[idx] * c12) * gs);
                }
            }
        }
    }
    free(dmu);
    free(ds1);
    free(ds12);
    return 0;
}

/* ---------------------------------------------------------------------------------------
 * Adam: gsx/src/gsx-cpu/optim.c:712-780. `step` is the post-increment step count.
 * ------------------------------------------------------------------------------------- */
void oracle_adam_step(int64_t count, float *param, const float *grad, float *m, float *v, float lr, float beta1,
    float beta2, float weight_decay, float epsilon, float max_grad, int64_t step)
{
    double bc1 = 1.0 - pow((double)beta1, (double)step);
    double bc2 = 1.0 - pow((double)beta2, (double)step);
    int64_t i;

    for(i = 0; i < count; ++i) {
        float g = grad[i];
        float m1, v1, mh, vh, p;

        if(max_grad > 0.0f) {
            if(g > max_grad) g = max_grad;
            else if(g < -max_grad) g = -max_grad;
        }
        m1 = beta1 * m[i] + (1.0f - beta1) * g;
        v1 = beta2 * v[i] + (1.0f - beta2) * g * g;
        mh = (float)((double)m1 / bc1);
        vh = (float)((double)v1 / bc2);
        p = param[i];
        m[i] = m1;
        v[i] = v1;
        if(weight_decay > 0.0f) {
            p -= lr * weight_decay * p;
        }
        p -= lr * (mh / (sqrtf(vh) + epsilon));
        param[i] = p;
    }
}

/* ---------------------------------------------------------------------------------------
 * Row gather: gsx/src/gsx-cpu/core.c:1248-1333. Returns 0, or -1 for an index out of range.
 * ------------------------------------------------------------------------------------- */
int oracle_gather_rows(const void *src, int64_t src_rows, int64_t row_bytes, const int32_t *index, int64_t count,
    void *dst)
{
    int64_t i;

    for(i = 0; i < count; ++i) {
        if(index[i] < 0 || index[i] >= src_rows) {
            return -1;
        }
        memcpy((unsigned char *)dst + i * row_bytes, (const unsigned char *)src + (int64_t)index[i] * row_bytes,
            (size_t)row_bytes);
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------
 * ADC default / ABSGS refine: gsx/src/gsx-cpu/adc/default.c:160-527, adc.c:48-80,229-248,
 * 491-559, host math gsx/src/gsx-core.c:2915-2940, Box-Muller gsx/src/gsx-random.c:86-112.
 * Fields are SH0-only SoA arrays with capacity for the grown set. The optimizer moments of
 * grown rows are zero and of kept rows are gathered; moments are passed as 5 (m, v) pairs
 * over the same row layout (mean3d 3, rotation 4, logscale 3, opacity 1, sh0 3 floats).
 * ------------------------------------------------------------------------------------- */
typedef struct oracle_adc_params {
    int32_t algorithm; /* 0 default, 1 absgs */
    float pruning_opacity_threshold;
    float opacity_clamp_value;
    float max_world_scale;
    float duplicate_grad_threshold;
    float duplicate_scale_threshold;
    float duplicate_absgrad_threshold;
    float scene_scale;
    int64_t refine_every, start_refine, end_refine, max_num_gaussians, reset_every, global_step;
    uint64_t seed;
    uint64_t rng_draws_consumed; /* draws earlier steps took from the adc object's stream */
} oracle_adc_params;

static float host_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
static float host_logit(float p) { return logf(p / (1.0f - p)); }

static float prob_to_logit(float p)
{
    float c = p;

    if(c <= 1e-6f) c = 1e-6f;
    if(c >= 1.0f - 1e-6f) c = 1.0f - 1e-6f;
    return host_logit(c);
}

static float next_normal(gsx_amd_pcg32 *rng)
{
    float u1 = gsx_pcg32_next_f32(rng);
    float u2 = gsx_pcg32_next_f32(rng);
    float mag;

    u1 = fmaxf(1e-7f, u1);
    mag = sqrtf(-2.0f * logf(u1));
    return mag * cosf(2.0f * (float)3.14159265358979323846264338327950288 * u2);
}

static int64_t nonneg(int64_t v) { return v <= 0 ? 0 : v; }

static int in_refine_window(const oracle_adc_params *p)
{
    uint64_t s = (uint64_t)p->global_step;

    if(p->refine_every == 0) return 0;
    if(s % (uint64_t)p->refine_every != 0) return 0;
    if(s < (uint64_t)nonneg(p->start_refine) || s > (uint64_t)nonneg(p->end_refine)) return 0;
    return 1;
}

static int in_reset_window(const oracle_adc_params *p)
{
    uint64_t s = (uint64_t)p->global_step;

    if(p->reset_every == 0) return 0;
    if(s % (uint64_t)p->reset_every != 0) return 0;
    if(s < (uint64_t)nonneg(p->start_refine) || s >= (uint64_t)nonneg(p->end_refine)) return 0;
    return 1;
}

static const int k_adc_widths[5] = { 3, 4, 3, 1, 3 };

/* fields[5] = mean3d, rotation, logscale, opacity, sh0 (row widths 3, 4, 3, 1, 3); moments[10]
 * = m, v per field (nullable => optimizer disabled). aux[3] = grad_acc, absgrad_acc,
 * visible_counter (each nullable). Arrays must have room for max(n, max_num_gaussians) rows.
 * Returns the new count; counts[4] = pruned, duplicated, grown, reset. Returns -1 on error. */
int64_t oracle_adc_step(int64_t n, float **fields, float **moments, float **aux, const oracle_adc_params *p,
    int64_t *counts)
{
    int64_t i, f, grow = 0, split_count = 0, dup_count = 0, keep = 0, n_after;
    int32_t *sources = NULL;
    uint8_t *modes = NULL;
    int64_t budget = 0, cap = nonneg(p->max_num_gaussians);
    float *mean3d = fields[0], *rot = fields[1], *ls = fields[2], *op = fields[3];
    const float *acc = p->algorithm == 1 ? aux[1] : aux[0];
    float grow_thr = p->algorithm == 1 ? p->duplicate_absgrad_threshold : p->duplicate_grad_threshold;
    gsx_amd_pcg32 rng;
    int32_t *keep_idx = NULL;

    counts[0] = counts[1] = counts[2] = counts[3] = 0;
    gsx_pcg32_seed2(&rng, p->seed, p->seed);
    gsx_pcg32_advance(&rng, p->rng_draws_consumed);
    n_after = n;
    if(in_refine_window(p) && n > 0) {
        if(acc == NULL) return -1;
        if(cap > n) budget = cap - n;
        if(budget > 0) {
            sources = (int32_t *)malloc(sizeof(int32_t) * (size_t)budget);
            modes = (uint8_t *)malloc((size_t)budget);
            if(sources == NULL || modes == NULL) {
                free(sources);
                free(modes);
                return -1;
            }
            /* default.c:160-219, 373-386: first-come by index until the budget is spent. */
            for(i = 0; i < n && grow < budget; ++i) {
                float counter = aux[2] != NULL ? aux[2][i] : 1.0f;
                float g, sx, sy, sz, mx;

                if(counter <= 0.0f) continue;
                g = acc[i] / (counter > 1.0f ? counter : 1.0f);
                if(g <= grow_thr) continue;
                sx = expf(ls[i * 3 + 0]);
                sy = expf(ls[i * 3 + 1]);
                sz = expf(ls[i * 3 + 2]);
                mx = sx;
                if(sy > mx) mx = sy;
                if(sz > mx) mx = sz;
                sources[grow] = (int32_t)i;
                modes[grow] = mx > p->duplicate_scale_threshold * p->scene_scale ? 2 : 1;
                if(modes[grow] == 2) split_count += 1;
                else dup_count += 1;
                grow += 1;
            }
        }
        if(grow > 0) {
            /* default.c:396-403: gather [0..n) ++ sources, i.e. append copies; moments of
             * the appended rows are zero (adc.c:438-444). */
            for(f = 0; f < 5; ++f) {
                int wdt = k_adc_widths[f];

                for(i = 0; i < grow; ++i) {
                    memcpy(fields[f] + (n + i) * wdt, fields[f] + (int64_t)sources[i] * wdt, sizeof(float) * (size_t)wdt);
                    if(moments != NULL) {
                        memset(moments[2 * f] + (n + i) * wdt, 0, sizeof(float) * (size_t)wdt);
                        memset(moments[2 * f + 1] + (n + i) * wdt, 0, sizeof(float) * (size_t)wdt);
                    }
                }
            }
            for(f = 0; f < 3; ++f) {
                if(aux[f] != NULL) {
                    for(i = 0; i < grow; ++i) aux[f][n + i] = aux[f][sources[i]];
                }
            }
            /* default.c:38-158 mutations in grow order; splits draw 6 normals each from the
             * single sequential stream. */
            for(i = 0; i < grow; ++i) {
                int64_t src = sources[i], tgt = n + i;

                if(modes[i] == 1) {
                    continue; /* duplicate: the gathered copy is already the mutation */
                }
                {
                    float qx = rot[src * 4 + 0], qy = rot[src * 4 + 1], qz = rot[src * 4 + 2], qw = rot[src * 4 + 3];
                    float sx = expf(ls[src * 3 + 0]), sy = expf(ls[src * 3 + 1]), sz = expf(ls[src * 3 + 2]);
                    float so = host_sigmoid(op[src]);
                    float r1x, r1y, r1z, r2x, r2y, r2z, t1x, t1y, t1z, t2x, t2y, t2z, qn, nsx, nsy, nsz, sop;
                    float m00, m01, m02, m10, m11, m12, m20, m21, m22;

                    nsx = sx / 1.6f;
                    nsy = sy / 1.6f;
                    nsz = sz / 1.6f;
                    r1x = next_normal(&rng);
                    r1y = next_normal(&rng);
                    r1z = next_normal(&rng);
                    r2x = next_normal(&rng);
                    r2y = next_normal(&rng);
                    r2z = next_normal(&rng);
                    t1x = r1x * (sx + 1e-5f);
                    t1y = r1y * (sy + 1e-5f);
                    t1z = r1z * (sz + 1e-5f);
                    t2x = r2x * (sx + 1e-5f);
                    t2y = r2y * (sy + 1e-5f);
                    t2z = r2z * (sz + 1e-5f);
                    /* adc.c:290-309 */
                    qn = sqrtf(qx * qx + qy * qy + qz * qz + qw * qw);
                    if(qn > 1e-8f) {
                        float iq = 1.0f / qn;

                        qx *= iq;
                        qy *= iq;
                        qz *= iq;
                        qw *= iq;
                    }
                    m00 = 1.0f - 2.0f * (qy * qy + qz * qz);
                    m01 = 2.0f * (qx * qy - qw * qz);
                    m02 = 2.0f * (qx * qz + qw * qy);
                    m10 = 2.0f * (qx * qy + qw * qz);
                    m11 = 1.0f - 2.0f * (qx * qx + qz * qz);
                    m12 = 2.0f * (qy * qz - qw * qx);
                    m20 = 2.0f * (qx * qz - qw * qy);
                    m21 = 2.0f * (qy * qz + qw * qx);
                    m22 = 1.0f - 2.0f * (qx * qx + qy * qy);
                    if(so < 0.0f) so = 0.0f;
                    if(so > 1.0f - 1e-6f) so = 1.0f - 1e-6f;
                    sop = 1.0f - sqrtf(1.0f - so);
                    mean3d[tgt * 3 + 0] = mean3d[src * 3 + 0] + (m00 * t1x + m01 * t1y + m02 * t1z);
                    mean3d[tgt * 3 + 1] = mean3d[src * 3 + 1] + (m10 * t1x + m11 * t1y + m12 * t1z);
                    mean3d[tgt * 3 + 2] = mean3d[src * 3 + 2] + (m20 * t1x + m21 * t1y + m22 * t1z);
                    ls[tgt * 3 + 0] = logf(nsx);
                    ls[tgt * 3 + 1] = logf(nsy);
                    ls[tgt * 3 + 2] = logf(nsz);
                    op[tgt] = prob_to_logit(sop);
                    mean3d[src * 3 + 0] = mean3d[src * 3 + 0] + (m00 * t2x + m01 * t2y + m02 * t2z);
                    mean3d[src * 3 + 1] = mean3d[src * 3 + 1] + (m10 * t2x + m11 * t2y + m12 * t2z);
                    mean3d[src * 3 + 2] = mean3d[src * 3 + 2] + (m20 * t2x + m21 * t2y + m22 * t2z);
                    ls[src * 3 + 0] = logf(nsx);
                    ls[src * 3 + 1] = logf(nsy);
                    ls[src * 3 + 2] = logf(nsz);
                    op[src] = prob_to_logit(sop);
                }
            }
            counts[1] = dup_count;
            counts[2] = split_count;
            n_after = n + grow;
        }
        /* default.c:221-273 keep predicate, then compaction (default.c:488-522). */
        keep_idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_after > 0 ? n_after : 1));
        if(keep_idx == NULL) {
            free(sources);
            free(modes);
            return -1;
        }
        {
            int prune_large = (uint64_t)p->global_step > (uint64_t)nonneg(p->reset_every);

            for(i = 0; i < n_after; ++i) {
                float o = host_sigmoid(op[i]);
                float sx = expf(ls[i * 3 + 0]), sy = expf(ls[i * 3 + 1]), sz = expf(ls[i * 3 + 2]);
                float mx = sx, rn;
                int not_large_ws = 1;

                if(sy > mx) mx = sy;
                if(sz > mx) mx = sz;
                if(p->max_world_scale > 0.0f) {
                    not_large_ws = mx < (p->max_world_scale * p->scene_scale);
                }
                rn = fabsf(rot[i * 4 + 0]) + fabsf(rot[i * 4 + 1]) + fabsf(rot[i * 4 + 2]) + fabsf(rot[i * 4 + 3]);
                if((o > p->pruning_opacity_threshold) && (not_large_ws || !prune_large) && rn > FLT_EPSILON) {
                    keep_idx[keep++] = (int32_t)i;
                }
            }
        }
        if(keep == 0) {
            keep_idx[0] = 0;
            keep = 1;
        }
        if(keep < n_after) {
            for(f = 0; f < 5; ++f) {
                int wdt = k_adc_widths[f];

                for(i = 0; i < keep; ++i) {
                    memmove(fields[f] + i * wdt, fields[f] + (int64_t)keep_idx[i] * wdt, sizeof(float) * (size_t)wdt);
                    if(moments != NULL) {
                        memmove(moments[2 * f] + i * wdt, moments[2 * f] + (int64_t)keep_idx[i] * wdt,
                            sizeof(float) * (size_t)wdt);
                        memmove(moments[2 * f + 1] + i * wdt, moments[2 * f + 1] + (int64_t)keep_idx[i] * wdt,
                            sizeof(float) * (size_t)wdt);
                    }
                }
            }
            counts[0] = n_after - keep;
            n_after = keep;
        }
        /* adc.c:446-452: aux statistics are zeroed after a refine. */
        for(f = 0; f < 3; ++f) {
            if(aux[f] != NULL) memset(aux[f], 0, sizeof(float) * (size_t)n_after);
        }
        free(keep_idx);
        free(sources);
        free(modes);
    }
    if(in_reset_window(p)) {
        /* default.c:275-314: clamp opacity logits to logit(clamp value), reset the opacity
         * optimizer moments. */
        float c = p->opacity_clamp_value;
        float mx;

        if(c > 1.0f) c = 1.0f;
        if(c < 1e-6f) c = 1e-6f;
        mx = prob_to_logit(c);
        for(i = 0; i < n_after; ++i) {
            if(op[i] < -FLT_MAX) op[i] = -FLT_MAX;
            if(op[i] > mx) op[i] = mx;
        }
        if(moments != NULL) {
            memset(moments[6], 0, sizeof(float) * (size_t)n_after);
            memset(moments[7], 0, sizeof(float) * (size_t)n_after);
        }
        counts[3] = 1;
    }
    return n_after;
}

/* Number of float inputs in [lo_bits, hi_bits] where gsx_expf differs from libm expf. */
/* gsx_expf_blend (the blend kernels' expf, exponent folded into a 209-entry table) against the
 * host expf over [lo_bits, hi_bits]; its domain is [-4.5, 0]. */
uint64_t oracle_expf_blend_mismatches(uint32_t lo_bits, uint32_t hi_bits, uint32_t stride)
{
    uint64_t table[GSX_EXPF_BLEND_TABLE_SIZE];
    uint64_t bad = 0;
    uint64_t u;
    uint32_t j;

    for(j = 0; j < GSX_EXPF_BLEND_TABLE_SIZE; ++j) {
        table[j] = gsx_expf_blend_entry(j);
    }
    if(stride == 0) stride = 1;
    for(u = lo_bits; u <= hi_bits; u += stride) {
        float x = gsx_f32_from_bits((uint32_t)u);
        float a = expf(x);
        float b = gsx_expf_blend(x, table);

        if(gsx_f32_bits(a) != gsx_f32_bits(b)) {
            bad += 1;
        }
    }
    return bad;
}

uint64_t oracle_expf_mismatches(uint32_t lo_bits, uint32_t hi_bits, uint32_t stride)
{
    uint64_t bad = 0;
    uint64_t u;

    if(stride == 0) stride = 1;
    for(u = lo_bits; u <= hi_bits; u += stride) {
        float x = gsx_f32_from_bits((uint32_t)u);
        float a = expf(x);
        float b = gsx_expf(x);

        if(gsx_f32_bits(a) != gsx_f32_bits(b) && !(a != a && b != b)) {
            bad += 1;
        }
    }
    return bad;
}

/* Mismatches of the logf / sinf / cosf restatements (which: 0 logf, 1 sinf, 2 cosf) against the
 * host libm over float bit patterns lo..hi in steps of `stride` (both NaN counts as equal).
 * OpenMP over the range: an exhaustive sweep of all 2^32 patterns takes a few seconds. */
uint64_t oracle_libm_mismatches(int which, uint32_t lo_bits, uint32_t hi_bits, uint32_t stride)
{
    uint64_t bad = 0;
    int64_t count, j;

    if(stride == 0) stride = 1;
    if(hi_bits < lo_bits) return 0;
    count = ((int64_t)hi_bits - (int64_t)lo_bits) / (int64_t)stride + 1;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for(j = 0; j < count; ++j) {
        const float x = gsx_f32_from_bits((uint32_t)((int64_t)lo_bits + j * (int64_t)stride));
        const float a = which == 0 ? logf(x) : (which == 1 ? sinf(x) : cosf(x));
        const float b = which == 0 ? gsx_logf(x) : (which == 1 ? gsx_sinf(x) : gsx_cosf(x));

        if(gsx_f32_bits(a) != gsx_f32_bits(b) && !(a != a && b != b)) {
            bad += 1;
        }
    }
    return bad;
}

/* Mismatches of gsx_powf against the host powf: `count` pseudo-random (x, y) bit patterns from
 * a xorshift64 stream seeded with `seed` (every other y drawn from the quarter-integers in
 * [-8, 8), so integer exponents and negative bases meet), plus, when domain != 0, every 53rd
 * float in [0, 1] with y = 1/k and k + 1 for k = 1..51. */
uint64_t oracle_powf_mismatches(uint64_t seed, int64_t count, int domain)
{
    uint64_t bad = 0;
    int64_t i;

#pragma omp parallel for reduction(+ : bad) schedule(static)
    for(i = 0; i < count; ++i) {
        uint64_t s = seed + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1);
        float x, y, a, b;

        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        x = gsx_f32_from_bits((uint32_t)s);
        y = gsx_f32_from_bits((uint32_t)(s >> 32));
        if(i & 1) y = (float)((s >> 40) % 64u) * 0.25f - 8.0f;
        a = powf(x, y);
        b = gsx_powf(x, y);
        if(gsx_f32_bits(a) != gsx_f32_bits(b) && !(a != a && b != b)) {
            bad += 1;
        }
    }
    if(domain) {
        int k;

#pragma omp parallel for reduction(+ : bad) schedule(dynamic)
        for(k = 1; k <= 51; ++k) {
            const float ys[2] = { 1.0f / (float)k, (float)(k + 1) };
            int j;

            for(j = 0; j < 2; ++j) {
                uint32_t u;

                for(u = 0; u <= 0x3f800000u; u += 53) {
                    const float a = powf(gsx_f32_from_bits(u), ys[j]);
                    const float b = gsx_powf(gsx_f32_from_bits(u), ys[j]);

                    if(gsx_f32_bits(a) != gsx_f32_bits(b)) {
                        bad += 1;
                    }
                }
            }
        }
    }
    return bad;
}

/* ---------------------------------------------------------------------------------------
 * Tiled evaluation for full-size scenes (configs 3 and 4: 3M and 6M Gaussians at 1080p,
 * where the per-Gaussian raster above walks 4e9 and 2e11 box pixels). Same arithmetic as
 * oracle_render_forward and oracle_tile_keys, reorganised so that it runs on all host cores
 * and stops where the CPU's loop can no longer change a pixel:
 *   - visible records from collect_visible over chunks of Gaussians in parallel, compacted
 *     in Gaussian order (render.c:850-1016);
 *   - the (depth, index) order of render.c:830-848 through a sort of
 *     bits(depth) << 32 | position keys (depth > near > 0, so the float bits order like the
 *     values, and positions follow the Gaussian index);
 *   - per tile, the Gaussians whose box meets the tile, in that order (with `cull`, only the
 *     instances the tile test keeps, exactly oracle_tile_keys' per-tile lists);
 *   - per pixel, the CPU's update (render.c:1035-1079) over its tile's list. Transmittance
 *     never rises, so after T < 1e-4 the CPU's own test skips every later entry and the walk
 *     stops there.
 * Pixels equal oracle_render_forward's bit for bit and the cut lists equal oracle_tile_keys'
 * key for key; the CPU tests check both on scenes that the serial functions finish.
 * ------------------------------------------------------------------------------------- */
#include <omp.h>

static int cmp_u64(const void *pa, const void *pb)
{
    uint64_t a = *(const uint64_t *)pa, b = *(const uint64_t *)pb;

    return a < b ? -1 : (a > b ? 1 : 0);
}

typedef struct tiled_lists {
    int64_t count;          /* visible Gaussians */
    vis *v;                 /* visible records in (depth, index) order */
    int32_t tiles_x, tiles_y;
    int64_t *tile_start;    /* [tiles + 1] */
    uint32_t *entries;      /* positions into v, per tile in list order */
} tiled_lists;

static void tiled_free(tiled_lists *t)
{
    free(t->v);
    free(t->tile_start);
    free(t->entries);
    memset(t, 0, sizeof(*t));
}

static int tiled_build(int64_t n, int deg, const float *mean3d, const float *rot, const float *ls,
    const float *op, const float *sh0, const float *sh1, const float *sh2, const float *sh3, const cam *k,
    int32_t tile, int cull, tiled_lists *out)
{
    const int64_t chunk = 1 << 16;
    int64_t nchunks = (n + chunk - 1) / chunk;
    int64_t *ccount = (int64_t *)calloc((size_t)(nchunks > 0 ? nchunks : 1), sizeof(int64_t));
    vis *all = (vis *)malloc(sizeof(vis) * (size_t)(n > 0 ? n : 1));
    uint64_t *order = NULL;
    int64_t count = 0, c, i;
    const int32_t tiles_x = (k->width + tile - 1) / tile, tiles_y = (k->height + tile - 1) / tile;
    const int64_t tiles = (int64_t)tiles_x * tiles_y;
    const int nparts = 256;
    int64_t *part_counts = NULL, *box_byte = NULL;
    uint8_t *kept = NULL;
    int ok = 1;

    memset(out, 0, sizeof(*out));
    if(ccount == NULL || all == NULL) {
        free(ccount);
        free(all);
        return -1;
    }
#pragma omp parallel for schedule(dynamic, 1)
    for(c = 0; c < nchunks; ++c) {
        int64_t i0 = c * chunk, m = n - i0 < chunk ? n - i0 : chunk, j;

        ccount[c] = collect_visible(m, deg, mean3d + 3 * i0, rot + 4 * i0, ls + 3 * i0, op + i0, sh0 + 3 * i0,
            deg >= 1 ? sh1 + 9 * i0 : NULL, deg >= 2 ? sh2 + 15 * i0 : NULL, deg >= 3 ? sh3 + 21 * i0 : NULL, k,
            all + i0, NULL);
        for(j = 0; j < ccount[c]; ++j) {
            all[i0 + j].g += i0;
        }
    }
    for(c = 0; c < nchunks; ++c) {
        if(count != c * chunk && ccount[c] > 0) {
            memmove(all + count, all + c * chunk, sizeof(vis) * (size_t)ccount[c]);
        }
        count += ccount[c];
    }
    free(ccount);

    order = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(count > 0 ? count : 1));
    out->v = (vis *)malloc(sizeof(vis) * (size_t)(count > 0 ? count : 1));
    out->tile_start = (int64_t *)calloc((size_t)tiles + 1, sizeof(int64_t));
    part_counts = (int64_t *)calloc((size_t)nparts * (size_t)tiles, sizeof(int64_t));
    box_byte = (int64_t *)malloc(sizeof(int64_t) * (size_t)(count + 1));
    if(order == NULL || out->v == NULL || out->tile_start == NULL || part_counts == NULL || box_byte == NULL) {
        ok = 0;
        goto done;
    }
#pragma omp parallel for schedule(static)
    for(i = 0; i < count; ++i) {
        order[i] = ((uint64_t)gsx_f32_bits(all[i].rec[ORACLE_REC_DEPTH]) << 32) | (uint64_t)i;
    }
    qsort(order, (size_t)count, sizeof(uint64_t), cmp_u64);
#pragma omp parallel for schedule(static)
    for(i = 0; i < count; ++i) {
        out->v[i] = all[order[i] & 0xFFFFFFFFu];
    }
    free(all);
    all = NULL;
    out->count = count;
    out->tiles_x = tiles_x;
    out->tiles_y = tiles_y;

    /* kept flag of every (Gaussian, box tile), one byte each, byte ranges per Gaussian */
    box_byte[0] = 0;
    for(i = 0; i < count; ++i) {
        const int32_t *bb = out->v[i].bb;
        int64_t bt = (int64_t)(bb[1] / tile - bb[0] / tile + 1) * (int64_t)(bb[3] / tile - bb[2] / tile + 1);

        box_byte[i + 1] = box_byte[i] + (cull ? bt : 0);
    }
    if(cull) {
        kept = (uint8_t *)malloc((size_t)(box_byte[count] > 0 ? box_byte[count] : 1));
        if(kept == NULL) {
            ok = 0;
            goto done;
        }
    }
    /* per part (a contiguous range of the depth order) and tile: entry counts */
#pragma omp parallel for schedule(dynamic, 1)
    for(c = 0; c < nparts; ++c) {
        int64_t lo = count * c / nparts, hi = count * (c + 1) / nparts, g;
        int64_t *pc = part_counts + (size_t)c * (size_t)tiles;

        for(g = lo; g < hi; ++g) {
            const int32_t *bb = out->v[g].bb;
            int64_t b = box_byte[g];
            int32_t tx, ty, txa = bb[0] / tile, txb = bb[1] / tile;
            const gsx_tile_span sp = vis_span(&out->v[g]);

            for(ty = bb[2] / tile; ty <= bb[3] / tile; ++ty) {
                if(cull) row_tiles(&out->v[g], &sp, ty, tile, &txa, &txb);
                for(tx = bb[0] / tile; tx <= bb[1] / tile; ++tx) {
                    int keep = 1;

                    if(cull) {
                        keep = txa <= tx && tx <= txb;
                        kept[b++] = (uint8_t)keep;
                    }
                    pc[(int64_t)ty * tiles_x + tx] += keep;
                }
            }
        }
    }
    /* exclusive prefix over (tile, part): each part's cursor within each tile */
    {
        int64_t total = 0, t;

        for(t = 0; t < tiles; ++t) {
            out->tile_start[t] = total;
            for(c = 0; c < nparts; ++c) {
                int64_t v = part_counts[(size_t)c * (size_t)tiles + (size_t)t];

                part_counts[(size_t)c * (size_t)tiles + (size_t)t] = total;
                total += v;
            }
        }
        out->tile_start[tiles] = total;
        out->entries = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(total > 0 ? total : 1));
        if(out->entries == NULL) {
            ok = 0;
            goto done;
        }
    }
#pragma omp parallel for schedule(dynamic, 1)
    for(c = 0; c < nparts; ++c) {
        int64_t lo = count * c / nparts, hi = count * (c + 1) / nparts, g;
        int64_t *pc = part_counts + (size_t)c * (size_t)tiles;

        for(g = lo; g < hi; ++g) {
            const int32_t *bb = out->v[g].bb;
            int64_t b = box_byte[g];
            int32_t tx, ty;

            for(ty = bb[2] / tile; ty <= bb[3] / tile; ++ty) {
                for(tx = bb[0] / tile; tx <= bb[1] / tile; ++tx) {
                    if(cull && !kept[b++]) continue;
                    out->entries[pc[(int64_t)ty * tiles_x + tx]++] = (uint32_t)g;
                }
            }
        }
    }
done:
    free(all);
    free(order);
    free(part_counts);
    free(box_byte);
    free(kept);
    if(!ok) {
        tiled_free(out);
        return -1;
    }
    return 0;
}

/* Renders with the tiled lists (see above) and/or returns the cut lists as sorted keys:
 * key = tile << 32 | bits(depth), value = Gaussian index, as oracle_tile_keys. out_keys /
 * out_values receive malloc'ed arrays (release with oracle_free). Returns the number of list
 * entries, or -1. */
int64_t oracle_tiled(int64_t n, int sh_degree, const float *mean3d, const float *rotation,
    const float *logscale, const float *opacity, const float *sh0, const float *sh1, const float *sh2,
    const float *sh3, const float *camera, int32_t tile, int cull, float *out_rgb, float *out_t,
    uint64_t **out_keys, uint32_t **out_values)
{
    cam k = cam_from(camera);
    tiled_lists tl;
    const size_t pixels = (size_t)k.width * (size_t)k.height;
    int64_t tiles, total, t;

    if(tiled_build(n, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, &k, tile, cull, &tl) != 0) {
        return -1;
    }
    tiles = (int64_t)tl.tiles_x * tl.tiles_y;
    total = tl.tile_start[tiles];
    if(out_rgb != NULL) {
#pragma omp parallel for schedule(dynamic, 4)
        for(t = 0; t < tiles; ++t) {
            const int32_t tx = (int32_t)(t % tl.tiles_x), ty = (int32_t)(t / tl.tiles_x);
            const int64_t e0 = tl.tile_start[t], e1 = tl.tile_start[t + 1];
            int32_t px, py;

            for(py = ty * tile; py < ty * tile + tile && py < k.height; ++py) {
                for(px = tx * tile; px < tx * tile + tile && px < k.width; ++px) {
                    size_t pix = (size_t)py * (size_t)k.width + (size_t)px;
                    float cr = 0.0f, cg = 0.0f, cb = 0.0f, tt = 1.0f;
                    int64_t e;

                    for(e = e0; e < e1; ++e) {
                        const vis *g = &tl.v[tl.entries[e]];
                        const float *r = g->rec;
                        float inv_a, inv_b, inv_c, dx, dy, power, alpha, wgt;

                        if(tt < T_THRESHOLD) break;
                        if(px < g->bb[0] || px > g->bb[1] || py < g->bb[2] || py > g->bb[3]) continue;
                        inv_a = r[ORACLE_REC_COV_C] * r[ORACLE_REC_INV_DET];
                        inv_b = -r[ORACLE_REC_COV_B] * r[ORACLE_REC_INV_DET];
                        inv_c = r[ORACLE_REC_COV_A] * r[ORACLE_REC_INV_DET];
                        dx = ((float)px + 0.5f) - r[ORACLE_REC_MEAN2D_X];
                        dy = ((float)py + 0.5f) - r[ORACLE_REC_MEAN2D_Y];
                        power = -0.5f * (inv_a * dx * dx + 2.0f * inv_b * dx * dy + inv_c * dy * dy);
                        if(power > 0.0f) power = 0.0f;
                        if(power < POWER_THRESHOLD) continue;
                        alpha = fminf(MAX_FRAGMENT_ALPHA, r[ORACLE_REC_OPACITY] * expf(power));
                        if(alpha < MIN_ALPHA) continue;
                        wgt = alpha * tt;
                        cr += wgt * r[ORACLE_REC_COLOR_R];
                        cg += wgt * r[ORACLE_REC_COLOR_G];
                        cb += wgt * r[ORACLE_REC_COLOR_B];
                        tt = tt * (1.0f - alpha);
                    }
                    out_rgb[0 * pixels + pix] = cr + tt * k.bg[0];
                    out_rgb[1 * pixels + pix] = cg + tt * k.bg[1];
                    out_rgb[2 * pixels + pix] = cb + tt * k.bg[2];
                    if(out_t != NULL) out_t[pix] = tt;
                }
            }
        }
    }
    if(out_keys != NULL && out_values != NULL) {
        *out_keys = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)(total > 0 ? total : 1));
        *out_values = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(total > 0 ? total : 1));
        if(*out_keys == NULL || *out_values == NULL) {
            free(*out_keys);
            free(*out_values);
            *out_keys = NULL;
            *out_values = NULL;
            tiled_free(&tl);
            return -1;
        }
#pragma omp parallel for schedule(dynamic, 16)
        for(t = 0; t < tiles; ++t) {
            int64_t e;

            for(e = tl.tile_start[t]; e < tl.tile_start[t + 1]; ++e) {
                const vis *g = &tl.v[tl.entries[e]];

                (*out_keys)[e] = ((uint64_t)t << 32) | (uint64_t)gsx_f32_bits(g->rec[ORACLE_REC_DEPTH]);
                (*out_values)[e] = (uint32_t)g->g;
            }
        }
    }
    tiled_free(&tl);
    return total;
}

void oracle_free(void *p) { free(p); }

/* ---------------------------------------------------------------------------------------
 * Tiled backward for full-size scenes (config 4: 6M Gaussians at 1080p, whose serial
 * backward would record every box pixel of 2e11). Same per-contribution arithmetic as
 * oracle_render_backward (render.c:1472-1969), reorganised per tile on all host cores:
 *   - the tile lists of tiled_build (with the tile test: it drops only instances that no
 *     pixel of the tile takes, so every pixel sees the same contributions as the CPU);
 *   - per pixel, the CPU's re-raster (render.c:1476-1515) over its tile's list, recording
 *     (entry, alpha, T_before) up to T < 1e-4 (the CPU's own test skips everything after);
 *   - per pixel, back to front, each contribution's terms (contrib_terms, render.c:1608-1656)
 *     with the pixel's suffix, which starts at T_final * bg and gains w * colour after each
 *     contribution (render.c:1658-1665), as the CPU's Gaussian-major loop updates it;
 *   - per Gaussian, its terms summed in double in a fixed order (tiles ascending, pixels in
 *     row-major order within a tile), then rounded to float. The CPU sums the same terms in
 *     float in box-raster order; the two sums differ only by the CPU's float rounding;
 *   - the parameter gradients of every visible Gaussian through project_grad_tail.
 * Per-pixel values (alpha, T_before, suffix, every term) equal the serial backward's bit for
 * bit; the CPU tests compare the gradients with oracle_render_backward on scenes it finishes.
 * ------------------------------------------------------------------------------------- */
typedef struct tile_sums {
    int64_t count;
    uint32_t *entry;   /* position in the depth-ordered visible records */
    double *sum;       /* [count][9] */
} tile_sums;

typedef struct tiled_pixel_contrib {
    uint32_t e;        /* entry within the tile's list */
    float alpha, tb;
} tiled_pixel_contrib;

int oracle_tiled_backward(int64_t n, int sh_degree, const float *mean3d, const float *rotation,
    const float *logscale, const float *opacity, const float *sh0, const float *sh1, const float *sh2,
    const float *sh3, const float *camera, int32_t tile, const float *grad_rgb, float *g_mean3d, float *g_rotation,
    float *g_logscale, float *g_opacity, float *g_sh0, float *g_sh1, float *g_sh2, float *g_sh3)
{
    cam k = cam_from(camera);
    m3 w = rotation_from_xyzw(k.qx, k.qy, k.qz, k.qw);
    v3 cc = camera_centre(&k, w);
    const size_t pixels = (size_t)k.width * (size_t)k.height;
    const grad_sinks gs = { g_mean3d, g_rotation, g_logscale, g_opacity, g_sh0, g_sh1, g_sh2, g_sh3 };
    tiled_lists tl;
    tile_sums *ts = NULL;
    double *gsum = NULL;
    int64_t tiles, t, i;
    int ok = 1;

    if(tiled_build(n, sh_degree, mean3d, rotation, logscale, opacity, sh0, sh1, sh2, sh3, &k, tile, 1, &tl) != 0) {
        return -1;
    }
    tiles = (int64_t)tl.tiles_x * tl.tiles_y;
    ts = (tile_sums *)calloc((size_t)(tiles > 0 ? tiles : 1), sizeof(tile_sums));
    gsum = (double *)calloc((size_t)(tl.count > 0 ? tl.count : 1) * 9u, sizeof(double));
    if(ts == NULL || gsum == NULL) {
        ok = 0;
        goto done;
    }

#pragma omp parallel reduction(&& : ok)
    {
        double *acc = NULL;            /* [list length][9] per entry of the current tile */
        uint8_t *hit = NULL;
        tiled_pixel_contrib *pc = NULL;
        int64_t cap = 0;

#pragma omp for schedule(dynamic, 2)
        for(t = 0; t < tiles; ++t) {
            const int32_t tx = (int32_t)(t % tl.tiles_x), ty = (int32_t)(t / tl.tiles_x);
            const int64_t e0 = tl.tile_start[t], len = tl.tile_start[t + 1] - e0;
            int64_t zeroed = 0, j, m;
            int32_t px, py;

            if(!ok || len == 0) continue;
            if(len > cap) {
                free(acc);
                free(hit);
                free(pc);
                cap = len;
                acc = (double *)malloc(sizeof(double) * 9u * (size_t)cap);
                hit = (uint8_t *)malloc((size_t)cap);
                pc = (tiled_pixel_contrib *)malloc(sizeof(tiled_pixel_contrib) * (size_t)cap);
                if(acc == NULL || hit == NULL || pc == NULL) {
                    ok = 0;
                    cap = 0;
                    continue;
                }
            }
            for(py = ty * tile; py < ty * tile + tile && py < k.height; ++py) {
                for(px = tx * tile; px < tx * tile + tile && px < k.width; ++px) {
                    const size_t pix = (size_t)py * (size_t)k.width + (size_t)px;
                    const float dox = grad_rgb[0 * pixels + pix], doy = grad_rgb[1 * pixels + pix];
                    const float doz = grad_rgb[2 * pixels + pix];
                    float tt = 1.0f;
                    int64_t nc = 0, q;
                    v3 s;

                    /* render.c:1476-1515 over the tile's list */
                    for(j = 0; j < len; ++j) {
                        const vis *g = &tl.v[tl.entries[e0 + j]];
                        const float *r = g->rec;
                        float inv_a, inv_b, inv_c, dx, dy, power, alpha;

                        if(tt < T_THRESHOLD) break;
                        if(px < g->bb[0] || px > g->bb[1] || py < g->bb[2] || py > g->bb[3]) continue;
                        inv_a = r[ORACLE_REC_COV_C] * r[ORACLE_REC_INV_DET];
                        inv_b = -r[ORACLE_REC_COV_B] * r[ORACLE_REC_INV_DET];
                        inv_c = r[ORACLE_REC_COV_A] * r[ORACLE_REC_INV_DET];
                        dx = ((float)px + 0.5f) - r[ORACLE_REC_MEAN2D_X];
                        dy = ((float)py + 0.5f) - r[ORACLE_REC_MEAN2D_Y];
                        power = -0.5f * (inv_a * dx * dx + 2.0f * inv_b * dx * dy + inv_c * dy * dy);
                        if(power > 0.0f) power = 0.0f;
                        if(power < POWER_THRESHOLD) continue;
                        alpha = fminf(MAX_FRAGMENT_ALPHA, r[ORACLE_REC_OPACITY] * expf(power));
                        if(alpha < MIN_ALPHA) continue;
                        pc[nc].e = (uint32_t)j;
                        pc[nc].alpha = alpha;
                        pc[nc].tb = tt;
                        nc += 1;
                        tt = tt * (1.0f - alpha);
                    }
                    if(nc == 0) continue;
                    for(; zeroed <= (int64_t)pc[nc - 1].e; ++zeroed) {
                        memset(acc + 9 * zeroed, 0, sizeof(double) * 9u);
                        hit[zeroed] = 0;
                    }
                    /* render.c:1547-1550 suffix start, then back to front */
                    s = mk3(tt * k.bg[0], tt * k.bg[1], tt * k.bg[2]);
                    for(q = nc; q > 0; --q) {
                        const tiled_pixel_contrib *c = &pc[q - 1];
                        const float *r = tl.v[tl.entries[e0 + c->e]].rec;
                        const conic_terms ct = conic_of(r);
                        double *a = acc + 9 * (int64_t)c->e;
                        float t9[9], wgt;
                        int op_ok = contrib_terms(r, &ct, px, py, dox, doy, doz, c->alpha, c->tb, s, t9);

                        for(m = 0; m < 8; ++m) {
                            a[m] += (double)t9[m];
                        }
                        if(op_ok) a[8] += (double)t9[8];
                        hit[c->e] = 1;
                        wgt = c->alpha * c->tb;
                        s.x += wgt * r[ORACLE_REC_COLOR_R];
                        s.y += wgt * r[ORACLE_REC_COLOR_G];
                        s.z += wgt * r[ORACLE_REC_COLOR_B];
                    }
                }
            }
            /* the tile's reached entries, in list order */
            {
                int64_t nh = 0, o = 0;

                for(j = 0; j < zeroed; ++j) nh += hit[j];
                ts[t].count = nh;
                if(nh == 0) continue;
                ts[t].entry = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)nh);
                ts[t].sum = (double *)malloc(sizeof(double) * 9u * (size_t)nh);
                if(ts[t].entry == NULL || ts[t].sum == NULL) {
                    ok = 0;
                    continue;
                }
                for(j = 0; j < zeroed; ++j) {
                    if(!hit[j]) continue;
                    ts[t].entry[o] = tl.entries[e0 + j];
                    memcpy(ts[t].sum + 9 * o, acc + 9 * j, sizeof(double) * 9u);
                    o += 1;
                }
            }
        }
        free(acc);
        free(hit);
        free(pc);
    }
    if(!ok) goto done;

    /* per Gaussian, tiles ascending */
    for(t = 0; t < tiles; ++t) {
        int64_t j, m;

        for(j = 0; j < ts[t].count; ++j) {
            double *d = gsum + 9 * (int64_t)ts[t].entry[j];

            for(m = 0; m < 9; ++m) {
                d[m] += ts[t].sum[9 * j + m];
            }
        }
    }

    memset(g_mean3d, 0, sizeof(float) * 3u * (size_t)n);
    memset(g_rotation, 0, sizeof(float) * 4u * (size_t)n);
    memset(g_logscale, 0, sizeof(float) * 3u * (size_t)n);
    memset(g_sh0, 0, sizeof(float) * 3u * (size_t)n);
    memset(g_opacity, 0, sizeof(float) * (size_t)n);
    if(sh_degree >= 1 && g_sh1 != NULL) memset(g_sh1, 0, sizeof(float) * 9u * (size_t)n);
    if(sh_degree >= 2 && g_sh2 != NULL) memset(g_sh2, 0, sizeof(float) * 15u * (size_t)n);
    if(sh_degree >= 3 && g_sh3 != NULL) memset(g_sh3, 0, sizeof(float) * 21u * (size_t)n);
#pragma omp parallel for schedule(static)
    for(i = 0; i < tl.count; ++i) {
        const double *d = gsum + 9 * i;
        screen_grad sg;

        sg.dc[0] = (float)d[0];
        sg.dc[1] = (float)d[1];
        sg.dc[2] = (float)d[2];
        sg.dm[0] = (float)d[3];
        sg.dm[1] = (float)d[4];
        sg.dcov[0] = (float)d[5];
        sg.dcov[1] = (float)d[6];
        sg.dcov[2] = (float)d[7];
        sg.dop = (float)d[8];
        project_grad_tail(&tl.v[i], &sg, sh_degree, &k, w, cc, mean3d, rotation, logscale, sh1, sh2, sh3, &gs);
    }
done:
    if(ts != NULL) {
        for(t = 0; t < tiles; ++t) {
            free(ts[t].entry);
            free(ts[t].sum);
        }
    }
    free(ts);
    free(gsum);
    tiled_free(&tl);
    return ok ? 0 : -1;
}
