/*
 * gsx_oracle.h - CPU restatement of the gsx CPU backend's hot-path algorithms.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load this library, and only as the checker. The product (gsx_amd/libgsx_hip.so)
 * never links, loads or calls it.
 *
 * Camera blocks are float[18]: fx, fy, cx, cy, width, height, qx, qy, qz, qw (world-to-camera
 * rotation, xyzw), tx, ty, tz, near, far, bg_r, bg_g, bg_b.
 * Visible records are float[ORACLE_REC_FLOATS] per Gaussian (see the enum below).
 *
 * Pinning (how each function is checked against something other than itself):
 *   oracle_render_forward / oracle_render_backward: bit-exact against the reference CPU
 *     backend built from its own sources (oracle/_ref), on seeded scenes and on the
 *     reference's finite-difference scenes; closed form (tests/render_runtime.cpp:671-722).
 *   oracle_tile_*: brute force (per-pixel membership of every tile list) and invariants; the
 *     tile test (oracle_tile_may_contribute) against per-pixel evaluation of the CPU's power and
 *     alpha cuts on random and adversarial Gaussians (it may keep, never drop, a contributing
 *     tile), and end to end by rendering from the culled lists bit-exactly like oracle/_ref.
 *   oracle_loss_*: against oracle/_ref bit-exact; SSIM also against an independent numpy
 *     float64 evaluation and the identical-image property.
 *   oracle_adam_step: against oracle/_ref bit-exact and the textbook Adam formula.
 *   oracle_adc_*: against oracle/_ref on seeded ADC scenarios (counts and all fields).
 *   gsx_expf (gsx_amd/csrc/gsx_math.h): against host glibc expf over all float inputs.
 */
#ifndef GSX_ORACLE_H
#define GSX_ORACLE_H

#include <stdint.h>

enum {
    ORACLE_REC_MEAN2D_X = 0,
    ORACLE_REC_MEAN2D_Y,
    ORACLE_REC_COV_A,
    ORACLE_REC_COV_B,
    ORACLE_REC_COV_C,
    ORACLE_REC_INV_DET,
    ORACLE_REC_DEPTH,
    ORACLE_REC_X_CAM,
    ORACLE_REC_Y_CAM,
    ORACLE_REC_Z_CAM,
    ORACLE_REC_COLOR_R,
    ORACLE_REC_COLOR_G,
    ORACLE_REC_COLOR_B,
    ORACLE_REC_OPACITY,
    ORACLE_REC_RAW_OPACITY,
    ORACLE_REC_DIR_X,
    ORACLE_REC_DIR_Y,
    ORACLE_REC_DIR_Z,
    ORACLE_REC_FLOATS
};

#endif /* GSX_ORACLE_H */
