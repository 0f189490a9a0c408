"""ctypes binding of libgsx_hip.so (declared in include/gsx_hip.h).

Loading fails loudly: there is no CPU fallback anywhere in this package. A missing library,
a missing symbol or a machine without a HIP device raises ``GsxHipError``.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgsx_hip.so")

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f = ctypes.c_float
_d = ctypes.c_double
_st = ctypes.c_int


class GsxHipError(RuntimeError):
    pass


# status codes (include/gsx_hip.h)
ERROR_INVALID_ARGUMENT = -1
ERROR_INVALID_STATE = -2
ERROR_OUT_OF_RANGE = -3
ERROR_OUT_OF_MEMORY = -4
ERROR_NOT_SUPPORTED = -5

# forward types of gsx_hip_render_forward (include/gsx_hip.h)
FORWARD_INFERENCE = 0
FORWARD_TRAIN_BORROW = 1
FORWARD_TRAIN_CLONE = 2


class Camera(ctypes.Structure):
    _fields_ = [("fx", _f), ("fy", _f), ("cx", _f), ("cy", _f), ("width", _i32), ("height", _i32),
                ("rot", _f * 4), ("transl", _f * 3), ("near_plane", _f), ("far_plane", _f), ("background", _f * 3)]

    @classmethod
    def from_block(cls, block) -> "Camera":
        """From the float[18] camera block used by gsx_amd.scenes."""
        b = [float(x) for x in block]
        c = cls()
        c.fx, c.fy, c.cx, c.cy = b[0], b[1], b[2], b[3]
        c.width, c.height = int(b[4]), int(b[5])
        c.rot[:] = b[6:10]
        c.transl[:] = b[10:13]
        c.near_plane, c.far_plane = b[13], b[14]
        c.background[:] = b[15:18]
        return c


class Gaussians(ctypes.Structure):
    _fields_ = [("count", _i64), ("sh_degree", _i32), ("mean3d", _vp), ("rotation", _vp), ("logscale", _vp),
                ("opacity", _vp), ("sh0", _vp), ("sh1", _vp), ("sh2", _vp), ("sh3", _vp)]


class GaussianGrads(ctypes.Structure):
    _fields_ = [("mean3d", _vp), ("rotation", _vp), ("logscale", _vp), ("opacity", _vp), ("sh0", _vp),
                ("sh1", _vp), ("sh2", _vp), ("sh3", _vp)]


class RenderStats(ctypes.Structure):
    _fields_ = [("gaussian_count", _i64), ("visible_count", _i64), ("instance_count", _i64), ("tile_count", _i32),
                ("sort_passes", _i32), ("depth_sort_passes", _i32), ("tile_bits", _i32),
                ("sorted_tile_bytes", _i32)]


class RenderBuffers(ctypes.Structure):
    _fields_ = [("sorted_tiles", _vp), ("sorted_values", _vp), ("tile_ranges", _vp), ("records", _vp),
                ("tile_counts", _vp), ("instance_gaussian", _vp), ("final_transmittance", _vp),
                ("last_contributor", _vp)]


ADAM_MAX_GROUPS = 16


class AdamGroup(ctypes.Structure):
    _fields_ = [("parameter", _vp), ("gradient", _vp), ("first_moment", _vp), ("second_moment", _vp), ("count", _i64),
                ("beta1", _f), ("beta2", _f), ("learning_rate", _f), ("weight_decay", _f), ("epsilon", _f),
                ("max_grad", _f), ("bias_correction1", _d), ("bias_correction2", _d)]


class AdcParams(ctypes.Structure):
    _fields_ = [("algorithm", _i32), ("pruning_opacity_threshold", _f), ("opacity_clamp_value", _f),
                ("max_world_scale", _f), ("max_screen_scale", _f), ("duplicate_grad_threshold", _f),
                ("duplicate_scale_threshold", _f), ("duplicate_absgrad_threshold", _f), ("scene_scale", _f),
                ("refine_every", _i64), ("start_refine", _i64), ("end_refine", _i64), ("max_num_gaussians", _i64),
                ("reset_every", _i64), ("noise_strength", _f), ("grow_ratio", _f), ("mean3d_learning_rate", _f)]


class GsRows(ctypes.Structure):
    _fields_ = [("count", _i64), ("sh_degree", _i32), ("mean3d", _vp), ("rotation", _vp), ("logscale", _vp),
                ("opacity", _vp), ("sh0", _vp), ("sh1", _vp), ("sh2", _vp), ("sh3", _vp), ("grad_acc", _vp),
                ("absgrad_acc", _vp), ("visible_counter", _vp), ("max_screen_radius", _vp),
                ("first_moment", _vp * 8), ("second_moment", _vp * 8)]


class PoolStats(ctypes.Structure):
    _fields_ = [("requests", ctypes.c_uint64), ("reuses", ctypes.c_uint64), ("device_allocations", ctypes.c_uint64),
                ("device_releases", ctypes.c_uint64), ("bytes_in_use", ctypes.c_uint64),
                ("bytes_cached", ctypes.c_uint64)]


# name -> (restype, argtypes); this table is also the symbol list tests check against the header.
SIGNATURES = {
    "gsx_hip_last_error_message": (ctypes.c_char_p, []),
    "gsx_hip_device_count": (_st, [ctypes.POINTER(_i32)]),
    "gsx_hip_device_name": (_st, [_i32, ctypes.c_char_p, ctypes.c_size_t]),
    "gsx_hip_malloc": (_st, [ctypes.POINTER(_vp), ctypes.c_size_t]),
    "gsx_hip_free": (_st, [_vp]),
    "gsx_hip_pool_malloc": (_st, [ctypes.POINTER(_vp), ctypes.c_size_t, _vp]),
    "gsx_hip_pool_free": (_st, [_vp, _vp]),
    "gsx_hip_pool_trim": (_st, []),
    "gsx_hip_pool_get_stats": (_st, [ctypes.POINTER(PoolStats)]),
    "gsx_hip_memcpy_htod": (_st, [_vp, _vp, ctypes.c_size_t]),
    "gsx_hip_memcpy_dtoh": (_st, [_vp, _vp, ctypes.c_size_t]),
    "gsx_hip_memcpy_dtod_async": (_st, [_vp, _vp, ctypes.c_size_t, _vp]),
    "gsx_hip_stream_create": (_st, [ctypes.POINTER(_vp)]),
    "gsx_hip_stream_destroy": (_st, [_vp]),
    "gsx_hip_stream_synchronize": (_st, [_vp]),
    "gsx_hip_event_create": (_st, [_vp]),
    "gsx_hip_event_destroy": (_st, [_vp]),
    "gsx_hip_event_record": (_st, [_vp, _vp]),
    "gsx_hip_event_synchronize": (_st, [_vp]),
    "gsx_hip_stream_wait_event": (_st, [_vp, _vp]),
    "gsx_hip_fill_f32": (_st, [_vp, _i64, _f, _vp]),
    "gsx_hip_copy_f32": (_st, [_vp, _vp, _i64, _vp]),
    "gsx_hip_render_context_create": (_st, [ctypes.POINTER(_vp)]),
    "gsx_hip_render_context_destroy": (_st, [_vp]),
    "gsx_hip_render_forward": (_st, [_vp, ctypes.POINTER(Camera), ctypes.POINTER(Gaussians), _i32, _vp, _vp, _vp]),
    "gsx_hip_render_backward": (_st, [_vp, _vp, ctypes.POINTER(GaussianGrads), _vp]),
    "gsx_hip_render_context_get_stats": (_st, [_vp, ctypes.POINTER(RenderStats)]),
    "gsx_hip_render_context_get_buffers": (_st, [_vp, ctypes.POINTER(RenderBuffers)]),
    "gsx_hip_render_context_set_timing": (_st, [_vp, _i32]),
    "gsx_hip_render_context_get_timings": (_st, [_vp, ctypes.POINTER(_f), _i32, ctypes.POINTER(_i32)]),
    "gsx_hip_memcpy_async": (_st, [_vp, _vp, ctypes.c_size_t, _vp]),
    "gsx_hip_set_device": (_st, [_i32]),
    "gsx_hip_device_total_memory": (_st, [_i32, ctypes.POINTER(ctypes.c_size_t)]),
    "gsx_hip_host_alloc": (_st, [ctypes.POINTER(_vp), ctypes.c_size_t]),
    "gsx_hip_host_free": (_st, [_vp]),
    "gsx_hip_host_device_pointer": (_st, [_vp, ctypes.POINTER(_vp)]),
    "gsx_hip_fill_pattern": (_st, [_vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "gsx_hip_fill_rand_f32": (_st, [_vp, _i64, ctypes.c_uint64, ctypes.c_uint64, _vp]),
    "gsx_hip_fill_randn_f32": (_st, [_vp, _i64, ctypes.c_uint64, ctypes.c_uint64, _f, _vp]),
    "gsx_hip_fill_randint_temp_bytes": (ctypes.c_size_t, [_i64]),
    "gsx_hip_fill_randint": (_st, [_vp, _i64, _i32, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32, _i64, _vp,
                                   ctypes.POINTER(_i64), _vp]),
    "gsx_hip_multinomial_i32": (_st, [_vp, _i64, _vp, _i64, ctypes.c_uint64, ctypes.c_uint64, _vp]),
    "gsx_hip_check_finite_f32": (_st, [_vp, _i64, _vp, _vp]),
    "gsx_hip_unary_f32": (_st, [_vp, _vp, _i64, _i32, _vp]),
    "gsx_hip_clamp_inplace": (_st, [_vp, _i64, _i32, _vp, _vp, _vp]),
    "gsx_hip_reduce_temp_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "gsx_hip_reduce_f32": (_st, [_vp, _vp, _i64, _i64, _i32, _vp, _vp, _vp]),
    "gsx_hip_dataloader_to_chw_f32": (_st, [_vp, _i32, _i64, _i64, _i64, _vp, _vp]),
    "gsx_hip_image_colorspace_f32": (_st, [_vp, _vp, _i64, _i32, _i32, _vp]),
    "gsx_hip_image_storage_convert": (_st, [_vp, _i32, _vp, _i32, _i64, _i64, _i64, _i32, _vp]),
    "gsx_hip_image_quantize_u8": (_st, [_vp, _vp, _i64, _vp]),
    "gsx_hip_image_dequantize_u8": (_st, [_vp, _vp, _i64, _vp]),
    "gsx_hip_scan_temp_bytes": (ctypes.c_size_t, [_i64]),
    "gsx_hip_scan_exclusive_u32": (_st, [_vp, _vp, _i64, _vp, _vp]),
    "gsx_hip_scan_exclusive_u32_noalloc": (_st, [_vp, _vp, _i64, _vp]),
    "gsx_hip_radix_sort_temp_bytes": (ctypes.c_size_t, [_i64]),
    "gsx_hip_radix_sort_pairs_u64": (_st, [_vp, _vp, _vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _vp,
                                           ctypes.POINTER(ctypes.c_int), _vp]),
    "gsx_hip_radix_sort_keys_u64": (_st, [_vp, _vp, _i64, ctypes.c_int, ctypes.c_int, _vp,
                                          ctypes.POINTER(ctypes.c_int), _vp]),
    "gsx_hip_loss_l1_f32_forward_kernel_launch": (_st, [_vp, _vp, _vp, _i64, _f, _vp]),
    "gsx_hip_loss_l1_f32_backward_kernel_launch": (_st, [_vp, _vp, _vp, _i64, _f, _vp]),
    "gsx_hip_loss_mse_f32_forward_kernel_launch": (_st, [_vp, _vp, _vp, _i64, _f, _vp]),
    "gsx_hip_loss_mse_f32_backward_kernel_launch": (_st, [_vp, _vp, _vp, _i64, _f, _vp]),
    "gsx_hip_loss_ssim_chw_f32_forward_kernel_launch": (_st, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _f, _vp, _f,
                                                              ctypes.c_int, _vp]),
    "gsx_hip_loss_ssim_chw_f32_backward_kernel_launch": (_st, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _f, _vp, _f,
                                                               ctypes.c_int, _vp]),
    "gsx_hip_adam_step_f32_kernel_launch": (_st, [_vp, _vp, _vp, _vp, _i64, _f, _f, _f, _f, _f, _f, _d, _d, _vp]),
    "gsx_hip_adam_step_multi_launch": (_st, [ctypes.POINTER(AdamGroup), _i32, _vp]),
    "gsx_hip_adc_context_create": (_st, [ctypes.POINTER(_vp), ctypes.c_uint64]),
    "gsx_hip_adc_context_destroy": (_st, [_vp]),
    "gsx_hip_adc_step": (_st, [_vp, ctypes.POINTER(AdcParams), ctypes.c_uint64, ctypes.POINTER(GsRows), _i64,
                               ctypes.POINTER(GsRows), ctypes.POINTER(_i32), ctypes.POINTER(_i64), _vp]),
    "gsx_hip_gather_rows_kernel_launch": (_st, [_vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
}

_LIB = None


def load(require_device: bool = True):
    """Load libgsx_hip.so and bind every entry point; raise if anything is missing."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise GsxHipError(f"{LIB_PATH} is missing; build it with __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    if require_device:
        n = _i32(0)
        st = _LIB.gsx_hip_device_count(ctypes.byref(n))
        if st != 0 or n.value < 1:
            raise GsxHipError("no HIP device is visible: the gsx_amd kernels need an MI355X (gfx950)")
    return _LIB


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = _LIB.gsx_hip_last_error_message().decode(errors="replace") if _LIB is not None else ""
        raise GsxHipError(f"{what} failed with status {status}: {msg}")
