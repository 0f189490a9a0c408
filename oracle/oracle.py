"""ctypes access to the CPU checkers.

TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this module, and only as the checker / the CPU baseline. The product path
(gsx_amd/) never imports it.

- ``Oracle``: the C restatement ``liboracle.so`` (gsx_oracle.c), citing the reference lines
  it follows; portable, built on every machine.
- ``Reference``: ``_ref/libgsxref.so``, the unmodified gsx core + CPU backend compiled from
  the reference sources where they lie, driven through gsx's public API by ref_driver.c.
  Present only when it was built in a container that has the reference tree.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REC_FLOATS = 18
REC = {name: i for i, name in enumerate(
    ["mean2d_x", "mean2d_y", "cov_a", "cov_b", "cov_c", "inv_det", "depth", "x_cam", "y_cam", "z_cam",
     "color_r", "color_g", "color_b", "opacity", "raw_opacity", "dir_x", "dir_y", "dir_z"])}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the checkers must be C-contiguous"
    return a.ctypes.data_as(_vp)


def _sh(scene, k):
    return getattr(scene, f"sh{k}") if scene.sh_degree >= k else None


class AdcParams(ctypes.Structure):
    _fields_ = [("algorithm", ctypes.c_int32), ("pruning_opacity_threshold", _f), ("opacity_clamp_value", _f),
                ("max_world_scale", _f), ("duplicate_grad_threshold", _f), ("duplicate_scale_threshold", _f),
                ("duplicate_absgrad_threshold", _f), ("scene_scale", _f), ("refine_every", _i64),
                ("start_refine", _i64), ("end_refine", _i64), ("max_num_gaussians", _i64),
                ("reset_every", _i64), ("global_step", _i64), ("seed", ctypes.c_uint64),
                ("rng_draws_consumed", ctypes.c_uint64)]


class Oracle:
    def __init__(self):
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(path)
        lib.oracle_preprocess.restype = _i64
        lib.oracle_preprocess.argtypes = [_i64, ctypes.c_int] + [_vp] * 12
        lib.oracle_tile_keys.restype = _i64
        lib.oracle_tile_keys.argtypes = [_i64, ctypes.c_int] + [_vp] * 9 + [ctypes.c_int32, _i64, _vp, _vp]
        lib.oracle_tile_ranges.argtypes = [_i64, _vp, _i64, _vp]
        lib.oracle_tile_may_contribute.restype = ctypes.c_int
        lib.oracle_tile_may_contribute.argtypes = [_f] * 6 + [ctypes.c_int] * 4
        lib.oracle_tile_band_columns.restype = None
        lib.oracle_tile_band_columns.argtypes = [_f] * 6 + [ctypes.c_int] * 6 + [ctypes.POINTER(ctypes.c_int)]
        lib.oracle_contribution_box.restype = None
        lib.oracle_contribution_box.argtypes = [_f] * 6 + [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_int)]
        lib.oracle_tile_logf.restype = _f
        lib.oracle_tile_logf.argtypes = [_f]
        lib.oracle_render_forward.restype = ctypes.c_int
        lib.oracle_render_forward.argtypes = [_i64, ctypes.c_int] + [_vp] * 12
        lib.oracle_render_backward.restype = ctypes.c_int
        lib.oracle_render_backward.argtypes = [_i64, ctypes.c_int] + [_vp] * 18
        for name in ("oracle_loss_l1", "oracle_loss_mse"):
            getattr(lib, name).argtypes = [_i64, _vp, _vp, _f, _f, _vp, _vp]
        lib.oracle_loss_ssim.restype = ctypes.c_int
        lib.oracle_loss_ssim.argtypes = [_i64, _i64, _i64, _i64, _vp, _vp, _f, _f, _vp, _vp]
        lib.oracle_adam_step.argtypes = [_i64, _vp, _vp, _vp, _vp, _f, _f, _f, _f, _f, _f, _i64]
        lib.oracle_gather_rows.restype = ctypes.c_int
        lib.oracle_gather_rows.argtypes = [_vp, _i64, _i64, _vp, _i64, _vp]
        lib.oracle_adc_step.restype = _i64
        lib.oracle_adc_step.argtypes = [_i64, _vp, _vp, _vp, ctypes.POINTER(AdcParams), _vp]
        lib.oracle_expf_mismatches.restype = ctypes.c_uint64
        lib.oracle_expf_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        lib.oracle_expf_blend_mismatches.restype = ctypes.c_uint64
        lib.oracle_expf_blend_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        lib.oracle_libm_mismatches.restype = ctypes.c_uint64
        lib.oracle_libm_mismatches.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        lib.oracle_powf_mismatches.restype = ctypes.c_uint64
        lib.oracle_powf_mismatches.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int]
        lib.oracle_tiled.restype = _i64
        lib.oracle_tiled.argtypes = [_i64, ctypes.c_int] + [_vp] * 9 + [ctypes.c_int32, ctypes.c_int, _vp, _vp,
                                                                         _vp, _vp]
        lib.oracle_tiled_backward.restype = ctypes.c_int
        lib.oracle_tiled_backward.argtypes = [_i64, ctypes.c_int] + [_vp] * 9 + [ctypes.c_int32] + [_vp] * 9
        lib.oracle_free.argtypes = [_vp]
        self.lib = lib

    # -- render -----------------------------------------------------------------------------
    def _scene_args(self, scene):
        return [_p(scene.mean3d), _p(scene.rotation), _p(scene.logscale), _p(scene.opacity), _p(scene.sh0),
                _p(_sh(scene, 1)), _p(_sh(scene, 2)), _p(_sh(scene, 3))]

    def preprocess(self, scene, camera):
        n = scene.count
        idx = np.empty(max(n, 1), np.int64)
        rec = np.empty((max(n, 1), REC_FLOATS), np.float32)
        bbox = np.empty((max(n, 1), 4), np.int32)
        v = self.lib.oracle_preprocess(n, scene.sh_degree, *self._scene_args(scene), _p(camera), _p(idx), _p(rec),
                                       _p(bbox))
        return idx[:v], rec[:v], bbox[:v]

    def tile_keys(self, scene, camera, tile=16):
        n = scene.count
        cap = 1 << 16
        while True:
            keys = np.empty(cap, np.uint64)
            vals = np.empty(cap, np.uint32)
            r = self.lib.oracle_tile_keys(n, scene.sh_degree, *self._scene_args(scene), _p(camera), tile, cap,
                                          _p(keys), _p(vals))
            if r >= 0:
                return keys[:r], vals[:r]
            cap = -r - 1 + 16

    def tile_may_contribute(self, mx, my, inv_a, inv_b, inv_c, opacity, px0, px1, py0, py1) -> bool:
        return bool(self.lib.oracle_tile_may_contribute(mx, my, inv_a, inv_b, inv_c, opacity, px0, px1, py0, py1))

    def tile_band_columns(self, mx, my, inv_a, inv_b, inv_c, opacity, box, py0, py1) -> tuple:
        """(first, last) kept pixel column of the band of rows [py0, py1] of the pixel box
        box = (x0, x1, y0, y1); first > last when none (tile_cull.h)."""
        out = (ctypes.c_int * 2)()
        self.lib.oracle_tile_band_columns(mx, my, inv_a, inv_b, inv_c, opacity, *box, py0, py1, out)
        return int(out[0]), int(out[1])

    def contribution_box(self, mx, my, inv_a, inv_b, inv_c, opacity, box) -> tuple:
        """(xa, xb, ya, yb): the rectangle of the pixel box (x0, x1, y0, y1) that holds every pixel
        that may receive a contribution (tile_cull.h gsx_contribution_box); empty when xa > xb or
        ya > yb."""
        out = (ctypes.c_int * 4)()
        self.lib.oracle_contribution_box(mx, my, inv_a, inv_b, inv_c, opacity, *box, out)
        return tuple(int(v) for v in out)

    def tile_ranges(self, keys, tile_count):
        ranges = np.zeros((tile_count, 2), np.uint32)
        self.lib.oracle_tile_ranges(len(keys), _p(np.ascontiguousarray(keys)), tile_count, _p(ranges))
        return ranges

    def render(self, scene, camera, visible_counter=None):
        w, h = int(camera[4]), int(camera[5])
        out = np.zeros((3, h, w), np.float32)
        t = np.zeros((h, w), np.float32)
        rc = self.lib.oracle_render_forward(scene.count, scene.sh_degree, *self._scene_args(scene), _p(camera),
                                            _p(out), _p(t), _p(visible_counter))
        assert rc == 0
        return out, t

    def _tiled(self, scene, camera, cull, render, keys, tile=16):
        w, h = int(camera[4]), int(camera[5])
        out = np.zeros((3, h, w), np.float32) if render else None
        t = np.zeros((h, w), np.float32) if render else None
        kp, vp = _vp(), _vp()
        r = self.lib.oracle_tiled(scene.count, scene.sh_degree, *self._scene_args(scene), _p(camera), tile,
                                  1 if cull else 0, _p(out), _p(t), ctypes.byref(kp) if keys else None,
                                  ctypes.byref(vp) if keys else None)
        if r < 0:
            raise MemoryError("oracle_tiled failed")
        k = v = None
        if keys:
            try:
                k = np.ctypeslib.as_array(ctypes.cast(kp, ctypes.POINTER(ctypes.c_uint64)), (max(r, 1),))[:r].copy()
                v = np.ctypeslib.as_array(ctypes.cast(vp, ctypes.POINTER(ctypes.c_uint32)), (max(r, 1),))[:r].copy()
            finally:
                self.lib.oracle_free(kp)
                self.lib.oracle_free(vp)
        return out, t, k, v, r

    def render_tiled(self, scene, camera, cull=True):
        """Same pixels as render() (bit for bit), from per-tile lists walked per pixel on all
        host cores; with cull, over the instances the tile test keeps."""
        out, t, _, _, _ = self._tiled(scene, camera, cull, True, False)
        return out, t

    def tile_keys_tiled(self, scene, camera, tile=16):
        """Same keys and values as tile_keys(), built per tile on all host cores."""
        _, _, k, v, _ = self._tiled(scene, camera, True, False, True, tile)
        return k, v

    def render_and_keys_tiled(self, scene, camera):
        out, t, k, v, _ = self._tiled(scene, camera, True, True, True)
        return out, t, k, v

    @staticmethod
    def _grad_sinks(scene):
        n = scene.count
        g = {"mean3d": np.zeros((n, 3), np.float32), "rotation": np.zeros((n, 4), np.float32),
             "logscale": np.zeros((n, 3), np.float32), "opacity": np.zeros((n,), np.float32),
             "sh0": np.zeros((n, 3), np.float32)}
        for k, c in ((1, 3), (2, 5), (3, 7)):
            if scene.sh_degree >= k:
                g[f"sh{k}"] = np.zeros((n, c, 3), np.float32)
        return g

    def render_backward_tiled(self, scene, camera, grad_rgb, tile=16):
        """The serial render_backward's gradients from per-tile walks on all host cores: the
        same per-contribution terms, each Gaussian's terms summed in double (tiles ascending)
        instead of the CPU's float sum in box-raster order."""
        g = self._grad_sinks(scene)
        rc = self.lib.oracle_tiled_backward(
            scene.count, scene.sh_degree, *self._scene_args(scene), _p(camera), tile,
            _p(np.ascontiguousarray(grad_rgb, dtype=np.float32)), _p(g["mean3d"]), _p(g["rotation"]),
            _p(g["logscale"]), _p(g["opacity"]), _p(g["sh0"]), _p(g.get("sh1")), _p(g.get("sh2")), _p(g.get("sh3")))
        if rc != 0:
            raise MemoryError("oracle_tiled_backward failed")
        return g

    def render_backward(self, scene, camera, grad_rgb):
        n = scene.count
        g = {"mean3d": np.zeros((n, 3), np.float32), "rotation": np.zeros((n, 4), np.float32),
             "logscale": np.zeros((n, 3), np.float32), "opacity": np.zeros((n,), np.float32),
             "sh0": np.zeros((n, 3), np.float32)}
        for k, c in ((1, 3), (2, 5), (3, 7)):
            if scene.sh_degree >= k:
                g[f"sh{k}"] = np.zeros((n, c, 3), np.float32)
        rc = self.lib.oracle_render_backward(
            n, scene.sh_degree, *self._scene_args(scene), _p(camera), _p(np.ascontiguousarray(grad_rgb)),
            _p(g["mean3d"]), _p(g["rotation"]), _p(g["logscale"]), _p(g["opacity"]), _p(g["sh0"]),
            _p(g.get("sh1")), _p(g.get("sh2")), _p(g.get("sh3")))
        assert rc == 0
        return g

    # -- loss / optim / adc ---------------------------------------------------------------------
    def loss(self, algorithm, pred, target, scale, loss_map, grad, mean=True):
        """algorithm: 'l1' | 'mse' | 'ssim'; pred/target [C,H,W] or [B,C,H,W]; accumulators updated."""
        count = pred.size
        grad_scale = np.float32(scale) / np.float32(count) if mean else np.float32(scale)
        if algorithm == "ssim":
            shape = pred.shape if pred.ndim == 4 else (1,) + pred.shape
            rc = self.lib.oracle_loss_ssim(shape[0], shape[1], shape[2], shape[3], _p(pred), _p(target), scale,
                                           grad_scale, _p(loss_map), _p(grad))
            assert rc == 0
        else:
            fn = self.lib.oracle_loss_l1 if algorithm == "l1" else self.lib.oracle_loss_mse
            fn(count, _p(pred), _p(target), scale, grad_scale, _p(loss_map), _p(grad))

    def adam_step(self, param, grad, m, v, lr, beta1, beta2, weight_decay, epsilon, max_grad, step):
        self.lib.oracle_adam_step(param.size, _p(param), _p(grad), _p(m), _p(v), lr, beta1, beta2, weight_decay,
                                  epsilon, max_grad, step)

    def gather_rows(self, src, index):
        out = np.empty((len(index),) + src.shape[1:], src.dtype)
        row_bytes = src.strides[0]
        rc = self.lib.oracle_gather_rows(_p(src), src.shape[0], row_bytes, _p(index), len(index), _p(out))
        if rc != 0:
            raise IndexError("gather index out of range")
        return out

    def adc_step(self, fields, moments, aux, params: AdcParams, capacity):
        """fields: dict mean3d/rotation/logscale/opacity/sh0 of n rows. Returns new dicts."""
        n = fields["mean3d"].shape[0]
        cap = max(capacity, n)
        widths = {"mean3d": 3, "rotation": 4, "logscale": 3, "opacity": 1, "sh0": 3}
        order = ["mean3d", "rotation", "logscale", "opacity", "sh0"]
        fa = {k: np.zeros((cap, widths[k]), np.float32) for k in order}
        for k in order:
            fa[k][:n] = fields[k].reshape(n, widths[k])
        ma = None
        if moments is not None:
            ma = {}
            for k in order:
                for j in (0, 1):
                    arr = np.zeros((cap, widths[k]), np.float32)
                    arr[:n] = moments[k][j].reshape(n, widths[k])
                    ma[(k, j)] = arr
        aa = [None, None, None]
        for j, k in enumerate(("grad_acc", "absgrad_acc", "visible_counter")):
            if aux.get(k) is not None:
                arr = np.zeros(cap, np.float32)
                arr[:n] = aux[k]
                aa[j] = arr
        fptrs = (_vp * 5)(*[fa[k].ctypes.data for k in order])
        mptrs = None
        if ma is not None:
            mptrs = (_vp * 10)(*[ma[(k, j)].ctypes.data for k in order for j in (0, 1)])
        aptrs = (_vp * 3)(*[None if a is None else a.ctypes.data for a in aa])
        counts = np.zeros(4, np.int64)
        new_n = self.lib.oracle_adc_step(n, fptrs, mptrs, aptrs, ctypes.byref(params), _p(counts))
        if new_n < 0:
            raise RuntimeError("oracle adc step failed")
        out_fields = {k: fa[k][:new_n].reshape((new_n,) if k == "opacity" else (new_n, widths[k])) for k in order}
        out_m = None
        if ma is not None:
            out_m = {k: (ma[(k, 0)][:new_n].copy(), ma[(k, 1)][:new_n].copy()) for k in order}
        return out_fields, out_m, counts

    def expf_mismatches(self, lo_bits, hi_bits, stride=1):
        return int(self.lib.oracle_expf_mismatches(lo_bits, hi_bits, stride))

    def expf_blend_mismatches(self, lo_bits, hi_bits, stride=1):
        return int(self.lib.oracle_expf_blend_mismatches(lo_bits, hi_bits, stride))

    def libm_mismatches(self, name, lo_bits=0, hi_bits=0xFFFFFFFF, stride=1):
        """Mismatches of gsx_logf / gsx_sinf / gsx_cosf against the host libm."""
        which = {"logf": 0, "sinf": 1, "cosf": 2}[name]
        return int(self.lib.oracle_libm_mismatches(which, lo_bits, hi_bits, stride))

    def powf_mismatches(self, seed, count, domain=False):
        return int(self.lib.oracle_powf_mismatches(seed, count, 1 if domain else 0))


class _OnBackend:
    """The driver library with every entry point run on one backend: the library keeps the
    selected backend in a global, so each call selects its own first."""

    _unselected = ("gsxref_use_backend", "gsxref_last_error")

    def __init__(self, lib, which):
        self._lib, self._which = lib, which

    def __getattr__(self, name):
        fn = getattr(self._lib, name)
        if not name.startswith("gsxref_") or name in self._unselected:
            return fn

        def call(*args):
            rc = self._lib.gsxref_use_backend(self._which)
            if rc != 0:
                raise RuntimeError(f"selecting the backend failed ({rc}): {self._lib.gsxref_last_error().decode()}")
            return fn(*args)
        return call


class Reference:
    """The unmodified reference core driven through gsx's public API.

    ``Reference()`` loads ``_ref/libgsxref.so`` (core + CPU backend). ``Reference(backend="hip")``
    loads ``_ref/libgsxref_hip.so``, the same core with the registry's GPU slot filled by the HIP
    backend plugin (gsx_amd/libgsx_hip_backend.so), and runs every call on that backend;
    ``backend="cpu"`` on that library runs the CPU backend of the same process.
    """

    path = os.path.join(HERE, "_ref", "libgsxref.so")
    hip_path = os.path.join(HERE, "_ref", "libgsxref_hip.so")
    hiptype_path = os.path.join(HERE, "_ref", "libgsxref_hiptype.so")
    BACKEND_TYPE = {"cpu": 0, "cuda": 1, "metal": 2, "hip": 3}  # gsx_backend_type + GSX_BACKEND_TYPE_HIP

    @classmethod
    def available(cls, hip: bool = False, hip_type: bool = False) -> bool:
        return os.path.exists(cls.hiptype_path if hip_type else (cls.hip_path if hip else cls.path))

    def __init__(self, backend: str | None = None, hip_type: bool = False):
        """hip_type: load ``_ref/libgsxref_hiptype.so`` instead, where the plugin registers under
        GSX_BACKEND_TYPE_HIP (a backend type of its own) and the CUDA slot stays empty;
        ``backend="hip"`` then selects the HIP-type device."""
        if hip_type:
            lib = ctypes.CDLL(self.hiptype_path)
        else:
            lib = ctypes.CDLL(self.path if backend is None else self.hip_path)
        lib.gsxref_last_error.restype = ctypes.c_char_p
        lib.gsxref_reduce.restype = ctypes.c_int
        lib.gsxref_reduce.argtypes = [ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp, _vp]
        lib.gsxref_elementwise.restype = ctypes.c_int
        lib.gsxref_elementwise.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]
        lib.gsxref_gather.restype = ctypes.c_int
        lib.gsxref_gather.argtypes = [ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int, _vp, _vp]
        lib.gsxref_random.restype = ctypes.c_int
        lib.gsxref_random.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_int, _f, _vp, ctypes.c_int, _vp]
        lib.gsxref_image.restype = ctypes.c_int
        lib.gsxref_image.argtypes = [ctypes.c_int] * 4 + [_vp, _vp]
        lib.gsxref_backend_device_name.restype = ctypes.c_char_p
        lib.gsxref_dataloader.restype = ctypes.c_int
        lib.gsxref_dataloader.argtypes = [ctypes.c_int] * 4 + [_vp, _vp, ctypes.c_int, ctypes.c_uint64, ctypes.c_int,
                                                                ctypes.c_int, _vp, _vp, _vp, _vp, _vp]
        lib.gsxref_render.restype = ctypes.c_int
        lib.gsxref_render.argtypes = [ctypes.c_int, ctypes.c_int] + [_vp] * 9 + [ctypes.c_int, _vp, _vp]
        lib.gsxref_render_grad.restype = ctypes.c_int
        lib.gsxref_render_grad.argtypes = [ctypes.c_int, ctypes.c_int] + [_vp] * 19
        lib.gsxref_loss.restype = ctypes.c_int
        lib.gsxref_loss.argtypes = [ctypes.c_int] * 6 + [_vp, _vp, _f, _vp, _vp]
        lib.gsxref_adam.restype = ctypes.c_int
        lib.gsxref_adam.argtypes = [ctypes.c_int, ctypes.c_int, _vp, _vp, _vp, _vp, _vp]
        lib.gsxref_adc.restype = ctypes.c_int
        lib.gsxref_adc.argtypes = [ctypes.c_int] + [_vp] * 10 + [ctypes.c_int, _vp] + [_vp] * 6
        lib.gsxref_train_step.restype = ctypes.c_int
        lib.gsxref_train_step.argtypes = [ctypes.c_int, ctypes.c_int] + [_vp] * 7 + [_f, _f, _vp, ctypes.c_int, _vp]
        lib.gsxref_session_fit.restype = ctypes.c_int
        lib.gsxref_session_fit.argtypes = [ctypes.c_int] * 3 + [_vp] * 7 + [_f, _f, _vp, ctypes.c_int, ctypes.c_int,
                                                                          _vp, _vp]
        self.StepHook = ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_double)
        lib.gsxref_set_step_hook.restype = None
        lib.gsxref_set_step_hook.argtypes = [self.StepHook]
        lib.gsxref_count_devices.restype = ctypes.c_int
        lib.gsxref_count_devices.argtypes = [ctypes.c_int]
        lib.gsxref_backend_type.restype = ctypes.c_int
        lib.gsxref_backend_family_name.restype = ctypes.c_char_p
        self._raw = lib
        slots = {"cpu": 0, "hip": 2 if hip_type else 1}
        self.lib = lib if backend is None else _OnBackend(lib, slots[backend])

    def session_fit(self, scene, camera, target_chw, warmup, iters, w_l1=0.8, w_ssim=0.2, lrs=(1e-3, 1e-2),
                    collect_timings=False, prefetch=0):
        """`warmup` + `iters` gsx_session_step calls configured as image-fit-demo's session (one
        image served by gsx_dataloader, L1 + SSIM loss items, Adam over the five SH0 roles,
        borrowed train state, no ADC). Returns (trained scene copy, seconds of the timed `iters`
        steps, the last step's report timings in us: dataloader, render fwd, loss fwd, loss bwd,
        render bwd, optim, adc, total)."""
        from gsx_amd import scenes as _scenes
        sc = _scenes.Scene(*(a.copy() for a in (scene.mean3d, scene.rotation, scene.logscale, scene.opacity,
                                                 scene.sh0)))
        hwc = np.ascontiguousarray(np.transpose(target_chw, (1, 2, 0)), dtype=np.float32)
        secs = np.zeros(1, np.float64)
        stage_us = np.zeros(8, np.float64)
        hyper = np.array(lrs, np.float32)
        self._check(self.lib.gsxref_session_fit(
            sc.count, warmup, iters, _p(sc.mean3d), _p(sc.rotation), _p(sc.logscale), _p(sc.opacity), _p(sc.sh0),
            _p(np.ascontiguousarray(camera, dtype=np.float32)), _p(hwc), w_l1, w_ssim, _p(hyper),
            1 if collect_timings else 0, prefetch, _p(secs), _p(stage_us)))
        return sc, float(secs[0]), stage_us

    def set_step_hook(self, fn):
        """fn(step, seconds) after each ADC step of adc() (the stream drained around the step), or
        None. The returned ctypes callback must stay referenced while it is installed."""
        cb = self.StepHook(fn) if fn is not None else self.StepHook()
        self._raw.gsxref_set_step_hook(cb)
        return cb

    def count_devices(self, backend_type: str) -> int:
        """Registered devices of a backend type (gsx_count_backend_devices_by_type)."""
        n = self._raw.gsxref_count_devices(self.BACKEND_TYPE[backend_type])
        if n < 0:
            raise RuntimeError(f"counting devices failed ({-n}): {self._raw.gsxref_last_error().decode()}")
        return n

    def backend_type(self) -> tuple:
        """(gsx_backend_type value, backend family name) of the selected backend's device."""
        return int(self.lib.gsxref_backend_type()), self.lib.gsxref_backend_family_name().decode()

    def device_name(self) -> str:
        return self.lib.gsxref_backend_device_name().decode()

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(f"reference call failed ({rc}): {self.lib.gsxref_last_error().decode()}")

    def _scene_args(self, scene):
        return [_p(scene.mean3d), _p(scene.rotation), _p(scene.logscale), _p(scene.opacity), _p(scene.sh0),
                _p(_sh(scene, 1)), _p(_sh(scene, 2)), _p(_sh(scene, 3))]

    def render(self, scene, camera, train=False, visible_counter=None):
        w, h = int(camera[4]), int(camera[5])
        out = np.zeros((3, h, w), np.float32)
        self._check(self.lib.gsxref_render(scene.count, scene.sh_degree, *self._scene_args(scene), _p(camera),
                                           1 if train else 0, _p(out), _p(visible_counter)))
        return out

    def render_grad(self, scene, camera, grad_rgb):
        n = scene.count
        w, h = int(camera[4]), int(camera[5])
        out = np.zeros((3, h, w), np.float32)
        g = {"mean3d": np.zeros((n, 3), np.float32), "rotation": np.zeros((n, 4), np.float32),
             "logscale": np.zeros((n, 3), np.float32), "opacity": np.zeros((n,), np.float32),
             "sh0": np.zeros((n, 3), np.float32)}
        for k, c in ((1, 3), (2, 5), (3, 7)):
            if scene.sh_degree >= k:
                g[f"sh{k}"] = np.zeros((n, c, 3), np.float32)
        self._check(self.lib.gsxref_render_grad(
            n, scene.sh_degree, *self._scene_args(scene), _p(camera), _p(np.ascontiguousarray(grad_rgb)), _p(out),
            _p(g["mean3d"]), _p(g["rotation"]), _p(g["logscale"]), _p(g["opacity"]), _p(g["sh0"]),
            _p(g.get("sh1")), _p(g.get("sh2")), _p(g.get("sh3"))))
        return out, g

    def loss(self, algorithm, pred, target, scale, loss_map, grad, mean=True):
        alg = {"l1": 0, "mse": 1, "ssim": 2}[algorithm]
        shape = pred.shape if pred.ndim == 4 else (1,) + pred.shape
        self._check(self.lib.gsxref_loss(alg, 0 if mean else 1, shape[0], shape[1], shape[2], shape[3], _p(pred),
                                         _p(target), scale, _p(loss_map), _p(grad)))

    def adam(self, param, grad, hyper, steps):
        self._check(self.lib.gsxref_adam(param.size, steps, _p(param), _p(grad),
                                         _p(np.asarray(hyper, np.float32)), None, None))

    def adc(self, fields, aux, params: AdcParams, capacity, noise_strength=0.0, grow_ratio=0.0, steps=1,
            optim_probe=False):
        """gsx_adc_step on a fresh set and Adam optimizer; `steps` consecutive global steps from
        params.global_step; optim_probe: an Adam step on normal gradients before and after, so
        the moments the ADC kept, moved or cleared show in the returned rows."""
        n = fields["mean3d"].shape[0]
        fp = np.array([params.pruning_opacity_threshold, params.opacity_clamp_value, params.max_world_scale, 0.0,
                       params.duplicate_grad_threshold, params.duplicate_scale_threshold,
                       params.duplicate_absgrad_threshold, params.scene_scale, noise_strength, grow_ratio],
                      np.float32)
        ip = np.array([params.algorithm, params.refine_every, params.start_refine, params.end_refine,
                       params.max_num_gaussians, params.reset_every, params.global_step, params.seed, steps,
                       1 if optim_probe else 0], np.int64)
        cap = max(capacity, n)
        out = {"mean3d": np.zeros((cap, 3), np.float32), "rotation": np.zeros((cap, 4), np.float32),
               "logscale": np.zeros((cap, 3), np.float32), "opacity": np.zeros((cap,), np.float32),
               "sh0": np.zeros((cap, 3), np.float32)}
        out_n = ctypes.c_int(0)
        counters = np.zeros(4, np.int64)
        self._check(self.lib.gsxref_adc(
            n, _p(fields["mean3d"]), _p(fields["rotation"]), _p(fields["logscale"]), _p(fields["opacity"]),
            _p(fields["sh0"]), _p(aux["grad_acc"]), _p(aux["absgrad_acc"]), _p(aux["visible_counter"]), _p(fp),
            _p(ip), cap, ctypes.byref(out_n), _p(out["mean3d"]), _p(out["rotation"]), _p(out["logscale"]),
            _p(out["opacity"]), _p(out["sh0"]), _p(counters)))
        k = out_n.value
        return {name: arr[:k] for name, arr in out.items()}, counters

    def train_steps(self, scene, camera, target, iters, w_l1=0.8, w_ssim=0.2, lrs=(1e-3, 1e-2),
                    skip_render_backward=False):
        """Seconds per stage (render forward, loss forward, loss backward, render backward, Adam)
        summed over `iters` steps; the updated scene."""
        stages = np.zeros(5, np.float64)
        sc = scene.copy()
        self._check(self.lib.gsxref_train_step(sc.count, iters, _p(sc.mean3d), _p(sc.rotation), _p(sc.logscale),
                                               _p(sc.opacity), _p(sc.sh0), _p(camera), _p(target), w_l1, w_ssim,
                                               _p(np.asarray(lrs, np.float32)), int(bool(skip_render_backward)),
                                               _p(stages)))
        return sc, stages

    # ---- tensor, random and image operations (gsx-core.h, gsx-random.h, extra/gsx-image.h)

    def reduce(self, op, x, start_axis, y=None):
        """op in sum/mean/max/mse/mae over axes [start_axis, ndim); returns the leading extents."""
        x = np.ascontiguousarray(x, np.float32)
        shape = np.asarray(x.shape, np.int32)
        out = np.zeros(x.shape[:start_axis] + (1,), np.float32)
        yy = None if y is None else np.ascontiguousarray(y, np.float32)
        code = {"sum": 0, "mean": 1, "max": 2, "mse": 3, "mae": 4}[op]
        self._check(self.lib.gsxref_reduce(code, x.ndim, _p(shape), start_axis, _p(x), _p(yy), _p(out)))
        return out.reshape(x.shape[:start_axis])

    def unary(self, op, x, inplace=False):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        code = {"exp": 0, "sigmoid": 1, "sigmoid_derivative": 2, "abs": 3}[op]
        self._check(self.lib.gsxref_elementwise(code, 1 if inplace else 0, x.size, _p(x), None, _p(out)))
        return out

    def clamp(self, x, lo, hi):
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros_like(x)
        params = np.array([lo, hi], np.float32)
        self._check(self.lib.gsxref_elementwise(4, 1, x.size, _p(x), _p(params), _p(out)))
        return out

    def check_finite(self, x) -> bool:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(1, np.float32)
        self._check(self.lib.gsxref_elementwise(5, 0, x.size, _p(x), None, _p(out)))
        return bool(out[0] != 0)

    def gather(self, x, index):
        x = np.ascontiguousarray(x, np.float32)
        x2 = x.reshape(x.shape[0], -1)
        index = np.ascontiguousarray(index, np.int32)
        out = np.zeros((index.size, x2.shape[1]), np.float32)
        self._check(self.lib.gsxref_gather(x2.shape[0], x2.shape[1], _p(x2), index.size, _p(index), _p(out)))
        return out.reshape((index.size,) + x.shape[1:])

    def random(self, kind, seed, count, param=0.0, cdf=None):
        """kind in rand/randn (param = sigma)/randint (param = bound)/multinomial (cdf)."""
        code = {"rand": 0, "randn": 1, "randint": 2, "multinomial": 3}[kind]
        out = np.zeros(count, np.float32 if code < 2 else np.int32)
        c = None if cdf is None else np.ascontiguousarray(cdf, np.float32)
        self._check(self.lib.gsxref_random(code, seed, count, param, _p(c), 0 if c is None else c.size, _p(out)))
        return out

    def image(self, kind, src, c, h, w):
        """kind in to_srgb/to_linear ([3,h,w] f32), hwc_to_chw/chw_to_hwc (f32), to_u8/from_u8 (CHW)."""
        code = {"to_srgb": 0, "to_linear": 1, "hwc_to_chw": 2, "chw_to_hwc": 3, "to_u8": 4, "from_u8": 5}[kind]
        src = np.ascontiguousarray(src)
        if code == 2:
            out = np.zeros((c, h, w), np.float32)
        elif code == 3:
            out = np.zeros((h, w, c), np.float32)
        elif code == 4:
            out = np.zeros((c, h, w), np.uint8)
        else:
            out = np.zeros((c, h, w), np.float32)
        self._check(self.lib.gsxref_image(code, c, h, w, _p(src), _p(out)))
        return out

    def dataloader(self, rgb, alpha=None, shuffle=True, seed=0, prefetch=0, steps=None):
        """Iterate gsx_dataloader over host images rgb [count, h, w, 3] (u8 or float32) and
        optional alpha [count, h, w]; returns CHW rgb [steps, 3, h, w], alpha [steps, h, w] or
        None, stable indices, epochs and the intrinsics' fx (100 + index) of every step."""
        rgb = np.ascontiguousarray(rgb)
        count, h, w, _ = rgb.shape
        is_u8 = rgb.dtype == np.uint8
        a = None if alpha is None else np.ascontiguousarray(alpha, rgb.dtype)
        steps = count if steps is None else steps
        out_rgb = np.zeros((steps, 3, h, w), np.float32)
        out_alpha = np.zeros((steps, h, w), np.float32) if a is not None else None
        idx = np.zeros(steps, np.int64)
        ep = np.zeros(steps, np.int64)
        fx = np.zeros(steps, np.float32)
        self._check(self.lib.gsxref_dataloader(count, h, w, 1 if is_u8 else 0, _p(rgb), _p(a), 1 if shuffle else 0,
                                               seed, prefetch, steps, _p(out_rgb), _p(out_alpha), _p(idx), _p(ep),
                                               _p(fx)))
        return out_rgb, out_alpha, idx, ep, fx
