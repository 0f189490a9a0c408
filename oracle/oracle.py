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
        lib.oracle_tiled.restype = _i64
        lib.oracle_tiled.argtypes = [_i64, ctypes.c_int] + [_vp] * 9 + [ctypes.c_int32, ctypes.c_int, _vp, _vp,
                                                                         _vp, _vp]
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


class Reference:
    """The unmodified reference CPU backend (oracle/_ref/libgsxref.so)."""

    path = os.path.join(HERE, "_ref", "libgsxref.so")

    @classmethod
    def available(cls) -> bool:
        return os.path.exists(cls.path)

    def __init__(self):
        lib = ctypes.CDLL(self.path)
        lib.gsxref_last_error.restype = ctypes.c_char_p
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
        lib.gsxref_train_step.argtypes = [ctypes.c_int, ctypes.c_int] + [_vp] * 7 + [_f, _f, _vp, _vp]
        self.lib = lib

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

    def adc(self, fields, aux, params: AdcParams, capacity):
        n = fields["mean3d"].shape[0]
        fp = np.array([params.pruning_opacity_threshold, params.opacity_clamp_value, params.max_world_scale, 0.0,
                       params.duplicate_grad_threshold, params.duplicate_scale_threshold,
                       params.duplicate_absgrad_threshold, params.scene_scale, 0, 0], np.float32)
        ip = np.array([params.algorithm, params.refine_every, params.start_refine, params.end_refine,
                       params.max_num_gaussians, params.reset_every, params.global_step, params.seed], np.int64)
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

    def train_steps(self, scene, camera, target, iters, w_l1=0.8, w_ssim=0.2, lrs=(1e-3, 1e-2)):
        stages = np.zeros(5, np.float64)
        sc = scene.copy()
        self._check(self.lib.gsxref_train_step(sc.count, iters, _p(sc.mean3d), _p(sc.rotation), _p(sc.logscale),
                                               _p(sc.opacity), _p(sc.sh0), _p(camera), _p(target), w_l1, w_ssim,
                                               _p(np.asarray(lrs, np.float32)), _p(stages)))
        return sc, stages
