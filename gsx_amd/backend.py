"""Host-side mirror of gsx's renderer / loss / optimizer interface over libgsx_hip.so.

Names and semantics follow the gsx public API (gsx/include/gsx/gsx-render.h, gsx-loss.h,
gsx-optim.h): a render context retains TRAIN state for exactly one backward; gradient sinks
of the render backward are overwritten; loss maps and prediction gradients accumulate; Adam
keeps per-group moments and step counts. Device memory and streams come from PyTorch (ROCm);
every computation runs in the HIP kernels of libgsx_hip.so.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import Camera, GaussianGrads, Gaussians, GsxHipError, check

__all__ = ["Camera", "Renderer", "Loss", "Adam", "DensityControl", "GsxHipError", "stream_handle", "ptr"]


def ptr(t: torch.Tensor | None):
    if t is None:
        return None
    if not t.is_cuda:
        raise GsxHipError("gsx_amd tensors must live on the HIP device")
    if not t.is_contiguous():
        raise GsxHipError("gsx_amd tensors must be contiguous")
    if t.dtype not in (torch.float32, torch.int32, torch.uint32, torch.int64, torch.uint64, torch.uint8):
        raise GsxHipError(f"unsupported dtype {t.dtype}")
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(stream: torch.cuda.Stream | None = None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


@dataclass
class GaussianTensors:
    mean3d: torch.Tensor
    rotation: torch.Tensor
    logscale: torch.Tensor
    opacity: torch.Tensor
    sh0: torch.Tensor
    sh_degree: int = 0
    sh1: torch.Tensor | None = None
    sh2: torch.Tensor | None = None
    sh3: torch.Tensor | None = None

    @property
    def count(self) -> int:
        return int(self.mean3d.shape[0])

    def to_struct(self) -> Gaussians:
        g = Gaussians()
        g.count = self.count
        g.sh_degree = self.sh_degree
        for name in ("mean3d", "rotation", "logscale", "opacity", "sh0", "sh1", "sh2", "sh3"):
            setattr(g, name, ptr(getattr(self, name)))
        return g

    @classmethod
    def from_scene(cls, scene, device="cuda") -> "GaussianTensors":
        def t(a):
            return None if a is None else torch.from_numpy(a).to(device)
        return cls(t(scene.mean3d), t(scene.rotation), t(scene.logscale), t(scene.opacity), t(scene.sh0),
                   scene.sh_degree, t(scene.sh1), t(scene.sh2), t(scene.sh3))

    def zeros_like_grads(self) -> "GaussianTensors":
        z = lambda a: None if a is None else torch.zeros_like(a)  # noqa: E731
        return GaussianTensors(z(self.mean3d), z(self.rotation), z(self.logscale), z(self.opacity), z(self.sh0),
                               self.sh_degree, z(self.sh1), z(self.sh2), z(self.sh3))

    def grads_struct(self) -> GaussianGrads:
        g = GaussianGrads()
        for name in ("mean3d", "rotation", "logscale", "opacity", "sh0", "sh1", "sh2", "sh3"):
            setattr(g, name, ptr(getattr(self, name)))
        return g


class Renderer:
    """gsx_renderer + gsx_render_context on the HIP backend (gsx-render.h:148-165)."""

    def __init__(self, width: int, height: int):
        self.lib = _lib.load()
        self.width = int(width)
        self.height = int(height)
        h = ctypes.c_void_p()
        check(self.lib.gsx_hip_render_context_create(ctypes.byref(h)), "render context create")
        self.handle = h

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.gsx_hip_render_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def render(self, camera: Camera, gaussians: GaussianTensors, train: bool = False,
               out_rgb: torch.Tensor | None = None, visible_counter: torch.Tensor | None = None,
               stream=None, borrow_train_state: bool = True) -> torch.Tensor:
        """train=True is GSX_RENDER_FORWARD_TYPE_TRAIN. borrow_train_state (gsx-render.h:101): True
        differentiates the backward at the values the Gaussian tensors hold when backward() is
        called, False at the values of this forward."""
        if camera.width != self.width or camera.height != self.height:
            raise GsxHipError("intrinsics geometry must match the renderer output geometry")
        if out_rgb is None:
            out_rgb = torch.empty((3, self.height, self.width), dtype=torch.float32, device="cuda")
        g = gaussians.to_struct()
        mode = (_lib.FORWARD_TRAIN_BORROW if borrow_train_state else _lib.FORWARD_TRAIN_CLONE) if train else \
            _lib.FORWARD_INFERENCE
        check(self.lib.gsx_hip_render_forward(self.handle, ctypes.byref(camera), ctypes.byref(g), mode,
                                              ptr(out_rgb), ptr(visible_counter), stream_handle(stream)),
              "render forward")
        return out_rgb

    def backward(self, grad_rgb: torch.Tensor, grads: GaussianTensors, stream=None) -> None:
        gg = grads.grads_struct()
        check(self.lib.gsx_hip_render_backward(self.handle, ptr(grad_rgb), ctypes.byref(gg), stream_handle(stream)),
              "render backward")

    def stats(self) -> _lib.RenderStats:
        s = _lib.RenderStats()
        check(self.lib.gsx_hip_render_context_get_stats(self.handle, ctypes.byref(s)), "get stats")
        return s

    def buffers(self) -> _lib.RenderBuffers:
        b = _lib.RenderBuffers()
        check(self.lib.gsx_hip_render_context_get_buffers(self.handle, ctypes.byref(b)), "get buffers")
        return b

    def set_timing(self, capacity: int) -> None:
        """Record per-stage HIP events for the next `capacity` forward/backward pairs (0 = off)."""
        check(self.lib.gsx_hip_render_context_set_timing(self.handle, int(capacity)), "set timing")

    STAGES = ("preprocess", "depth_order", "emit", "sort", "ranges", "blend_forward", "blend_backward", "instance_reduce",
              "projection_backward")

    def timings(self) -> dict:
        arr = (ctypes.c_float * len(self.STAGES))()
        written = ctypes.c_int32(0)
        check(self.lib.gsx_hip_render_context_get_timings(self.handle, arr, len(self.STAGES), ctypes.byref(written)),
              "get timings")
        return {name: float(arr[i]) for i, name in enumerate(self.STAGES[: written.value])}


class Loss:
    """gsx_loss for L1 / MSE / SSIM (gsx-loss.h). grad_normalization 'mean' divides by the
    element count (gsx-tensor-helpers.h:236-244)."""

    def __init__(self, algorithm: str, grad_normalization: str = "mean"):
        if algorithm not in ("l1", "mse", "ssim"):
            raise GsxHipError(f"unknown loss algorithm {algorithm}")
        self.lib = _lib.load()
        self.algorithm = algorithm
        self.mean = grad_normalization == "mean"
        self._pred = None
        self._target = None
        self._workspace = None

    def _grad_scale(self, numel: int, scale: float) -> float:
        s = ctypes.c_float(scale).value
        return ctypes.c_float(s / ctypes.c_float(float(numel)).value).value if self.mean else s

    @staticmethod
    def _image_layout(t: torch.Tensor):
        if t.dim() == 3:
            return 1, t.shape[0], t.shape[1], t.shape[2]
        if t.dim() == 4:
            return t.shape[0], t.shape[1], t.shape[2], t.shape[3]
        raise GsxHipError("ssim expects [C,H,W] or [B,C,H,W]")

    def forward(self, prediction: torch.Tensor, target: torch.Tensor, loss_map: torch.Tensor, scale: float = 1.0,
                train: bool = True, stream=None) -> None:
        n = prediction.numel()
        st = stream_handle(stream)
        if self.algorithm == "ssim":
            outer, c, h, w = self._image_layout(prediction)
            if self._workspace is None or self._workspace.numel() < 3 * n:
                self._workspace = torch.empty(3 * n, dtype=torch.float32, device="cuda")
            check(self.lib.gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(
                ptr(loss_map), ptr(prediction), ptr(target), outer, c, h, w, scale,
                ptr(self._workspace) if train else None, 0.0, 0, st), "ssim forward")
        elif self.algorithm == "l1":
            check(self.lib.gsx_hip_loss_l1_f32_forward_kernel_launch(ptr(loss_map), ptr(prediction), ptr(target), n,
                                                                     scale, st), "l1 forward")
        else:
            check(self.lib.gsx_hip_loss_mse_f32_forward_kernel_launch(ptr(loss_map), ptr(prediction), ptr(target), n,
                                                                      scale, st), "mse forward")
        self._pred, self._target = (prediction, target) if train else (None, None)

    def backward(self, grad_prediction: torch.Tensor, scale: float = 1.0, stream=None) -> None:
        if self._pred is None:
            raise GsxHipError("loss backward requires a train forward on the same context")
        n = self._pred.numel()
        gs = self._grad_scale(n, scale)
        st = stream_handle(stream)
        if self.algorithm == "ssim":
            outer, c, h, w = self._image_layout(self._pred)
            check(self.lib.gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(
                ptr(grad_prediction), ptr(self._pred), ptr(self._target), outer, c, h, w, gs, ptr(self._workspace),
                0.0, 0, st), "ssim backward")
        elif self.algorithm == "l1":
            check(self.lib.gsx_hip_loss_l1_f32_backward_kernel_launch(ptr(grad_prediction), ptr(self._pred),
                                                                      ptr(self._target), n, gs, st), "l1 backward")
        else:
            check(self.lib.gsx_hip_loss_mse_f32_backward_kernel_launch(ptr(grad_prediction), ptr(self._pred),
                                                                       ptr(self._target), n, gs, st), "mse backward")


class Adam:
    """gsx_optim (Adam) over parameter groups, all groups in one launch per step."""

    def __init__(self, groups):
        """groups: list of dicts with parameter, gradient, learning_rate and optional beta1, beta2,
        weight_decay, epsilon, max_grad (defaults 0.9, 0.999, 0, 1e-8, 0)."""
        if len(groups) > _lib.ADAM_MAX_GROUPS:
            raise GsxHipError("too many parameter groups")
        self.lib = _lib.load()
        self.groups = []
        for g in groups:
            p = g["parameter"]
            self.groups.append(dict(parameter=p, gradient=g["gradient"], learning_rate=float(g["learning_rate"]),
                                    beta1=float(g.get("beta1", 0.9)), beta2=float(g.get("beta2", 0.999)),
                                    weight_decay=float(g.get("weight_decay", 0.0)),
                                    epsilon=float(g.get("epsilon", 1e-8)), max_grad=float(g.get("max_grad", 0.0)),
                                    m=torch.zeros_like(p), v=torch.zeros_like(p), step=0))

    def step(self, stream=None) -> None:
        arr = (_lib.AdamGroup * len(self.groups))()
        for i, g in enumerate(self.groups):
            g["step"] += 1
            b1 = ctypes.c_float(g["beta1"]).value
            b2 = ctypes.c_float(g["beta2"]).value
            a = arr[i]
            a.parameter = ptr(g["parameter"])
            a.gradient = ptr(g["gradient"])
            a.first_moment = ptr(g["m"])
            a.second_moment = ptr(g["v"])
            a.count = g["parameter"].numel()
            a.beta1, a.beta2 = b1, b2
            a.learning_rate = g["learning_rate"]
            a.weight_decay = g["weight_decay"]
            a.epsilon = g["epsilon"]
            a.max_grad = g["max_grad"]
            a.bias_correction1 = 1.0 - math.pow(b1, float(g["step"]))
            a.bias_correction2 = 1.0 - math.pow(b2, float(g["step"]))
        check(self.lib.gsx_hip_adam_step_multi_launch(arr, len(self.groups), stream_handle(stream)), "adam step")


FIELD_WIDTHS = {"mean3d": 3, "rotation": 4, "logscale": 3, "opacity": 1, "sh0": 3, "sh1": 9, "sh2": 15, "sh3": 21}
PARAM_FIELDS = ("mean3d", "rotation", "logscale", "opacity", "sh0", "sh1", "sh2", "sh3")
AUX_FIELDS = ("grad_acc", "absgrad_acc", "visible_counter", "max_screen_radius")


class DensityControl:
    """gsx_adc (DEFAULT / ABSGS) on the HIP backend (gsx-adc.h). Rows live in capacity-sized
    device buffers: growth appends in place, pruning compacts into a second buffer set."""

    def __init__(self, params: dict, seed: int = 0):
        self.lib = _lib.load()
        p = _lib.AdcParams()
        for name, _ in _lib.AdcParams._fields_:
            if name in params:
                setattr(p, name, params[name])
        self.params = p
        h = ctypes.c_void_p()
        check(self.lib.gsx_hip_adc_context_create(ctypes.byref(h), int(seed)), "adc context create")
        self.handle = h

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            self.lib.gsx_hip_adc_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def rows_struct(count: int, sh_degree: int, fields: dict, moments: dict | None) -> _lib.GsRows:
        r = _lib.GsRows()
        r.count = count
        r.sh_degree = sh_degree
        for name in PARAM_FIELDS + AUX_FIELDS:
            setattr(r, name, ptr(fields.get(name)))
        if moments is not None:
            for k, name in enumerate(PARAM_FIELDS):
                if name in moments:
                    r.first_moment[k] = ptr(moments[name][0])
                    r.second_moment[k] = ptr(moments[name][1])
        return r

    def step(self, global_step: int, count: int, sh_degree: int, fields: dict, moments: dict | None,
             capacity: int, out_fields: dict, out_moments: dict | None, stream=None):
        """Returns (new_count, result_in_out, counts[pruned, duplicated, grown, reset])."""
        rows = self.rows_struct(count, sh_degree, fields, moments)
        out = self.rows_struct(0, sh_degree, out_fields, out_moments)
        in_out = ctypes.c_int32(0)
        counts = (ctypes.c_int64 * 4)()
        check(self.lib.gsx_hip_adc_step(self.handle, ctypes.byref(self.params), int(global_step), ctypes.byref(rows),
                                        int(capacity), ctypes.byref(out), ctypes.byref(in_out), counts,
                                        stream_handle(stream)), "adc step")
        new_count = out.count if in_out.value else rows.count
        return int(new_count), bool(in_out.value), list(counts)
