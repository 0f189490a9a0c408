"""Loading of the golden fixtures in tests/golden (written by tests/golden/make_goldens.py from the
reference CPU backend built from its own sources)."""
from __future__ import annotations

import os

import numpy as np

from gsx_amd import scenes

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RENDER_CASES = ("render_c0", "render_c1_sh3", "render_c3", "render_c2_sh1")
FD_CASES = ("fd_gradient", "fd_alpha_saturation", "fd_rotated_anisotropic", "fd_hard_culling")
GRAD_FIELDS = ("mean3d", "rotation", "logscale", "opacity", "sh0", "sh1", "sh2", "sh3")


def load(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def scene_of(d: dict) -> scenes.Scene:
    deg = int(d["in_sh_degree"])
    sc = scenes.Scene(d["in_mean3d"], d["in_rotation"], d["in_logscale"], d["in_opacity"], d["in_sh0"], deg)
    for k in (1, 2, 3):
        if deg >= k:
            setattr(sc, f"sh{k}", d[f"in_sh{k}"])
    return sc


def grads_of(d: dict) -> dict:
    return {k: d[f"grad_{k}"] for k in GRAD_FIELDS if f"grad_{k}" in d}


# tests/render_runtime.cpp:934-1089: (field, component, tolerance) checked against central
# differences with epsilon 1e-3 on the loss sum(out_rgb * grad_rgb)
FD_CHECKS = {
    "fd_gradient": [("mean3d", 0, 3e-2), ("mean3d", 1, 3e-2), ("mean3d", 2, 3e-2), ("rotation", 2, 5e-2),
                    ("logscale", 1, 3e-2), ("sh0", 1, 2e-2), ("sh1", 5, 2e-2), ("opacity", 0, 2e-2)],
    "fd_alpha_saturation": [("opacity", 0, 1e-2)],
    "fd_rotated_anisotropic": [("mean3d", 2, 5e-2), ("rotation", 2, 5e-2), ("rotation", 3, 5e-2),
                               ("logscale", 0, 5e-2), ("logscale", 1, 5e-2)],
    "fd_hard_culling": [("mean3d", 1, 5e-2), ("mean3d", 2, 5e-2), ("rotation", 2, 5e-2), ("logscale", 0, 5e-2),
                        ("logscale", 1, 5e-2)],
}


def central_difference(render, scene: scenes.Scene, field: str, index: int, grad_rgb: np.ndarray,
                       eps: float = 1e-3) -> float:
    """(L(x + eps) - L(x - eps)) / (2 eps) with L = sum(render(scene) * grad_rgb) in float32, as
    numerical_gradient / dot_product of tests/render_runtime.cpp:154-165, 469-501."""
    arr = getattr(scene, field)
    flat = arr.reshape(-1)
    orig = flat[index]
    flat[index] = np.float32(orig + np.float32(eps))
    plus = np.float32(np.sum(render(scene).astype(np.float32) * grad_rgb, dtype=np.float32))
    flat[index] = np.float32(orig - np.float32(eps))
    minus = np.float32(np.sum(render(scene).astype(np.float32) * grad_rgb, dtype=np.float32))
    flat[index] = orig
    return float((plus - minus) / np.float32(2.0 * eps))
