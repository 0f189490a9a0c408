"""Seeded synthetic scenes, cameras and targets for the benchmark configurations.

The generator is host C (``csrc/scenes.c``, built into ``libgsx_scenes.so``) and uses
gsx's own pcg32 seeding and Box-Muller conventions (gsx/src/gsx-random.c:14-29, 86-112),
so the same bytes can be handed to the gsx CPU backend and to the gfx950 path.

A camera is a float32[18] block: fx, fy, cx, cy, width, height, qx, qy, qz, qw (world to
camera rotation, xyzw), tx, ty, tz, near, far, bg_r, bg_g, bg_b.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libgsx_scenes.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        lib = ctypes.CDLL(path)
        lib.gsx_scene_generate.restype = ctypes.c_int
        lib.gsx_scene_generate.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_int64] + [ctypes.c_void_p] * 6
        lib.gsx_scene_look_at.argtypes = [ctypes.c_void_p] * 3
        lib.gsx_scene_target.restype = ctypes.c_int
        lib.gsx_scene_target.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_int32, ctypes.c_void_p]
        lib.gsx_scene_pcg32_stream.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
        _LIB = lib
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


@dataclass
class Scene:
    mean3d: np.ndarray
    rotation: np.ndarray
    logscale: np.ndarray
    opacity: np.ndarray
    sh0: np.ndarray
    sh_degree: int = 0
    sh1: np.ndarray | None = None
    sh2: np.ndarray | None = None
    sh3: np.ndarray | None = None

    @property
    def count(self) -> int:
        return int(self.mean3d.shape[0])

    def copy(self) -> "Scene":
        return Scene(*(None if v is None else (v.copy() if isinstance(v, np.ndarray) else v)
                       for v in (self.mean3d, self.rotation, self.logscale, self.opacity, self.sh0,
                                 self.sh_degree, self.sh1, self.sh2, self.sh3)))


def generate(kind: int, seed: int, n: int, params) -> Scene:
    p = np.zeros(8, np.float32)
    p[: len(params)] = params
    arrays = [np.empty((n, 3), np.float32), np.empty((n, 4), np.float32), np.empty((n, 3), np.float32),
              np.empty((n,), np.float32), np.empty((n, 3), np.float32)]
    rc = _lib().gsx_scene_generate(kind, seed, n, _ptr(p), *[_ptr(a) for a in arrays])
    if rc != 0:
        raise ValueError(f"unknown scene kind {kind}")
    return Scene(*arrays)


def cube_scene(seed: int, n: int, extent=1.0, logscale=(-4.6, -3.0), logscale_normal=False,
               opacity=(0.0, 1.0), sh_sd=0.5) -> Scene:
    """Config 0/1/4 distributions: means U[-e,e]^3, N(0,1)^4 normalised rotations."""
    return generate(0, seed, n, [extent, logscale[0], logscale[1], 1.0 if logscale_normal else 0.0,
                                 opacity[0], opacity[1], sh_sd])


def plane_scene(seed: int, n: int, logscale=(-6.0, -5.0), z_sd=0.01, sh_sd=0.5) -> Scene:
    """Config 2: image-fit init on z = 0, opacity logit(0.1)."""
    return generate(1, seed, n, [logscale[0], logscale[1], z_sd, sh_sd])


def cluster_scene(seed: int, n: int, logscale=(-4.5, 0.6), opacity_sd=1.5, sh_sd=0.5,
                  shell_fraction=0.2, shell_radius=10.0) -> Scene:
    """Config 3: 64 anisotropic clusters plus a radius-10 background shell."""
    return generate(2, seed, n, [logscale[0], logscale[1], opacity_sd, sh_sd, shell_fraction, shell_radius])


def look_at(eye, target=(0.0, 0.0, 0.0)) -> np.ndarray:
    out = np.zeros(7, np.float32)
    _lib().gsx_scene_look_at(_ptr(np.asarray(eye, np.float32)), _ptr(np.asarray(target, np.float32)), _ptr(out))
    return out


def camera(width: int, height: int, fx: float, fy: float | None = None, cx: float | None = None,
           cy: float | None = None, pose=(1.0, 0.0, 0.0, 0.0, 0.0, 0.0, 4.0), near=0.01, far=100.0,
           background=(0.0, 0.0, 0.0)) -> np.ndarray:
    """Pinhole camera block. The default pose is "at (0,0,4) looking at the origin":
    rot = (1,0,0,0) xyzw (180 degrees about x), transl = (0,0,4)."""
    fy = fx if fy is None else fy
    cx = width / 2.0 if cx is None else cx
    cy = height / 2.0 if cy is None else cy
    return np.array([fx, fy, cx, cy, width, height, *pose, near, far, *background], np.float32)


def orbit_pose(index: int, count: int = 24, radius: float = 6.0, height: float = 0.0) -> np.ndarray:
    theta = 2.0 * math.pi * index / count
    eye = (radius * math.cos(theta), height, radius * math.sin(theta))
    return look_at(eye)


def target_image(kind: int, seed: int, width: int, height: int, param: int) -> np.ndarray:
    out = np.empty((3, height, width), np.float32)
    rc = _lib().gsx_scene_target(kind, seed, width, height, param, _ptr(out))
    if rc != 0:
        raise ValueError("unknown target kind")
    return out


def pcg32_stream(seed: int, count: int, normal: bool) -> np.ndarray:
    out = np.empty(count, np.float32)
    _lib().gsx_scene_pcg32_stream(seed, count, 1 if normal else 0, _ptr(out))
    return out


@dataclass
class Workload:
    name: str
    scene: Scene
    camera: np.ndarray
    target: np.ndarray | None = None
    extra: dict = field(default_factory=dict)


def config0(n: int = 100_000, width: int = 640, height: int = 480) -> Workload:
    """CPU-backend forward render: 100k Gaussians, seed 0, 640x480, f=500."""
    sc = cube_scene(0, n)
    cam = camera(width, height, 500.0 * width / 640.0, cx=width / 2.0, cy=height / 2.0, near=0.01, far=100.0)
    return Workload("c0", sc, cam)


def config1(n: int = 500_000, width: int = 1280, height: int = 720) -> Workload:
    """Forward + backward with L1: 500k Gaussians, seed 1, 1280x720, f=1000, blurred-noise target."""
    sc = cube_scene(1, n)
    f = 1000.0 * width / 1280.0
    cam = camera(width, height, f, near=0.01, far=100.0)
    return Workload("c1", sc, cam, target_image(0, 101, width, height, 2))


def config2(n: int = 1_000_000, size: int = 1024) -> Workload:
    """Image-fit training: 1M Gaussians on z=0, 1024^2, f=2048, sinusoid target."""
    sc = plane_scene(2, n)
    cam = camera(size, size, 2048.0 * size / 1024.0, near=0.01, far=100.0)
    return Workload("c2", sc, cam, target_image(1, 102, size, size, 32))


def config3(n: int = 3_000_000, width: int = 1920, height: int = 1080, pose_index: int = 0) -> Workload:
    """Scene-scale training: clusters + shell, 24 orbit poses at r=6, 1080p, f=1600."""
    sc = cluster_scene(3, n)
    cam = camera(width, height, 1600.0 * width / 1920.0, pose=tuple(orbit_pose(pose_index)), near=0.01, far=100.0)
    return Workload("c3", sc, cam, target_image(0, 103 + pose_index, width, height, 2))


def metric_scene(n: int = 1_000_000, width: int = 1920, height: int = 1080, pose_index: int = 0) -> Workload:
    """The headline metric workload: the config-3 generator at N = 1M, 1080p, SH0."""
    w = config3(n, width, height, pose_index)
    w.name = "metric"
    return w


def config4(n: int = 6_000_000, width: int = 1920, height: int = 1080) -> Workload:
    """Sort/blend stress: U[-2,2]^3, logscale N(-3, 0.8), opacity N(1, 1), 1080p."""
    sc = cube_scene(4, n, extent=2.0, logscale=(-3.0, 0.8), logscale_normal=True, opacity=(1.0, 1.0))
    cam = camera(width, height, 1600.0 * width / 1920.0, pose=(1.0, 0.0, 0.0, 0.0, 0.0, 0.0, 6.0),
                 near=0.5, far=50.0)
    return Workload("c4", sc, cam, target_image(0, 104, width, height, 2))
