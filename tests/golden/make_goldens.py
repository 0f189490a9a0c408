"""Write the golden fixtures of this directory from the reference CPU backend.

The reference library is oracle/_ref/libgsxref.so, compiled from the unmodified gsx sources
by `make -C oracle ref` (needs /root/reference, so this script runs in the build container
only). Each fixture is an .npz holding the inputs and the reference outputs of one case, so
the tests never need the reference at run time:

  render_*.npz  scene fields, camera block float[18], grad_rgb; out_rgb, visible_counter,
                gradients per field (gsx_renderer_render / gsx_renderer_backward, CPU backend)
  fd_*.npz      the four finite-difference scenes of tests/render_runtime.cpp:249-467 with
                their reference outputs and gradients
  loss.npz      L1 / MSE / SSIM map and gradient accumulation (gsx_loss_evaluate, MEAN)
  adam.npz      five gsx_optim_step calls on one group
  adc_*.npz     one gsx_adc_step (default / ABSGS) with seeded statistics

Usage: python tests/golden/make_goldens.py   (from the repository root)
"""
from __future__ import annotations

import os
import platform
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from gsx_amd import scenes  # noqa: E402
from oracle.oracle import AdcParams, Reference  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def provenance() -> str:
    gcc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    libc = " ".join(platform.libc_ver())
    return (f"reference CPU backend (oracle/_ref/libgsxref.so, gcc -O3 -std=c11, no -march), {gcc}, {libc}; "
            "scenes from gsx_amd/csrc/scenes.c (pcg32 seeded (seed, seed), fields filled in order mean3d, "
            "rotation, logscale, opacity, sh0)")


def scene_arrays(sc: scenes.Scene) -> dict:
    d = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
         "sh0": sc.sh0, "sh_degree": np.int32(sc.sh_degree)}
    for k in (1, 2, 3):
        arr = getattr(sc, f"sh{k}")
        if sc.sh_degree >= k and arr is not None:
            d[f"sh{k}"] = arr
    return d


def render_case(ref: Reference, name: str, sc: scenes.Scene, cam: np.ndarray, grad_rgb: np.ndarray) -> None:
    counter = np.zeros(sc.count, np.float32)
    ref.render(sc, cam, train=True, visible_counter=counter)
    out, grads = ref.render_grad(sc, cam, grad_rgb)
    payload = {f"in_{k}": v for k, v in scene_arrays(sc).items()}
    payload.update(camera=cam, grad_rgb=grad_rgb, out_rgb=out, visible_counter=counter,
                   provenance=np.array(provenance()))
    payload.update({f"grad_{k}": v for k, v in grads.items()})
    np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **payload)


def with_sh(sc: scenes.Scene, degree: int, seed: int) -> scenes.Scene:
    rng = np.random.default_rng(seed)
    sc.sh_degree = degree
    sc.sh1 = (0.2 * rng.standard_normal((sc.count, 3, 3))).astype(np.float32) if degree >= 1 else None
    sc.sh2 = (0.2 * rng.standard_normal((sc.count, 5, 3))).astype(np.float32) if degree >= 2 else None
    sc.sh3 = (0.2 * rng.standard_normal((sc.count, 7, 3))).astype(np.float32) if degree >= 3 else None
    return sc


def one(mean, rot, ls, sh0, op, sh1=None) -> scenes.Scene:
    f = lambda v, shape: np.asarray(v, np.float32).reshape(shape)  # noqa: E731
    sc = scenes.Scene(f(mean, (1, 3)), f(rot, (1, 4)), f(ls, (1, 3)), f([op], (1,)), f(sh0, (1, 3)))
    if sh1 is not None:
        sc.sh_degree = 1
        sc.sh1 = f(sh1, (1, 3, 3))
    return sc


def cam_block(w, h, fx, fy, cx, cy, bg, near=0.1, far=10.0) -> np.ndarray:
    # identity pose (rot xyzw = 0,0,0,1; transl 0)
    return np.array([fx, fy, cx, cy, w, h, 0, 0, 0, 1, 0, 0, 0, near, far, *bg], np.float32)


def fd_scenes():
    """The scenes of tests/render_runtime.cpp:249-467 (inputs and upstream gradients as there)."""
    gradient = one([0.2, -0.1, 3.5], [0.1, -0.05, 0.02, 0.99], [-0.2, 0.1, -0.05], [0.1, -0.2, 0.3], 0.4,
                   sh1=[0.05, -0.02, 0.01, -0.03, 0.04, -0.05, 0.02, 0.01, -0.04])
    g_gradient = np.array([0.3, -0.1, 0.2, 0.05, -0.2, 0.4, -0.3, 0.1, 0.25, -0.15, 0.35, -0.05],
                          np.float32).reshape(3, 2, 2)
    saturation = one([0.0, 0.0, 2.0], [0, 0, 0, 1], [0, 0, 0], [1.2, -0.3, 0.5], 5.3)
    g_saturation = np.array([0.7, -0.4, 0.2], np.float32).reshape(3, 1, 1)
    aniso = one([0.35, 0.1, 3.6], [0, 0, 0.1305262, 0.9914449], [-0.2, -0.6, -0.4], [0.1, 0.4, 0.9], -0.1)
    g_aniso = np.array([((i % 19) - 9) * np.float32(0.07) for i in range(3 * 64)], np.float32).reshape(3, 8, 8)
    culling = one([0.0, 0.0, 3.5], [0, 0, 0.1305262, 0.9914449], [-1.8, -2.0, -1.9], [0.1, 0.4, 0.9], -0.1)
    g_culling = np.array([((i % 29) - 14) * np.float32(0.03) for i in range(3 * 64 * 64)],
                         np.float32).reshape(3, 64, 64)
    bg = (0.05, 0.1, 0.2)
    return {
        "fd_gradient": (gradient, cam_block(2, 2, 3.0, 2.5, 0.8, 1.1, bg), g_gradient),
        "fd_alpha_saturation": (saturation, cam_block(1, 1, 1.0, 1.0, 0.5, 0.5, bg), g_saturation),
        "fd_rotated_anisotropic": (aniso, cam_block(8, 8, 12.0, 11.0, 4.0, 4.0, bg), g_aniso),
        "fd_hard_culling": (culling, cam_block(64, 64, 50.0, 66.6666718, 32.0, 32.0, (0.02, 0.02, 0.03)),
                            g_culling),
    }


def adc_case(ref: Reference, name: str, algorithm: int, step: int, max_num: int, n: int, seed: int) -> None:
    sc = scenes.cube_scene(seed, n)
    rng = np.random.default_rng(seed)
    aux = {"grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
           "absgrad_acc": (rng.random(n) * 4e-3).astype(np.float32),
           "visible_counter": rng.integers(0, 4, n).astype(np.float32)}
    fields = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
              "sh0": sc.sh0}
    params = dict(algorithm=algorithm, pruning_opacity_threshold=0.1, opacity_clamp_value=0.3, max_world_scale=0.05,
                  duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01, duplicate_absgrad_threshold=4e-4,
                  scene_scale=1.0, refine_every=100, start_refine=0, end_refine=1000, max_num_gaussians=max_num,
                  reset_every=300, global_step=step, seed=77)
    out, counts = ref.adc({k: v.copy() for k, v in fields.items()}, aux, AdcParams(**params), max_num)
    payload = {f"in_{k}": v for k, v in fields.items()}
    payload.update({f"aux_{k}": v for k, v in aux.items()})
    payload.update({f"out_{k}": v for k, v in out.items()})
    payload.update({f"param_{k}": np.array(v) for k, v in params.items()})
    payload.update(counts=counts, provenance=np.array(provenance()))
    np.savez_compressed(os.path.join(OUT, f"{name}.npz"), **payload)


def main() -> None:
    if not Reference.available():
        raise SystemExit("oracle/_ref/libgsxref.so is missing: run `make -C oracle ref` here first")
    ref = Reference()
    rng = np.random.default_rng(2024)

    w = scenes.config0(n=1500, width=64, height=48)
    render_case(ref, "render_c0", w.scene, w.camera, rng.standard_normal((3, 48, 64)).astype(np.float32))
    w = scenes.config1(n=800, width=80, height=48)
    cam = w.camera.copy()
    cam[15:18] = (0.2, 0.1, 0.05)
    render_case(ref, "render_c1_sh3", with_sh(w.scene, 3, 5), cam,
                rng.standard_normal((3, 48, 80)).astype(np.float32))
    w = scenes.config3(n=2000, width=96, height=54)
    render_case(ref, "render_c3", w.scene, w.camera, rng.standard_normal((3, 54, 96)).astype(np.float32))
    w = scenes.config2(n=1000, size=64)
    render_case(ref, "render_c2_sh1", with_sh(w.scene, 1, 6), w.camera,
                rng.standard_normal((3, 64, 64)).astype(np.float32))
    for name, (sc, cam, g) in fd_scenes().items():
        render_case(ref, name, sc, cam, g)

    p = rng.random((3, 24, 40), dtype=np.float32)
    t = rng.random((3, 24, 40), dtype=np.float32)
    payload = {"pred": p, "target": t, "scale": np.float32(0.3), "provenance": np.array(provenance())}
    for alg in ("l1", "mse", "ssim"):
        m0 = rng.random(p.shape, dtype=np.float32)
        g0 = rng.random(p.shape, dtype=np.float32)
        m, g = m0.copy(), g0.copy()
        ref.loss(alg, p, t, 0.3, m, g)
        payload.update({f"{alg}_map_in": m0, f"{alg}_grad_in": g0, f"{alg}_map": m, f"{alg}_grad": g})
    np.savez_compressed(os.path.join(OUT, "loss.npz"), **payload)

    p0 = rng.standard_normal(1000).astype(np.float32)
    g = (0.1 * rng.standard_normal(1000)).astype(np.float32)
    hyper = np.array([1e-2, 0.9, 0.999, 0.01, 1e-8, 0.05], np.float32)
    p1 = p0.copy()
    ref.adam(p1, g, hyper, 5)
    np.savez_compressed(os.path.join(OUT, "adam.npz"), param=p0, grad=g, hyper=hyper, steps=np.int32(5),
                        param_after=p1, provenance=np.array(provenance()))

    adc_case(ref, "adc_default", 0, 100, 2600, 1500, 41)
    adc_case(ref, "adc_absgs_reset", 1, 600, 2000, 1500, 42)
    print("wrote", sorted(f for f in os.listdir(OUT) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
