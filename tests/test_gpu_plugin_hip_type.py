"""The HIP backend as a gsx backend type of its own (GSX_BACKEND_TYPE_HIP), not a tenant of the
CUDA slot: oracle/_ref/libgsxref_hiptype.so is the unmodified reference core with the two
registry additions of oracle/hip_backend_type.sed (the type check of gsx-backend.c:184-194
and the HIP bootstrap call beside gsx-backend.c:225-235) and the plugin built with
-DGSX_HIP_BACKEND_TYPE=GSX_BACKEND_TYPE_HIP. The registry then lists the MI355X under its own
type, the CUDA slot stays empty, and gsx's public API renders on it as on the CPU backend of
the same process: images and visibility counters bit-identical, gradients within 1e-3
relative L2, a few image-fit steps within 1e-3 of the CPU backend's parameter updates.
"""
import numpy as np
import pytest

from gsx_amd import scenes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def typed():
    from oracle.oracle import Reference
    if not Reference.available(hip_type=True):
        pytest.skip("oracle/_ref/libgsxref_hiptype.so was not built (needs the reference tree at build time)")
    return Reference(backend="cpu", hip_type=True), Reference(backend="hip", hip_type=True)


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_registry_lists_a_hip_type_device(typed):
    cpu, hip = typed
    print("[case] hip-type registry", flush=True)
    assert cpu.count_devices("hip") >= 1
    assert cpu.count_devices("cuda") == 0
    assert cpu.count_devices("cpu") == 1
    assert hip.backend_type() == (3, "hip")
    assert cpu.backend_type() == (0, "cpu")
    assert hip.device_name()


def test_hip_type_renders_like_the_cpu_backend(typed):
    cpu, hip = typed
    w = scenes.config1(n=20000, width=160, height=120)
    sc = w.scene
    cam = w.camera.copy()
    cam[15:18] = (0.2, 0.1, 0.05)
    print(f"[case] hip-type render n={sc.count}", flush=True)
    assert np.array_equal(hip.render(sc, cam), cpu.render(sc, cam))
    ca = np.full(sc.count, 1.0, np.float32)
    cb = ca.copy()
    assert np.array_equal(hip.render(sc, cam, train=True, visible_counter=cb),
                          cpu.render(sc, cam, train=True, visible_counter=ca))
    assert np.array_equal(cb, ca)
    grad_rgb = np.random.default_rng(7).standard_normal((3, 120, 160)).astype(np.float32)
    img_c, g_c = cpu.render_grad(sc, cam, grad_rgb)
    img_h, g_h = hip.render_grad(sc, cam, grad_rgb)
    assert np.array_equal(img_h, img_c)
    for k in g_c:
        assert _rel(g_h[k], g_c[k]) <= 1e-3, k


def test_hip_type_train_steps(typed):
    cpu, hip = typed
    w = scenes.config2(n=20000, size=128)
    print("[case] hip-type image-fit steps", flush=True)
    sc_c, _ = cpu.train_steps(w.scene, w.camera, w.target, 3)
    sc_h, _ = hip.train_steps(w.scene, w.camera, w.target, 3)
    for k in ("mean3d", "rotation", "logscale", "opacity", "sh0"):
        d_c = getattr(sc_c, k).astype(np.float64) - getattr(w.scene, k)
        d_h = getattr(sc_h, k).astype(np.float64) - getattr(w.scene, k)
        assert _rel(d_h, d_c) <= 1e-3, k
