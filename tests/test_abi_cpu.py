"""The C-ABI library loads without a device and exports every function include/gsx_hip.h declares,
with the Python binding table covering the same set (no compute calls: no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "gsx_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(gsx_hip_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    names = _declared()
    assert "gsx_hip_render_forward" in names and "gsx_hip_adc_step" in names
    assert len(names) >= 30


def test_library_exports_every_declared_symbol():
    from gsx_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libgsx_hip.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    from gsx_amd import _lib
    assert set(_lib.SIGNATURES) == _declared()
    lib = _lib.load(require_device=False)
    for name in _lib.SIGNATURES:
        assert getattr(lib, name).argtypes is not None


def test_missing_device_fails_loudly():
    """No CPU fallback: asking for a device where there is none raises."""
    import torch
    from gsx_amd import _lib
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    with pytest.raises(_lib.GsxHipError):
        _lib.load(require_device=True)


def test_struct_sizes_match_header_layout():
    """ctypes mirrors of the ABI structs have the C sizes (natural alignment, LP64)."""
    from gsx_amd import _lib
    assert ctypes.sizeof(_lib.Camera) == 4 * 18
    assert ctypes.sizeof(_lib.Gaussians) == 8 + 8 + 8 * 8
    assert ctypes.sizeof(_lib.AdamGroup) == 4 * 8 + 8 + 6 * 4 + 2 * 8
    assert ctypes.sizeof(_lib.AdcParams) == 4 * 9 + 4 + 5 * 8 + 3 * 4 + 4
    assert ctypes.sizeof(_lib.GsRows) == 8 + 8 + 12 * 8 + 16 * 8
    assert ctypes.sizeof(_lib.RenderStats) == 3 * 8 + 6 * 4


PLUGIN_PATH = os.path.join(ROOT, "gsx_amd", "libgsx_hip_backend.so")


def test_backend_plugin_exports_the_bootstrap():
    """The gsx backend plugin links libgsx_hip.so and exports the provider bootstrap gsx's
    registry calls (gsx-backend.c:225-235)."""
    if not os.path.exists(PLUGIN_PATH):
        pytest.skip("the plugin is built only where gsx's headers are present")
    from oracle.oracle import Reference
    if not Reference.available(hip=True):
        pytest.skip("oracle/_ref/libgsxref_hip.so was not built")
    # the plugin's gsx symbols resolve against the core it is linked into
    lib = ctypes.CDLL(Reference.hip_path)
    assert hasattr(lib, "gsx_hip_backend_provider_bootstrap")


def test_core_with_plugin_runs_cpu_backend_without_device():
    """Without a device the HIP provider reports NOT_SUPPORTED, the registry keeps the CPU
    backend, and selecting the GPU slot fails with an error (no fallback)."""
    import numpy as np
    import torch
    from oracle.oracle import Reference
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    if not Reference.available(hip=True):
        pytest.skip("oracle/_ref/libgsxref_hip.so was not built")
    cpu = Reference(backend="cpu")
    assert cpu.device_name() == "cpu0"
    assert np.array_equal(cpu.reduce("sum", np.ones((2, 5), np.float32), 1), [5.0, 5.0])
    with pytest.raises(RuntimeError):
        Reference(backend="hip").device_name()
