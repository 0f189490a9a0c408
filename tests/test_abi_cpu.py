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
    assert ctypes.sizeof(_lib.AdcParams) == 4 * 9 + 4 + 5 * 8
    assert ctypes.sizeof(_lib.GsRows) == 8 + 8 + 12 * 8 + 16 * 8
    assert ctypes.sizeof(_lib.RenderStats) == 3 * 8 + 6 * 4
