"""gsx_hip_scan_exclusive_u32_noalloc (partial sums in the library's static device array) against
gsx_hip_scan_exclusive_u32 (partial sums in a caller workspace): bit-identical outputs on two
calls in a row, the second smaller than the first, so stale partials of the first call would
show; and sizes past the static array are rejected before anything runs."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

MAX_ELEMENTS = 65536 * 1024


def _scan_both(lib, x):
    from gsx_amd import _lib
    n = len(x)
    xi = torch.from_numpy(x.view(np.int32).copy()).cuda() if n else torch.empty(1, dtype=torch.int32, device="cuda")
    ref = torch.full((n + 1,), -1, dtype=torch.int32, device="cuda")
    got = torch.full((n + 1,), -2, dtype=torch.int32, device="cuda")
    temp = torch.empty(lib.gsx_hip_scan_temp_bytes(n), dtype=torch.uint8, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.gsx_hip_scan_exclusive_u32(xi.data_ptr(), ref.data_ptr(), n, temp.data_ptr(), s), "scan")
    _lib.check(lib.gsx_hip_scan_exclusive_u32_noalloc(xi.data_ptr(), got.data_ptr(), n, s), "scan noalloc")
    torch.cuda.synchronize()
    return ref.cpu().numpy().view(np.uint32), got.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("sizes", [(3_000_001, 70_000), (MAX_ELEMENTS, 5), (4097, 0)])
def test_noalloc_scan_matches_workspace_scan(sizes):
    from gsx_amd import _lib
    lib = _lib.load()
    for k, n in enumerate(sizes):
        print(f"[case] noalloc scan call {k} n={n}", flush=True)
        x = np.random.default_rng(n + k).integers(0, 7, size=n, dtype=np.uint32)
        ref, got = _scan_both(lib, x)
        assert np.array_equal(got, ref)
        expect = np.concatenate([[0], np.cumsum(x, dtype=np.uint64)]).astype(np.uint32)
        assert np.array_equal(got, expect)


def test_noalloc_scan_rejects_sizes_past_the_scratch():
    from gsx_amd import _lib
    lib = _lib.load()
    x = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # checked on the host before any launch, so the undersized buffers are never touched
    rc = lib.gsx_hip_scan_exclusive_u32_noalloc(x.data_ptr(), out.data_ptr(), MAX_ELEMENTS + 1, s)
    assert rc == _lib.ERROR_OUT_OF_RANGE
    assert b"static scratch" in lib.gsx_hip_last_error_message()
    torch.cuda.synchronize()
