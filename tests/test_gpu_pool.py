"""The stream-ordered device pool of libgsx_hip.so (gsx_hip_pool_*): size-class reuse, stream
ordering of a block reused on another stream, its errors and release, and its purpose: after a
warm-up, density-control refines at 1M rows through the gsx plugin (gsx_adc_step, whose commit
reallocates the whole Gaussian set and the optimizer's moments through gsx_gs_resize,
gsx/src/gsx-core.c:2811-2869) make no further device allocation.
"""
import ctypes
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _stats(lib):
    from gsx_amd import _lib
    s = _lib.PoolStats()
    _lib.check(lib.gsx_hip_pool_get_stats(ctypes.byref(s)), "pool stats")
    return s


def _malloc(lib, nbytes, stream):
    from gsx_amd import _lib
    p = ctypes.c_void_p()
    _lib.check(lib.gsx_hip_pool_malloc(ctypes.byref(p), nbytes, stream), "pool malloc")
    assert p.value
    return p


def test_pool_reuse_ordering_and_release():
    from gsx_amd import _lib
    from gsx_amd.backend import stream_handle
    lib = _lib.load()
    print("[case] pool unit", flush=True)
    st = stream_handle()
    # start from an empty cache (earlier tests' freed blocks would otherwise serve these requests)
    torch.cuda.synchronize()
    _lib.check(lib.gsx_hip_pool_trim(), "pool trim")
    # same size class (1000 and 900 bytes round to 1024): the freed block comes back, no hipMalloc
    p = _malloc(lib, 1000, st)
    a = _stats(lib)
    _lib.check(lib.gsx_hip_pool_free(p, st), "pool free")
    q = _malloc(lib, 900, st)
    b = _stats(lib)
    assert q.value == p.value
    assert b.device_allocations == a.device_allocations and b.reuses == a.reuses + 1
    _lib.check(lib.gsx_hip_pool_free(q, st), "pool free")
    # 8 MiB and 8 MiB - 100 KiB share a class; 16 MiB is two classes past the cache's reach
    mib = 1 << 20
    r = _malloc(lib, 8 * mib, st)
    _lib.check(lib.gsx_hip_pool_free(r, st), "pool free")
    c = _stats(lib)
    r2 = _malloc(lib, 8 * mib - 100 * 1024, st)
    assert r2.value == r.value and _stats(lib).device_allocations == c.device_allocations
    big = _malloc(lib, 16 * mib, st)
    assert _stats(lib).device_allocations == c.device_allocations + 1
    _lib.check(lib.gsx_hip_pool_free(big, st), "pool free")
    # reuse on another stream waits for the freeing stream's queued work: a fill queued on stream A
    # before the free is what stream B reads from the reused block
    side_a, side_b = torch.cuda.Stream(), torch.cuda.Stream()
    sa, sb = stream_handle(side_a), stream_handle(side_b)
    torch.cuda.synchronize()
    pattern = np.array([0x3F800000 + 7], np.uint32)  # one 4-byte pattern
    _lib.check(lib.gsx_hip_fill_pattern(r2, 8 * mib - 100 * 1024, pattern.ctypes.data_as(ctypes.c_void_p), 4, sa),
               "fill on A")
    _lib.check(lib.gsx_hip_pool_free(r2, sa), "free on A")
    r3 = _malloc(lib, 8 * mib - 64 * 1024, sb)
    assert r3.value == r2.value
    host = torch.empty((8 * mib - 100 * 1024) // 4, dtype=torch.int32, pin_memory=True)  # the filled bytes
    _lib.check(lib.gsx_hip_memcpy_async(ctypes.c_void_p(host.data_ptr()), r3, host.numel() * 4, sb), "copy on B")
    _lib.check(lib.gsx_hip_stream_synchronize(sb), "sync B")
    assert np.all(host.numpy().view(np.uint32) == pattern[0])
    _lib.check(lib.gsx_hip_pool_free(r3, sb), "pool free")
    torch.cuda.synchronize()
    # a pointer the pool did not hand out is rejected
    assert lib.gsx_hip_pool_free(ctypes.c_void_p(host.data_ptr()), st) == -1  # GSX_HIP_ERROR_INVALID_ARGUMENT
    # trim releases every cached block of the device
    before = _stats(lib)
    assert before.bytes_cached > 0
    _lib.check(lib.gsx_hip_pool_trim(), "pool trim")
    after = _stats(lib)
    assert after.bytes_cached == 0 and after.device_releases > before.device_releases
    assert after.bytes_in_use == before.bytes_in_use


def test_plugin_refines_reuse_the_pool():
    """Two ABSGS refines of the 1M metric scene through the gsx plugin, each on a fresh Gaussian
    set, Adam optimizer and density-control object (two trainings in one process): the second
    makes no device allocation, and both give the same rows."""
    from gsx_amd import _lib, scenes
    from oracle.oracle import AdcParams, Reference
    if not Reference.available(hip=True):
        pytest.skip("oracle/_ref/libgsxref_hip.so was not built (needs the reference tree at build time)")
    lib = _lib.load()
    hip = Reference(backend="hip")
    sc = scenes.metric_scene().scene
    n = sc.count
    rng = np.random.default_rng(7)
    fields = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
              "sh0": sc.sh0}
    aux = {"grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
           "absgrad_acc": (rng.random(n) * 8e-3).astype(np.float32),
           "visible_counter": rng.integers(0, 20, n).astype(np.float32)}
    cap = n + n // 5
    params = AdcParams(algorithm=1, pruning_opacity_threshold=0.05, opacity_clamp_value=0.3, max_world_scale=0.5,
                       duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01,
                       duplicate_absgrad_threshold=4e-4, scene_scale=4.0, refine_every=100, start_refine=0,
                       end_refine=1000, max_num_gaussians=cap, reset_every=0, global_step=100, seed=3)
    seconds = []
    hook = hip.set_step_hook(lambda k, s: seconds.append(s))
    try:
        print(f"[case] plugin ABSGS refine n={n}, warm-up", flush=True)
        out0, cnt0 = hip.adc(fields, aux, params, cap, optim_probe=True)
        s0 = _stats(lib)
        print("[case] plugin ABSGS refine, second run", flush=True)
        out1, cnt1 = hip.adc(fields, aux, params, cap, optim_probe=True)
        s1 = _stats(lib)
    finally:
        hip.set_step_hook(None)
        del hook
    assert np.array_equal(cnt0, cnt1) and cnt0[1] > 0 and cnt0[0] > 0
    for k in out0:
        assert np.array_equal(out0[k], out1[k]), k
    print(f"[pool] requests {s1.requests - s0.requests}, reuses {s1.reuses - s0.reuses}, "
          f"device allocations {s1.device_allocations - s0.device_allocations}", flush=True)
    assert s1.device_allocations == s0.device_allocations
    assert s1.reuses > s0.reuses
    record = {"workload": "one ABSGS refine of the 1M metric scene (seeded statistics, Adam moments) through the "
                          "gsx plugin (gsx_adc_step, committed by gsx_gs_resize and gsx_optim_resize)",
              "rows_before": n, "rows_after": int(out1["mean3d"].shape[0]),
              "counts_pruned_duplicated_grown_reset": [int(c) for c in cnt1],
              "refine_ms_first_run": round(1000 * seconds[0], 3), "refine_ms_second_run": round(1000 * seconds[1], 3),
              "pool_requests_second_run": int(s1.requests - s0.requests),
              "pool_reuses_second_run": int(s1.reuses - s0.reuses),
              "device_allocations_second_run": int(s1.device_allocations - s0.device_allocations)}
    os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
    with open(os.path.join(ROOT, "gpurun_out", "plugin_refine_1m.json"), "w") as f:
        json.dump(record, f, indent=1)
    print(f"[plugin refine record] {json.dumps(record)}", flush=True)
