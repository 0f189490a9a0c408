"""GPU parity of adaptive density control and the row gather against the CPU oracle
(restatement of gsx/src/gsx-cpu/adc/default.c and adc.c, itself checked bit-exact against the
reference CPU backend in test_oracle_cpu.py).

Counts, the surviving row order and every row are compared bit-exact, split rows included: the
split offsets come from Box-Muller normals whose logf / cosf are the glibc-exact restatements of
gsx_math.h (checked against the host libm in test_oracle_cpu.py), so they equal the oracle's
glibc results bit for bit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _scene(n, seed):
    from gsx_amd import scenes
    sc = scenes.cube_scene(seed, n)
    rng = np.random.default_rng(seed)
    fields = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
              "sh0": sc.sh0}
    aux = {"grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
           "absgrad_acc": (rng.random(n) * 4e-3).astype(np.float32),
           "visible_counter": rng.integers(0, 4, n).astype(np.float32)}
    moments = {k: ((rng.standard_normal(v.shape) * 1e-3).astype(np.float32),
                   (rng.random(v.shape) * 1e-6).astype(np.float32)) for k, v in fields.items()}
    return fields, aux, moments


CASES = [  # algorithm, global_step, max_num, n
    (0, 100, 5000, 2000),
    (1, 200, 5000, 2000),
    (0, 100, 2100, 2000),   # budget smaller than the candidate count
    (1, 600, 3000, 2000),   # refine + reset window, prune_large active
    (0, 300, 1500, 2000),   # no growth budget; reset only (step % 300 == 0, < end)
    (1, 100, 400_000, 300_000),
]


@pytest.mark.parametrize("algorithm,step,max_num,n", CASES)
def test_adc_step_matches_oracle(oracle, algorithm, step, max_num, n):
    from gsx_amd.backend import DensityControl
    from oracle.oracle import AdcParams
    fields, aux, moments = _scene(n, 31 + algorithm + step)
    params = dict(algorithm=algorithm, pruning_opacity_threshold=0.1, opacity_clamp_value=0.3, max_world_scale=0.05,
                  duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01, duplicate_absgrad_threshold=4e-4,
                  scene_scale=1.0, refine_every=100, start_refine=0, end_refine=1000, max_num_gaussians=max_num,
                  reset_every=300)
    print(f"[case] adc alg={algorithm} step={step} max={max_num} n={n}", flush=True)
    cap = max(n, max_num)

    def dev(arr, width):
        t = torch.zeros((cap, width) if width > 1 else (cap,), dtype=torch.float32, device="cuda")
        t[:n] = torch.from_numpy(arr.reshape(n, width) if width > 1 else arr)
        return t

    widths = {"mean3d": 3, "rotation": 4, "logscale": 3, "opacity": 1, "sh0": 3}
    d_fields = {k: dev(v, widths[k]) for k, v in fields.items()}
    d_fields.update({k: dev(v, 1) for k, v in aux.items()})
    d_moms = {k: (dev(m, widths[k]), dev(v, widths[k])) for k, (m, v) in moments.items()}
    o_fields = {k: torch.zeros_like(v) for k, v in d_fields.items()}
    o_moms = {k: (torch.zeros_like(a), torch.zeros_like(b)) for k, (a, b) in d_moms.items()}
    adc = DensityControl(params, seed=77)
    count, in_out, counts = adc.step(step, n, 0, d_fields, d_moms, cap, o_fields, o_moms)
    torch.cuda.synchronize()
    res_f = o_fields if in_out else d_fields
    res_m = o_moms if in_out else d_moms

    op = AdcParams(algorithm=algorithm, pruning_opacity_threshold=0.1, opacity_clamp_value=0.3,
                   max_world_scale=0.05, duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01,
                   duplicate_absgrad_threshold=4e-4, scene_scale=1.0, refine_every=100, start_refine=0,
                   end_refine=1000, max_num_gaussians=max_num, reset_every=300, global_step=step, seed=77)
    ref_f, ref_m, ref_counts = oracle.adc_step({k: v.copy() for k, v in fields.items()}, moments,
                                               {k: v.copy() for k, v in aux.items()}, op, cap)
    assert count == ref_f["mean3d"].shape[0]
    assert list(counts) == list(ref_counts)
    for k in ("rotation", "sh0", "mean3d", "logscale", "opacity"):
        assert np.array_equal(res_f[k][:count].cpu().numpy().reshape(ref_f[k].shape), ref_f[k]), k
    for k in ref_m:
        for j in (0, 1):
            got = res_m[k][j][:count].cpu().numpy().reshape(ref_m[k][j].shape)
            assert np.array_equal(got, ref_m[k][j]), (k, j)
    for k in ("grad_acc", "absgrad_acc", "visible_counter"):
        if counts[0] or counts[1] or counts[2] or step % 100 == 0:
            assert float(res_f[k][:count].abs().max()) == 0.0


def test_adc_rng_persists_across_steps(oracle):
    """Two refines in a row on one context: the second step's splits draw where the first
    stopped (12 draws per split), like the CPU adc object's stream (gsx-cpu/adc.c:466)."""
    from gsx_amd.backend import DensityControl
    from oracle.oracle import AdcParams
    n0, cap = 1000, 10_000
    fields, aux, _ = _scene(n0, 5)
    params = dict(algorithm=1, pruning_opacity_threshold=0.0, opacity_clamp_value=0.3, max_world_scale=0.0,
                  duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.001, duplicate_absgrad_threshold=4e-4,
                  scene_scale=1.0, refine_every=100, start_refine=0, end_refine=1000, max_num_gaussians=cap,
                  reset_every=0)
    widths = {"mean3d": 3, "rotation": 4, "logscale": 3, "opacity": 1, "sh0": 3}
    adc = DensityControl(params, seed=9)

    def dev(arr, width, n):
        t = torch.zeros((cap, width) if width > 1 else (cap,), dtype=torch.float32, device="cuda")
        t[:n] = torch.from_numpy(arr.reshape(n, width) if width > 1 else arr)
        return t

    d = {k: dev(v, widths[k], n0) for k, v in fields.items()}
    d.update({k: dev(v, 1, n0) for k, v in aux.items()})
    o = {k: torch.zeros_like(v) for k, v in d.items()}
    n1, in_out, c1 = adc.step(100, n0, 0, d, None, cap, o, None)
    cur = o if in_out else d
    other = d if in_out else o
    torch.cuda.synchronize()
    step1 = {k: cur[k][:n1].cpu().numpy().reshape((n1, widths[k]) if widths[k] > 1 else (n1,)).copy()
             for k in widths}
    aux2 = {"grad_acc": np.full(n1, 1.0, np.float32), "absgrad_acc": np.full(n1, 1.0, np.float32),
            "visible_counter": np.full(n1, 1.0, np.float32)}
    for k, v in aux2.items():
        cur[k][:n1] = torch.from_numpy(v).cuda()
    n2, in_out2, c2 = adc.step(200, n1, 0, cur, None, cap, other, None)
    torch.cuda.synchronize()
    assert c1[2] > 0 and c2[2] > 0
    res = other if in_out2 else cur
    op = AdcParams(**params, global_step=100, seed=9)
    f1, _, k1 = oracle.adc_step({k: v.copy() for k, v in fields.items()}, None,
                                {k: v.copy() for k, v in aux.items()}, op, cap)
    assert n1 == f1["mean3d"].shape[0] and list(c1) == list(k1)
    op2 = AdcParams(**params, global_step=200, seed=9, rng_draws_consumed=12 * int(c1[2]))
    f2, _, k2 = oracle.adc_step(step1, None, aux2, op2, cap)
    assert n2 == f2["mean3d"].shape[0] and list(c2) == list(k2)
    for k in widths:
        got = res[k][:n2].cpu().numpy().reshape(f2[k].shape)
        assert np.array_equal(got, f2[k]), k


def test_gather_rows(oracle):
    import ctypes
    from gsx_amd import _lib
    from gsx_amd.backend import ptr
    lib = _lib.load()
    rng = np.random.default_rng(3)
    for row_bytes_f, rows in ((3, 1000), (4, 777), (21, 50)):
        src = rng.standard_normal((rows, row_bytes_f)).astype(np.float32)
        idx = rng.integers(0, rows, 2 * rows).astype(np.int32)
        s = torch.from_numpy(src).cuda()
        i = torch.from_numpy(idx).cuda()
        d = torch.empty((len(idx), row_bytes_f), dtype=torch.float32, device="cuda")
        flag = torch.zeros(1, dtype=torch.int32, device="cuda")
        _lib.check(lib.gsx_hip_gather_rows_kernel_launch(ptr(s), ptr(d), row_bytes_f * 4, len(idx), ptr(i), rows,
                                                         ptr(flag), None))
        torch.cuda.synchronize()
        assert np.array_equal(d.cpu().numpy(), oracle.gather_rows(src, idx))
        assert int(flag.item()) == 0
    # out-of-range index raises the flag (the CPU returns GSX_ERROR_OUT_OF_RANGE)
    bad = torch.tensor([0, 5000], dtype=torch.int32, device="cuda")
    d = torch.empty((2, 4), dtype=torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.zeros((10, 4), dtype=torch.float32, device="cuda")
    _lib.check(lib.gsx_hip_gather_rows_kernel_launch(ptr(s), ptr(d), 16, 2, ptr(bad), 10, ptr(flag), None))
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
