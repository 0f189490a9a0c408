"""Parity at the stated sizes of BASELINE.json's GPU configurations.

C1: 500k Gaussians, 1280x720, TRAIN forward + L1 + backward: image and L1 gradient bit-exact,
    the five parameter gradients within 1e-3 relative L2 of the CPU oracle.
C2: 1M Gaussians, 1024^2 image fit: forward bit-exact; the first step's gradients against the
    oracle; 1000 steps of 0.8 L1 + 0.2 (1 - SSIM) + Adam (lr mean3d 1e-3, others 1e-2) on the
    GPU: the loss falls, the parameters stay finite, and the last parameters render bit-exactly
    like the oracle renders them.
C3: 3M Gaussians, 1920x1080: sorted keys, values and tile ranges bit-exact, image bit-exact,
    gradients within 1e-3 relative L2.
C4: 6M Gaussians, 1920x1080 (about 335M tile instances after the tile test): keys, values,
    ranges and image bit-exact; TRAIN forward + backward deterministic, gradients within 1e-3
    relative L2 of the oracle's tiled backward; one full-size ABSGS density-control step with
    counts and rows equal to the oracle's.

The oracle's tiled paths (oracle_tiled: per-tile lists walked per pixel on all host cores) give
the same pixels and keys as its serial restatement bit for bit, and its tiled backward the
serial backward's gradients up to the CPU's float summation order (within 1e-4 relative L2);
tests/test_oracle_cpu.py checks both on scenes the serial functions finish. C1-C3 gradients are
checked against the serial backward, C4's against the tiled one.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GRAD_TOL = 1e-3


def _rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _setup(workload):
    from gsx_amd.backend import Camera, GaussianTensors, Renderer
    cam = Camera.from_block(workload.camera)
    g = GaussianTensors.from_scene(workload.scene)
    return Renderer(cam.width, cam.height), cam, g


def _dtoh(lib, src, count, dtype):
    out = np.empty(count, dtype)
    if count:
        from gsx_amd import _lib
        _lib.check(lib.gsx_hip_memcpy_dtoh(out.ctypes.data_as(ctypes.c_void_p), src, out.nbytes), "dtoh")
    return out


def _check_keys_and_ranges(r, scene_count, keys_ref, vals_ref, oracle):
    """Sorted keys, values (emission positions mapped to Gaussians) and ranges against the
    oracle's tile keys (tile << 32 | bits(depth), value = Gaussian index)."""
    st = r.stats()
    assert st.instance_count == len(keys_ref)
    buf = r.buffers()
    n_inst = st.instance_count
    assert st.sorted_tile_bytes == 4
    tile = _dtoh(r.lib, buf.sorted_tiles, n_inst, np.uint32)
    vals = _dtoh(r.lib, buf.sorted_values, n_inst, np.uint32)
    inst_g = _dtoh(r.lib, buf.instance_gaussian, n_inst, np.uint32)
    ranges = _dtoh(r.lib, buf.tile_ranges, 2 * st.tile_count, np.uint32).reshape(st.tile_count, 2)
    g_sorted = inst_g[vals]
    # stable: within a tile the emission positions ascend
    assert np.all((tile[1:] != tile[:-1]) | (vals[1:] > vals[:-1]))
    del vals
    assert np.array_equal(g_sorted, vals_ref)
    depth_of = np.zeros(scene_count, np.uint64)
    depth_of[vals_ref] = keys_ref & np.uint64(0xFFFFFFFF)
    assert np.array_equal((tile.astype(np.uint64) << np.uint64(32)) | depth_of[g_sorted], keys_ref)
    del g_sorted
    assert np.all(tile[1:] >= tile[:-1])
    del tile
    # emission order: one contiguous run per Gaussian, runs in (depth, index) order
    starts = np.flatnonzero(np.r_[True, inst_g[1:] != inst_g[:-1]])
    run_g = inst_g[starts].astype(np.int64)
    del inst_g, starts
    assert len(np.unique(run_g)) == len(run_g)
    order = np.lexsort((run_g, depth_of[run_g]))
    assert np.array_equal(order, np.arange(len(run_g)))
    assert np.array_equal(ranges, oracle.tile_ranges(keys_ref, st.tile_count))
    nonempty = ranges[ranges[:, 1] > ranges[:, 0]]
    assert int((nonempty[:, 1].astype(np.int64) - nonempty[:, 0]).sum()) == n_inst
    return st


def _grads_vs_oracle(oracle, w, grad_rgb_np, grads):
    ref = oracle.render_backward(w.scene, w.camera, grad_rgb_np)
    errs = {}
    for field in ("mean3d", "rotation", "logscale", "opacity", "sh0"):
        errs[field] = _rel_l2(getattr(grads, field).cpu().numpy(), ref[field])
    print(f"[grads] {errs}", flush=True)
    for field, err in errs.items():
        assert err <= GRAD_TOL, f"{field}: relative L2 {err:.3e}"


@pytest.mark.timeout(600)
def test_c1_full_train_step(oracle):
    from gsx_amd import scenes
    from gsx_amd.backend import Loss
    w = scenes.config1()
    print(f"[case] C1 full n={w.scene.count} 1280x720", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=True)
    target = torch.from_numpy(w.target).cuda()
    loss_map = torch.zeros_like(img)
    grad = torch.zeros_like(img)
    l1 = Loss("l1")
    l1.forward(img, target, loss_map, 1.0)
    l1.backward(grad, 1.0)
    grads = g.zeros_like_grads()
    for t in (grads.mean3d, grads.rotation, grads.logscale, grads.opacity, grads.sh0):
        t.fill_(123.0)
    r.backward(grad, grads)
    torch.cuda.synchronize()
    ref_img, _ = oracle.render_tiled(w.scene, w.camera, cull=False)
    got = img.cpu().numpy()
    assert np.array_equal(got, ref_img), f"max abs {np.abs(got - ref_img).max()}"
    ref_map = np.zeros_like(ref_img)
    ref_grad = np.zeros_like(ref_img)
    oracle.loss("l1", ref_img, w.target, 1.0, ref_map, ref_grad)
    assert np.array_equal(loss_map.cpu().numpy(), ref_map)
    assert np.array_equal(grad.cpu().numpy(), ref_grad)
    _grads_vs_oracle(oracle, w, ref_grad, grads)


def _gs_scene(g):
    from gsx_amd import scenes
    return scenes.Scene(*(t.detach().cpu().numpy().copy() for t in (g.mean3d, g.rotation, g.logscale, g.opacity,
                                                                     g.sh0)))


@pytest.mark.timeout(600)
def test_c2_full_image_fit(oracle):
    from gsx_amd import scenes
    from gsx_amd.backend import Adam, Loss
    w = scenes.config2()
    print(f"[case] C2 full n={w.scene.count} 1024x1024, 1000 steps", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=False)
    torch.cuda.synchronize()
    ref_img, _ = oracle.render_tiled(w.scene, w.camera, cull=False)
    assert np.array_equal(img.cpu().numpy(), ref_img)

    target = torch.from_numpy(w.target).cuda()
    grads = g.zeros_like_grads()
    l1, ssim = Loss("l1"), Loss("ssim")
    opt = Adam([dict(parameter=g.mean3d, gradient=grads.mean3d, learning_rate=1e-3),
                dict(parameter=g.rotation, gradient=grads.rotation, learning_rate=1e-2),
                dict(parameter=g.logscale, gradient=grads.logscale, learning_rate=1e-2),
                dict(parameter=g.opacity, gradient=grads.opacity, learning_rate=1e-2),
                dict(parameter=g.sh0, gradient=grads.sh0, learning_rate=1e-2)])
    loss_map = torch.empty_like(img)
    grad = torch.empty_like(img)
    losses = []
    for step in range(1000):
        img = r.render(cam, g, train=True, out_rgb=img)
        loss_map.zero_()
        grad.zero_()
        l1.forward(img, target, loss_map, 0.8)
        ssim.forward(img, target, loss_map, 0.2)
        l1.backward(grad, 0.8)
        ssim.backward(grad, 0.2)
        r.backward(grad, grads)
        if step == 0:
            torch.cuda.synchronize()
            # first step: the image is the oracle's (checked above); the fused 0.8 L1 + 0.2 SSIM
            # map and image gradient at the full 1024^2 against the oracle's losses
            got_img = img.cpu().numpy()
            assert np.array_equal(got_img, ref_img)
            ref_map = np.zeros_like(ref_img)
            ref_grad = np.zeros_like(ref_img)
            oracle.loss("l1", ref_img, w.target, 0.8, ref_map, ref_grad)
            oracle.loss("ssim", ref_img, w.target, 0.2, ref_map, ref_grad)
            map_err = float(np.abs(loss_map.cpu().numpy() - ref_map).max())
            grad_err = _rel_l2(grad.cpu().numpy(), ref_grad)
            print(f"[c2] step-0 loss map max-abs {map_err:.2e}, image gradient rel L2 {grad_err:.2e}", flush=True)
            assert map_err <= 1e-5 and grad_err <= GRAD_TOL
            # the render gradients of the oracle's upstream gradient against the oracle
            _grads_vs_oracle(oracle, w, ref_grad, grads)
        opt.step()
        if step % 100 == 0 or step == 999:
            losses.append(float(loss_map.double().mean()))
    torch.cuda.synchronize()
    print(f"[c2] loss every 100 steps: {[round(x, 5) for x in losses]}", flush=True)
    assert losses[-1] < 0.8 * losses[0]
    for name in ("mean3d", "rotation", "logscale", "opacity", "sh0"):
        assert bool(torch.isfinite(getattr(g, name)).all()), name
    final = r.render(cam, g, train=False)
    torch.cuda.synchronize()
    sc = _gs_scene(g)
    ref_final, _ = oracle.render_tiled(sc, w.camera, cull=False)
    assert np.array_equal(final.cpu().numpy(), ref_final)


@pytest.mark.timeout(600)
def test_c3_full_keys_image_gradients(oracle):
    from gsx_amd import scenes
    w = scenes.config3()
    print(f"[case] C3 full n={w.scene.count} 1920x1080 pose 0", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=True)
    torch.cuda.synchronize()
    ref_img, ref_t, keys_ref, vals_ref = oracle.render_and_keys_tiled(w.scene, w.camera)
    assert np.array_equal(img.cpu().numpy(), ref_img)
    st = _check_keys_and_ranges(r, w.scene.count, keys_ref, vals_ref, oracle)
    print(f"[c3] instances {st.instance_count}", flush=True)
    del keys_ref, vals_ref
    rng = np.random.default_rng(11)
    grad_rgb = rng.standard_normal((3, cam.height, cam.width)).astype(np.float32)
    grads = g.zeros_like_grads()
    r.backward(torch.from_numpy(grad_rgb).cuda(), grads)
    torch.cuda.synchronize()
    _grads_vs_oracle(oracle, w, grad_rgb, grads)


@pytest.mark.timeout(600)
def test_c3_full_other_poses(oracle):
    from gsx_amd import scenes
    from gsx_amd.backend import Camera
    base = scenes.config3()
    r, _, g = _setup(base)
    for pose in (6, 13):
        w = scenes.config3(pose_index=pose)
        print(f"[case] C3 full pose {pose}", flush=True)
        cam = Camera.from_block(w.camera)
        img = r.render(cam, g, train=False)
        torch.cuda.synchronize()
        ref_img, _ = oracle.render_tiled(base.scene, w.camera, cull=True)
        assert np.array_equal(img.cpu().numpy(), ref_img)


@pytest.mark.timeout(900)
def test_c4_full_keys_ranges_image(oracle):
    from gsx_amd import scenes
    w = scenes.config4()
    print(f"[case] C4 full n={w.scene.count} 1920x1080", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=False)
    torch.cuda.synchronize()
    ref_img, _, keys_ref, vals_ref = oracle.render_and_keys_tiled(w.scene, w.camera)
    print(f"[c4] oracle instances {len(keys_ref)}", flush=True)
    assert np.array_equal(img.cpu().numpy(), ref_img)
    st = _check_keys_and_ranges(r, w.scene.count, keys_ref, vals_ref, oracle)
    print(f"[c4] instances {st.instance_count}, sort passes {st.sort_passes}", flush=True)


@pytest.mark.timeout(600)
def test_c4_full_train_backward_deterministic(oracle):
    """C4 at full size: two TRAIN forward + backward runs are bit-identical, and the five
    gradient fields are within 1e-3 relative L2 of the oracle's tiled backward (the serial
    backward's per-contribution terms, summed per Gaussian in double on all host cores)."""
    from gsx_amd import scenes
    w = scenes.config4()
    print(f"[case] C4 full TRAIN forward + backward n={w.scene.count}", flush=True)
    r, cam, g = _setup(w)
    rng = np.random.default_rng(12)
    grad_rgb = torch.from_numpy(rng.standard_normal((3, cam.height, cam.width)).astype(np.float32)).cuda()
    results = []
    for _ in range(2):
        img = r.render(cam, g, train=True)
        grads = g.zeros_like_grads()
        r.backward(grad_rgb, grads)
        torch.cuda.synchronize()
        results.append((img.cpu().numpy(), {k: getattr(grads, k).cpu().numpy()
                                            for k in ("mean3d", "rotation", "logscale", "opacity", "sh0")}))
    (img_a, ga), (img_b, gb) = results
    assert np.array_equal(img_a, img_b)
    for k in ga:
        assert np.all(np.isfinite(ga[k])), k
        assert np.array_equal(ga[k], gb[k]), k
    assert np.abs(ga["mean3d"]).max() > 0.0
    ref = oracle.render_backward_tiled(w.scene, w.camera, grad_rgb.cpu().numpy())
    errs = {k: _rel_l2(ga[k], ref[k]) for k in ga}
    touched = int((ref["opacity"] != 0).sum())
    print(f"[c4 grads] {errs}, Gaussians with gradients {touched}", flush=True)
    for k, err in errs.items():
        assert err <= GRAD_TOL, f"{k}: relative L2 {err:.3e}"


@pytest.mark.timeout(600)
def test_c4_full_absgs_step(oracle):
    """One ABSGS refine at the full 6M rows (BASELINE config 4 refines every 100 of 500
    iterations), with seeded accumulated absolute gradients and visibility counts."""
    from gsx_amd import scenes
    from gsx_amd.backend import DensityControl
    from oracle.oracle import AdcParams
    w = scenes.config4()
    sc = w.scene
    n = sc.count
    max_num = n + n // 10
    rng = np.random.default_rng(404)
    fields = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
              "sh0": sc.sh0}
    aux = {"grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
           "absgrad_acc": (rng.random(n) * 8e-3).astype(np.float32),
           "visible_counter": rng.integers(0, 20, n).astype(np.float32)}
    params = dict(algorithm=1, pruning_opacity_threshold=0.1, opacity_clamp_value=0.3, max_world_scale=0.5,
                  duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01, duplicate_absgrad_threshold=4e-4,
                  scene_scale=4.0, refine_every=100, start_refine=0, end_refine=500, max_num_gaussians=max_num,
                  reset_every=0)
    print(f"[case] C4 ABSGS step n={n} max={max_num}", flush=True)
    widths = {"mean3d": 3, "rotation": 4, "logscale": 3, "opacity": 1, "sh0": 3}
    cap = max_num

    def dev(arr, width):
        t = torch.zeros((cap, width) if width > 1 else (cap,), dtype=torch.float32, device="cuda")
        t[:n] = torch.from_numpy(arr.reshape(n, width) if width > 1 else arr)
        return t

    d_fields = {k: dev(v, widths[k]) for k, v in fields.items()}
    d_fields.update({k: dev(v, 1) for k, v in aux.items()})
    o_fields = {k: torch.zeros_like(v) for k, v in d_fields.items()}
    adc = DensityControl(params, seed=2024)
    count, in_out, counts = adc.step(100, n, 0, d_fields, None, cap, o_fields, None)
    torch.cuda.synchronize()
    res = o_fields if in_out else d_fields
    op = AdcParams(**params, global_step=100, seed=2024)
    ref_f, _, ref_counts = oracle.adc_step({k: v.copy() for k, v in fields.items()}, None,
                                           {k: v.copy() for k, v in aux.items()}, op, cap)
    print(f"[c4 adc] counts {list(counts)} oracle {list(ref_counts)} final {count}", flush=True)
    assert list(counts) == list(ref_counts)
    assert count == ref_f["mean3d"].shape[0]
    assert counts[2] > 0 and counts[1] > 0 and counts[0] > 0
    for k in ("rotation", "sh0", "mean3d", "logscale", "opacity"):
        assert np.array_equal(res[k][:count].cpu().numpy().reshape(ref_f[k].shape), ref_f[k]), k
