"""GPU parity of the render path against the CPU oracle (restatement of gsx/src/gsx-cpu/render.c).

Bars: sorted key/value permutation and tile ranges bit-exact;
rendered image within 1e-4 max-abs (the kernels reproduce the CPU's float operations, so the
test demands bit equality); gradients within 1e-3 relative L2 per parameter field.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GRAD_TOL = 1e-3  # relative L2 per gradient field (north_star)
IMAGE_TOL = 1e-4  # max-abs (north_star); bit equality is asserted where the path is exact


def _setup(workload):
    from gsx_amd.backend import Camera, GaussianTensors, Renderer
    cam = Camera.from_block(workload.camera)
    g = GaussianTensors.from_scene(workload.scene)
    return Renderer(cam.width, cam.height), cam, g


def _rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _workloads():
    from gsx_amd import scenes
    return {
        "c0_small": lambda: scenes.config0(n=20_000, width=160, height=120),
        "c1_small": lambda: scenes.config1(n=30_000, width=200, height=120),
        "c0_full": lambda: scenes.config0(),
        "c2_small": lambda: scenes.config2(n=20_000, size=128),
        "c3_small": lambda: scenes.config3(n=30_000, width=240, height=135),
        "c4_small": lambda: scenes.config4(n=3_000, width=160, height=96),
        # 1080p with few Gaussians: five near-plane boxes cover all 8160 tiles (emitted by a wave
        # each, their instance runs summed in 16 chunks), fifteen runs exceed 32 instances
        "c3_1080": lambda: scenes.config3(n=20_000, width=1920, height=1080),
        # 4096 x 4096: 65536 tiles (16 tile bits, two 8-bit sort passes); near-plane boxes span
        # 256 tile rows, so one box's rows take several steps of the row walks
        "c3_4k": lambda: scenes.config3(n=6_000, width=4096, height=4096),
        # every Gaussian at depth exactly 4 (z = 0 facing the default camera): each tile's list is
        # ordered by Gaussian index alone, which the depth sort must keep through its compaction
        "ties": lambda: scenes.Workload("ties", scenes.plane_scene(5, 3_000, logscale=(-4.0, -3.0), z_sd=0.0),
                                        scenes.camera(160, 120, 200.0)),
    }


@pytest.mark.parametrize("name", ["c0_small", "c1_small", "c0_full", "c2_small", "c3_small", "c4_small", "c3_1080",
                                  "ties"])
def test_forward_image_bit_exact(oracle, name):
    w = _workloads()[name]()
    print(f"[case] forward {name} n={w.scene.count} {int(w.camera[4])}x{int(w.camera[5])}", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=False)
    torch.cuda.synchronize()
    ref, ref_t = oracle.render(w.scene, w.camera)
    got = img.cpu().numpy()
    assert np.abs(got - ref).max() <= IMAGE_TOL
    assert np.array_equal(got, ref), f"max abs {np.abs(got - ref).max()}"
    buf = r.buffers()
    t = torch.empty(cam.width * cam.height, dtype=torch.float32, device="cuda")
    from gsx_amd import _lib
    _lib.check(r.lib.gsx_hip_memcpy_dtod_async(t.data_ptr(), buf.final_transmittance, t.numel() * 4, None), "copy")
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy().reshape(ref_t.shape), ref_t)


def test_nonfinite_colour_stays_non_finite_and_the_rest_bit_exact(oracle):
    """The finite-input precondition of gsx_hip_render_forward: Gaussians with an infinite SH0
    colour make the CPU's pixels that take them infinite; the blend kernels may also turn other
    pixels of the waves that evaluate them into NaN. Every pixel the CPU renders non-finite is
    non-finite here, and every pixel finite here equals the CPU's bit for bit."""
    from gsx_amd import scenes
    w = _workloads()["c0_small"]()
    fields = [np.array(a, copy=True) for a in (w.scene.mean3d, w.scene.rotation, w.scene.logscale, w.scene.opacity,
                                               w.scene.sh0)]
    rng = np.random.default_rng(9)
    hot = rng.choice(w.scene.count, 6, replace=False)
    fields[4][hot] = np.inf
    sc = scenes.Scene(*fields)
    print(f"[case] non-finite colour, Gaussians {hot.tolist()}", flush=True)
    r, cam, g = _setup(scenes.Workload("nonfinite", sc, w.camera))
    img = r.render(cam, g, train=False)
    torch.cuda.synchronize()
    ref, _ = oracle.render(sc, w.camera)
    got = img.cpu().numpy()
    assert (~np.isfinite(ref)).any()  # the case is exercised
    assert np.all(~np.isfinite(got)[~np.isfinite(ref)])
    fin = np.isfinite(got)
    assert np.array_equal(got[fin], ref[fin])
    print(f"[nonfinite] CPU {int((~np.isfinite(ref)).sum())} pixels, HIP {int((~fin).sum())}", flush=True)


def _border_scene(seed, n, fx, width, height):
    """Gaussians whose centres lie around and beyond the screen edges of the default camera
    (at (0, 0, 4) facing the origin), with scales up to radii of about 130 pixels: many boxes
    reach into the screen from outside, and many just miss it."""
    from gsx_amd import scenes
    rng = np.random.default_rng(seed)
    zc = rng.uniform(2.0, 8.0, n)
    sx = rng.uniform(-140.0, width + 140.0, n)
    sy = rng.uniform(-140.0, height + 140.0, n)
    xc = (sx - width / 2) * zc / fx
    yc = (sy - height / 2) * zc / fx
    mean = np.stack([xc, -yc, 4.0 - zc], 1).astype(np.float32)  # camera: y and z flipped
    rot = rng.normal(size=(n, 4)).astype(np.float32)
    ls = rng.uniform(-3.5, 0.3, (n, 3)).astype(np.float32)
    op = rng.uniform(-1.0, 3.0, (n, 1)).astype(np.float32)
    sh0 = rng.normal(0.0, 0.5, (n, 3)).astype(np.float32)
    return scenes.Scene(mean, rot, ls, op, sh0)


def _visible_set_parity(oracle, sc, camera):
    from gsx_amd import scenes
    r, cam, g = _setup(scenes.Workload("border", sc, camera))
    counter = torch.zeros(sc.count, dtype=torch.float32, device="cuda")
    img = r.render(cam, g, train=True, visible_counter=counter)  # only a TRAIN forward counts
    torch.cuda.synchronize()
    ref_counter = np.zeros(sc.count, np.float32)
    ref, _ = oracle.render(sc, camera, visible_counter=ref_counter)
    got = counter.cpu().numpy()
    print(f"[visible] CPU {int(ref_counter.sum())}, HIP {int(got.sum())} of {sc.count}", flush=True)
    assert np.array_equal(got, ref_counter)
    return r, img, ref


def test_visibility_at_the_screen_edges(oracle):
    """Visibility at the screen edges: the visible set, the image and the instance count equal
    the CPU's on a scene of Gaussians around and beyond the edges (centres up to 140 pixels
    outside the screen, radii up to ~130, 1322 of the 1784 visible ones centred off-screen)."""
    from gsx_amd import scenes
    cam_block = scenes.camera(160, 120, 125.0)
    sc = _border_scene(21, 4000, 125.0, 160, 120)
    print("[case] border scene 4000 Gaussians 160x120", flush=True)
    r, img, ref = _visible_set_parity(oracle, sc, cam_block)
    assert np.array_equal(img.cpu().numpy(), ref)
    keys_ref, _ = oracle.tile_keys(sc, cam_block, 16)
    assert r.stats().instance_count == len(keys_ref)


def test_visibility_of_non_finite_shapes(oracle):
    """A non-finite rotation or scale gives the CPU's projection a NaN radius and a box that
    covers the screen (visible) even where the centre lies far outside the screen: the visible
    set equals the CPU's."""
    from gsx_amd import scenes
    cam_block = scenes.camera(160, 120, 125.0)
    sc = _border_scene(22, 600, 125.0, 160, 120)
    rng = np.random.default_rng(23)
    bad = rng.choice(sc.count, 12, replace=False)
    rot, ls = sc.rotation.copy(), sc.logscale.copy()
    rot[bad[:4], 1] = np.nan
    ls[bad[4:8], 2] = np.nan
    ls[bad[8:10], 0] = np.inf
    rot[bad[10:], 3] = np.inf
    sc = scenes.Scene(sc.mean3d, rot, ls, sc.opacity, sc.sh0)
    print(f"[case] non-finite shapes {bad.tolist()}", flush=True)
    _visible_set_parity(oracle, sc, cam_block)


@pytest.mark.parametrize("name", ["c0_small", "c3_small", "c4_small", "c3_1080", "c3_4k", "ties"])
def test_sorted_keys_and_ranges_bit_exact(oracle, name):
    import ctypes
    w = _workloads()[name]()
    print(f"[case] sort {name}", flush=True)
    r, cam, g = _setup(w)
    r.render(cam, g, train=False)
    torch.cuda.synchronize()
    st = r.stats()
    keys_ref, vals_ref = oracle.tile_keys(w.scene, w.camera, 16)
    assert st.instance_count == len(keys_ref)
    buf = r.buffers()
    assert st.sorted_tile_bytes == 4
    tile = np.empty(st.instance_count, np.uint32)
    vals = np.empty(st.instance_count, np.uint32)
    ranges = np.empty((st.tile_count, 2), np.uint32)
    lib = r.lib
    if st.instance_count:
        lib.gsx_hip_memcpy_dtoh(tile.ctypes.data_as(ctypes.c_void_p), buf.sorted_tiles, tile.nbytes)
        lib.gsx_hip_memcpy_dtoh(vals.ctypes.data_as(ctypes.c_void_p), buf.sorted_values, vals.nbytes)
    lib.gsx_hip_memcpy_dtoh(ranges.ctypes.data_as(ctypes.c_void_p), buf.tile_ranges, ranges.nbytes)
    inst_g = np.empty(st.instance_count, np.uint32)
    if st.instance_count:
        lib.gsx_hip_memcpy_dtoh(inst_g.ctypes.data_as(ctypes.c_void_p), buf.instance_gaussian, inst_g.nbytes)
    # sorted tiles with the emission positions as values; the oracle's keys are
    # tile << 32 | bits(depth) with the Gaussian index as value
    assert st.tile_bits == max(int(st.tile_count - 1).bit_length(), 0)
    assert np.array_equal(np.sort(vals), np.arange(st.instance_count, dtype=np.uint32))  # a permutation
    assert np.array_equal(inst_g[vals], vals_ref)  # sorted values are emission positions
    # stable: within a tile the emission positions ascend
    assert np.all((tile[1:] != tile[:-1]) | (vals[1:] > vals[:-1]))
    depth_of = np.zeros(w.scene.count, np.uint64)
    depth_of[vals_ref] = keys_ref & np.uint64(0xFFFFFFFF)
    assert np.array_equal((tile.astype(np.uint64) << np.uint64(32)) | depth_of[inst_g[vals]], keys_ref)
    # emission order: each Gaussian's positions are one contiguous run, runs in (depth, index)
    # order of their Gaussians
    if st.instance_count:
        starts = np.flatnonzero(np.r_[True, inst_g[1:] != inst_g[:-1]])
        run_g = inst_g[starts].astype(np.int64)
        assert len(np.unique(run_g)) == len(run_g)
        order = np.lexsort((run_g, depth_of[run_g]))
        assert np.array_equal(order, np.arange(len(run_g)))
    assert np.array_equal(ranges, oracle.tile_ranges(keys_ref, st.tile_count))
    # invariants: tiles non-decreasing, ranges partition [0, I)
    assert np.all(tile[1:] >= tile[:-1])
    nonempty = ranges[ranges[:, 1] > ranges[:, 0]]
    assert int((nonempty[:, 1] - nonempty[:, 0]).sum()) == st.instance_count


@pytest.mark.parametrize("name", ["c0_small", "c1_small", "c3_small", "c3_1080", "ties"])
def test_backward_gradients(oracle, name):
    w = _workloads()[name]()
    print(f"[case] backward {name}", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=True)
    rng = np.random.default_rng(7)
    grad_rgb = rng.standard_normal((3, cam.height, cam.width)).astype(np.float32)
    grads = g.zeros_like_grads()
    for t in (grads.mean3d, grads.rotation, grads.logscale, grads.opacity, grads.sh0):
        t.fill_(123.0)  # sinks are overwritten, not accumulated
    r.backward(torch.from_numpy(grad_rgb).cuda(), grads)
    torch.cuda.synchronize()
    # the TRAIN forward's image (it also writes the backward's state) equals the oracle's
    assert np.array_equal(img.cpu().numpy(), oracle.render(w.scene, w.camera)[0])
    ref = oracle.render_backward(w.scene, w.camera, grad_rgb)
    for field in ("mean3d", "rotation", "logscale", "opacity", "sh0"):
        err = _rel_l2(getattr(grads, field).cpu().numpy(), ref[field])
        assert err <= GRAD_TOL, f"{field}: relative L2 {err:.3e}"


def _with_sh(scene, degree, seed):
    sc = scene.copy()
    rng = np.random.default_rng(seed)
    sc.sh_degree = degree
    for k, c in ((1, 3), (2, 5), (3, 7)):
        setattr(sc, f"sh{k}", (0.2 * rng.standard_normal((sc.count, c, 3))).astype(np.float32) if degree >= k else None)
    return sc


@pytest.mark.parametrize("degree", [1, 3])
@pytest.mark.parametrize("offset", [0, 1])
def test_backward_overwrites_every_sink(oracle, degree, offset):
    """Every gradient sink, the SH bands' included, starts at 123 and ends as the oracle's gradient.
    The blend backward's workgroups zero the sinks (16-byte stores where a sink is 16-byte aligned,
    offset 0; scalar stores where it is not, offset 1: every sink but the rotation gradient, which
    the ABI requires 16-byte aligned), and the projection backward writes the rows of the Gaussians
    some tile reached. The scene has Gaussians that no tile reaches, whose
    rows only the zeroing sets."""
    from gsx_amd import scenes
    from gsx_amd.backend import GaussianTensors
    base = scenes.config3(n=30_000, width=240, height=135)
    w = scenes.Workload("c3_sh", _with_sh(base.scene, degree, 11), base.camera)
    print(f"[case] sinks degree={degree} offset={offset}", flush=True)
    r, cam, g = _setup(w)
    r.render(cam, g, train=True)
    rng = np.random.default_rng(5)
    grad_rgb = rng.standard_normal((3, cam.height, cam.width)).astype(np.float32)

    def sink(t, off=offset):
        if t is None:
            return None
        buf = torch.full((t.numel() + off,), 123.0, dtype=torch.float32, device="cuda")
        return buf[off:].view(t.shape)

    z = g.zeros_like_grads()
    grads = GaussianTensors(sink(z.mean3d), sink(z.rotation, 0), sink(z.logscale), sink(z.opacity), sink(z.sh0),
                            z.sh_degree, sink(z.sh1), sink(z.sh2), sink(z.sh3))
    r.backward(torch.from_numpy(grad_rgb).cuda(), grads)
    torch.cuda.synchronize()
    ref = oracle.render_backward(w.scene, w.camera, grad_rgb)
    unreached = np.all(ref["mean3d"] == 0.0, axis=1) & (ref["opacity"] == 0.0)
    assert unreached.sum() > 1000, "the scene must hold Gaussians no tile reaches"
    fields = ["mean3d", "rotation", "logscale", "opacity", "sh0"] + [f"sh{k}" for k in range(1, degree + 1)]
    for field in fields:
        got = getattr(grads, field).cpu().numpy()
        assert np.all(got.reshape(g.mean3d.shape[0], -1)[unreached] == 0.0), f"{field}: unreached rows not zeroed"
        err = _rel_l2(got, ref[field])
        assert err <= GRAD_TOL, f"{field}: relative L2 {err:.3e}"


@pytest.mark.parametrize("size", [(1, 1), (17, 5), (5, 40), (16, 16), (33, 1)])
def test_tiny_images(oracle, size):
    """Images of one to three tiles, partial in either direction or both (one pixel, one row, one
    column): the TRAIN image is bit-exact and the gradients are within the bar. 2000 Gaussians of
    the config-0 cube fill each image; 25 to 1933 of them contribute."""
    from gsx_amd import scenes
    width, height = size
    w = scenes.Workload("tiny", scenes.cube_scene(3, 2000), scenes.camera(width, height, 2.0 * max(width, height)))
    print(f"[case] tiny {width}x{height}", flush=True)
    r, cam, g = _setup(w)
    img = r.render(cam, g, train=True)
    rng = np.random.default_rng(5)
    grad_rgb = rng.standard_normal((3, height, width)).astype(np.float32)
    grads = g.zeros_like_grads()
    r.backward(torch.from_numpy(grad_rgb).cuda(), grads)
    torch.cuda.synchronize()
    assert np.array_equal(img.cpu().numpy(), oracle.render(w.scene, w.camera)[0])
    ref = oracle.render_backward(w.scene, w.camera, grad_rgb)
    for field in ("mean3d", "rotation", "logscale", "opacity", "sh0"):
        err = _rel_l2(getattr(grads, field).cpu().numpy(), ref[field])
        assert err <= GRAD_TOL, f"{field}: relative L2 {err:.3e}"


def _mutated(scene, seed):
    sc = scene.copy()
    rng = np.random.default_rng(seed)
    sc.mean3d += (0.02 * rng.standard_normal(sc.mean3d.shape)).astype(np.float32)
    sc.logscale += (0.1 * rng.standard_normal(sc.logscale.shape)).astype(np.float32)
    sc.sh0 += (0.2 * rng.standard_normal(sc.sh0.shape)).astype(np.float32)
    sc.opacity -= np.float32(0.4)
    return sc


def _train_step_grads(r, cam, g, grad_rgb, borrow, mutate_to=None):
    from gsx_amd.backend import GaussianTensors
    r.render(cam, g, train=True, borrow_train_state=borrow)
    if mutate_to is not None:
        src = GaussianTensors.from_scene(mutate_to)
        for name in ("mean3d", "logscale", "sh0", "opacity"):
            getattr(g, name).copy_(getattr(src, name))
    grads = g.zeros_like_grads()
    r.backward(grad_rgb, grads)
    torch.cuda.synchronize()
    return {k: getattr(grads, k).cpu().numpy() for k in ("mean3d", "rotation", "logscale", "opacity", "sh0")}


@pytest.mark.parametrize("name", ["c0_small", "c3_1080"])
def test_borrowed_train_state_tracks_input_mutations(oracle, name):
    """tests/render_runtime.cpp:743-810: after a TRAIN forward with a borrowed state, the caller
    overwrites mean3d, logscale, sh0 and opacity; the backward's gradients are those of a fresh
    forward + backward at the new values."""
    from gsx_amd.backend import GaussianTensors
    w = _workloads()[name]()
    print(f"[case] borrowed state {name}", flush=True)
    mut = _mutated(w.scene, 21)
    r, cam, g = _setup(w)
    rng = np.random.default_rng(8)
    grad_np = rng.standard_normal((3, cam.height, cam.width)).astype(np.float32)
    grad_rgb = torch.from_numpy(grad_np).cuda()
    got = _train_step_grads(r, cam, g, grad_rgb, borrow=True, mutate_to=mut)
    r2, _, _ = _setup(w)
    expect = _train_step_grads(r2, cam, GaussianTensors.from_scene(mut), grad_rgb, borrow=False)
    for k in got:
        assert np.array_equal(got[k], expect[k]), k
    ref = oracle.render_backward(mut, w.camera, grad_np)
    for k in got:
        assert _rel_l2(got[k], ref[k]) <= GRAD_TOL, k
    # the context keeps working: an unchanged borrowed step next
    g2 = GaussianTensors.from_scene(mut)
    again = _train_step_grads(r, cam, g2, grad_rgb, borrow=True)
    for k in got:
        assert np.array_equal(again[k], expect[k]), k


def test_cloned_train_state_ignores_input_mutations(oracle):
    """borrow_train_state = false: the backward differentiates at the forward's values even when
    the caller changes its arrays in between (gsx-cpu/render.c:286-360 clones them)."""
    from gsx_amd.backend import GaussianTensors
    w = _workloads()["c1_small"]()
    r, cam, g = _setup(w)
    rng = np.random.default_rng(9)
    grad_np = rng.standard_normal((3, cam.height, cam.width)).astype(np.float32)
    grad_rgb = torch.from_numpy(grad_np).cuda()
    got = _train_step_grads(r, cam, g, grad_rgb, borrow=False, mutate_to=_mutated(w.scene, 22))
    r2, _, g_fresh = _setup(w)
    expect = _train_step_grads(r2, cam, g_fresh, grad_rgb, borrow=True)
    for k in got:
        assert np.array_equal(got[k], expect[k]), k
    ref = oracle.render_backward(w.scene, w.camera, grad_np)
    for k in got:
        assert _rel_l2(got[k], ref[k]) <= GRAD_TOL, k
    assert not np.array_equal(g.mean3d.cpu().numpy(), w.scene.mean3d)  # the caller's change stands


def test_visible_counter_train_forward(oracle):
    w = _workloads()["c1_small"]()
    r, cam, g = _setup(w)
    counter = torch.full((w.scene.count,), 2.0, dtype=torch.float32, device="cuda")
    r.render(cam, g, train=True, visible_counter=counter)
    r.render(cam, g, train=False, visible_counter=counter)  # inference does not count
    torch.cuda.synchronize()
    ref = np.full(w.scene.count, 2.0, np.float32)
    oracle.render(w.scene, w.camera, visible_counter=ref)
    assert np.array_equal(counter.cpu().numpy(), ref)


def test_backward_requires_train_state():
    from gsx_amd.backend import GsxHipError
    w = _workloads()["c0_small"]()
    r, cam, g = _setup(w)
    grads = g.zeros_like_grads()
    grad_rgb = torch.zeros((3, cam.height, cam.width), dtype=torch.float32, device="cuda")
    with pytest.raises(GsxHipError):
        r.backward(grad_rgb, grads)
    r.render(cam, g, train=True)
    r.backward(grad_rgb, grads)
    with pytest.raises(GsxHipError):  # consumed once
        r.backward(grad_rgb, grads)


def test_empty_and_fully_culled_scenes(oracle):
    from gsx_amd import scenes
    w = scenes.config0(n=500, width=64, height=48)
    sc = w.scene.copy()
    sc.opacity[:] = -10.0  # below the logit cull of render.c:109
    r, cam, g = _setup(scenes.Workload("culled", sc, w.camera))
    img = r.render(cam, g, train=True)
    grads = g.zeros_like_grads()
    r.backward(torch.ones_like(img), grads)
    torch.cuda.synchronize()
    assert r.stats().instance_count == 0
    assert np.array_equal(img.cpu().numpy(), oracle.render(sc, w.camera)[0])
    assert float(grads.mean3d.abs().max()) == 0.0


def test_context_reuse_then_empty_scene(oracle):
    # the list counters of a context are rebuilt by every forward, also by one without Gaussians
    from gsx_amd import scenes
    from gsx_amd.backend import GaussianTensors
    w = scenes.config0(n=500, width=64, height=48)
    r, cam, g = _setup(w)
    r.render(cam, g, train=False)
    torch.cuda.synchronize()
    assert r.stats().instance_count > 0
    sc = w.scene
    empty = scenes.Scene(*(np.ascontiguousarray(a[:0]) for a in (sc.mean3d, sc.rotation, sc.logscale, sc.opacity,
                                                                  sc.sh0)))
    img = r.render(cam, GaussianTensors.from_scene(empty), train=False)
    torch.cuda.synchronize()
    assert r.stats().instance_count == 0
    assert np.array_equal(img.cpu().numpy(), oracle.render(empty, w.camera)[0])


def test_context_reuse_alternating_scenes(oracle):
    # one context, forwards that alternate between a scene with near-plane boxes covering every
    # tile and a subset of it: the big-box counter slots alternate between forwards, and the
    # tile ranges of the tiles a forward leaves empty are rewritten by that forward
    from gsx_amd import scenes
    from gsx_amd.backend import GaussianTensors
    w = _workloads()["c3_1080"]()
    sc = w.scene
    part = scenes.Scene(*(np.ascontiguousarray(a[:3000]) for a in (sc.mean3d, sc.rotation, sc.logscale, sc.opacity,
                                                                   sc.sh0)))
    r, cam, g_full = _setup(w)
    g_part = GaussianTensors.from_scene(part)
    refs = {"full": oracle.render(sc, w.camera)[0], "part": oracle.render(part, w.camera)[0]}
    counts = {}
    for name, g in (("full", g_full), ("part", g_part), ("full", g_full), ("part", g_part)):
        print(f"[case] reuse {name}", flush=True)
        img = r.render(cam, g, train=False)
        torch.cuda.synchronize()
        assert np.array_equal(img.cpu().numpy(), refs[name])
        st = r.stats()
        counts.setdefault(name, st.instance_count)
        assert st.instance_count == counts[name]
    assert counts["full"] > counts["part"] > 0


def test_background_only_pixels(oracle):
    from gsx_amd import scenes
    w = scenes.config0(n=50, width=64, height=48)
    cam_block = w.camera.copy()
    cam_block[15:18] = (0.25, 0.5, 0.75)
    r, cam, g = _setup(scenes.Workload("bg", w.scene, cam_block))
    img = r.render(cam, g).cpu().numpy()
    ref = oracle.render(w.scene, cam_block)[0]
    assert np.array_equal(img, ref)


def test_stats_right_after_forward_on_a_side_stream(oracle):
    """get_stats called straight after a forward queued on a non-blocking stream (no host wait in
    between) reports that forward's visible count: two scenes with different counts, rendered one
    after the other by one context, each against the oracle's count of Gaussians that pass the
    culls (gsx-cpu/render.c:850-1016)."""
    from gsx_amd import scenes
    from gsx_amd.backend import Camera, GaussianTensors, Renderer
    side = torch.cuda.Stream()
    works = [scenes.config1(n=40_000, width=320, height=180), scenes.config1(n=9_000, width=320, height=180)]
    expected = [len(oracle.preprocess(w.scene, w.camera)[0]) for w in works]
    assert expected[0] != expected[1]
    r = Renderer(320, 180)
    for w, want in zip(works + works, expected + expected):
        cam = Camera.from_block(w.camera)
        g = GaussianTensors.from_scene(w.scene)
        torch.cuda.synchronize()
        print(f"[case] stats after forward n={w.scene.count} on a side stream", flush=True)
        with torch.cuda.stream(side):
            r.render(cam, g, train=True, stream=side)
            got = r.stats().visible_count
        assert got == want
    torch.cuda.synchronize()
