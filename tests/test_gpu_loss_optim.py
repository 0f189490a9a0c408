"""GPU parity of the loss, optimizer and sort kernels against the CPU oracle.

L1 / MSE and Adam reproduce the CPU arithmetic exactly (bit equality). SSIM runs in float32
with separable windows where the CPU uses a float64 2D window, so its loss map is held to
1e-5 max-abs and its gradient to 1e-3 relative L2 (tighter than the reference's own
CUDA-vs-CPU tolerances of 2e-3 / 3e-3, tests/cuda_loss_runtime.cpp:427-428).
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SSIM_MAP_TOL = 1e-5   # max-abs on the loss map
SSIM_GRAD_TOL = 1e-3  # relative L2 on the accumulated gradient


def _images(seed, shape):
    rng = np.random.default_rng(seed)
    p = rng.random(shape, dtype=np.float32)
    t = np.clip(p + 0.1 * rng.standard_normal(shape).astype(np.float32), 0, 1).astype(np.float32)
    return p, t


@pytest.mark.parametrize("alg", ["l1", "mse"])
def test_pointwise_losses_bit_exact(oracle, alg):
    from gsx_amd.backend import Loss
    p, t = _images(1, (3, 37, 53))
    base_map = np.random.default_rng(2).random(p.shape, dtype=np.float32)
    base_grad = np.random.default_rng(3).random(p.shape, dtype=np.float32)
    loss = Loss(alg)
    pm, gm = torch.from_numpy(base_map).cuda(), torch.from_numpy(base_grad).cuda()
    pt, tt = torch.from_numpy(p).cuda(), torch.from_numpy(t).cuda()
    loss.forward(pt, tt, pm, 0.7)
    loss.backward(gm, 0.7)
    torch.cuda.synchronize()
    ref_map, ref_grad = base_map.copy(), base_grad.copy()
    oracle.loss(alg, p, t, 0.7, ref_map, ref_grad)
    assert np.array_equal(pm.cpu().numpy(), ref_map)
    assert np.array_equal(gm.cpu().numpy(), ref_grad)


# images narrower or lower than the 11-pixel window (every output is boundary: map 0, no gradient),
# with widths that take the 16-byte halo path (multiples of 4) and the one-float path
@pytest.mark.parametrize("shape", [(3, 64, 80), (2, 3, 33, 47), (3, 11, 12), (3, 1080 // 8, 1920 // 8),
                                   (3, 1080, 1920), (3, 1024, 1024), (1, 1, 1), (3, 4, 7), (2, 2, 10, 10),
                                   (3, 16, 4), (3, 9, 64)])
def test_ssim_forward_backward(oracle, shape):
    from gsx_amd.backend import Loss
    p, t = _images(4, shape)
    base_map = np.full(shape, 0.5, np.float32)
    base_grad = np.full(shape, -0.25, np.float32)
    loss = Loss("ssim")
    pm, gm = torch.from_numpy(base_map).cuda(), torch.from_numpy(base_grad).cuda()
    pt, tt = torch.from_numpy(p).cuda(), torch.from_numpy(t).cuda()
    loss.forward(pt, tt, pm, 0.2)
    loss.backward(gm, 0.2)
    torch.cuda.synchronize()
    ref_map, ref_grad = base_map.copy(), base_grad.copy()
    oracle.loss("ssim", p, t, 0.2, ref_map, ref_grad)
    got_map = pm.cpu().numpy()
    assert np.abs(got_map - ref_map).max() <= SSIM_MAP_TOL
    # boundary is overwritten with 0 (gsx-cpu/loss.c:471-481)
    assert np.all(got_map[..., :5, :] == 0.0) and np.all(got_map[..., :, -5:] == 0.0)
    d = gm.cpu().numpy().astype(np.float64) - base_grad
    dr = ref_grad.astype(np.float64) - base_grad
    assert np.linalg.norm(d - dr) / max(np.linalg.norm(dr), 1e-30) <= SSIM_GRAD_TOL


@pytest.mark.parametrize("shape", [(3, 1024, 1024), (3, 1080, 1920)])
def test_ssim_smooth_images(oracle, shape):
    """Smooth, low-variance images (the image-fit target and a slightly shifted copy, values
    near 0.5): window variances are far below the means' squares, the case where a float32
    E[x^2] - mu^2 cancels. Same bars as above, against the oracle's float64 SSIM."""
    from gsx_amd import scenes
    from gsx_amd.backend import Loss
    c, h, w = shape
    t = scenes.config2(n=1, size=max(h, w)).target[:, :h, :w].copy()
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float32)
    p = np.clip(0.9 * t + 0.05 + 0.02 * np.sin(xx / 37.0 + yy / 53.0)[None], 0, 1).astype(np.float32)
    base_map = np.zeros(shape, np.float32)
    base_grad = np.zeros(shape, np.float32)
    loss = Loss("ssim")
    pm, gm = torch.from_numpy(base_map).cuda(), torch.from_numpy(base_grad).cuda()
    loss.forward(torch.from_numpy(p).cuda(), torch.from_numpy(t).cuda(), pm, 0.2)
    loss.backward(gm, 0.2)
    torch.cuda.synchronize()
    ref_map, ref_grad = base_map.copy(), base_grad.copy()
    oracle.loss("ssim", p, t, 0.2, ref_map, ref_grad)
    map_err = float(np.abs(pm.cpu().numpy() - ref_map).max())
    g = gm.cpu().numpy().astype(np.float64)
    grad_err = np.linalg.norm(g - ref_grad) / max(np.linalg.norm(ref_grad), 1e-30)
    print(f"[ssim smooth {shape}] map max-abs {map_err:.2e}, grad rel L2 {grad_err:.2e}", flush=True)
    assert map_err <= SSIM_MAP_TOL
    assert grad_err <= SSIM_GRAD_TOL


def test_ssim_identical_images_zero_interior():
    from gsx_amd.backend import Loss
    p, _ = _images(5, (3, 40, 40))
    loss = Loss("ssim")
    m = torch.zeros((3, 40, 40), dtype=torch.float32, device="cuda")
    pt = torch.from_numpy(p).cuda()
    loss.forward(pt, pt, m, 1.0)
    torch.cuda.synchronize()
    assert float(m.abs().max()) <= 1e-6


def test_ssim_vector_and_scalar_halo_agree():
    """The SSIM kernels stage their halos with 16-byte loads when the width is a multiple of 4
    and the arrays are 16-byte aligned, and one float at a time otherwise. The same images in
    storage shifted by one float take the scalar path; map, dm workspace and gradient must be
    bit-identical to the aligned run's (the two stagings differ only outside the image, where
    no kept output looks)."""
    from gsx_amd import _lib
    from gsx_amd.backend import ptr
    lib = _lib.load()
    p, t = _images(7, (3, 64, 80))
    n = p.size
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for off in (0, 1):
        buf = torch.zeros(8 * n + 8, device="cuda")
        pt, tt, m, g = (buf[off + k * n: off + (k + 1) * n].view(p.shape) for k in range(4))
        ws = buf[off + 4 * n: off + 7 * n]
        pt.copy_(torch.from_numpy(p))
        tt.copy_(torch.from_numpy(t))
        m.fill_(0.5)
        g.fill_(-0.25)
        assert (ptr(pt).value % 16 == 0) == (off == 0)
        _lib.check(lib.gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(ptr(m), ptr(pt), ptr(tt), 1, 3, 64, 80, 0.2,
                                                                       ptr(ws), 0.8, 1, s))
        _lib.check(lib.gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(ptr(g), ptr(pt), ptr(tt), 1, 3, 64, 80,
                                                                        1e-3, ptr(ws), 2e-3, 1, s))
        torch.cuda.synchronize()
        outs.append((m.clone(), ws.clone(), g.clone()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


def test_fused_l1_ssim_matches_sequential():
    from gsx_amd import _lib
    from gsx_amd.backend import ptr
    lib = _lib.load()
    p, t = _images(6, (3, 50, 70))
    pt, tt = torch.from_numpy(p).cuda(), torch.from_numpy(t).cuda()
    n = p.size
    ws1 = torch.empty(3 * n, device="cuda")
    ws2 = torch.empty(3 * n, device="cuda")
    m1 = torch.zeros_like(pt)
    g1 = torch.zeros_like(pt)
    m2 = torch.zeros_like(pt)
    g2 = torch.zeros_like(pt)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    gs_l1 = np.float32(0.8) / np.float32(n)
    gs_ss = np.float32(0.2) / np.float32(n)
    _lib.check(lib.gsx_hip_loss_l1_f32_forward_kernel_launch(ptr(m1), ptr(pt), ptr(tt), n, 0.8, s))
    _lib.check(lib.gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(ptr(m1), ptr(pt), ptr(tt), 1, 3, 50, 70, 0.2,
                                                                   ptr(ws1), 0.0, 0, s))
    _lib.check(lib.gsx_hip_loss_l1_f32_backward_kernel_launch(ptr(g1), ptr(pt), ptr(tt), n, float(gs_l1), s))
    _lib.check(lib.gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(ptr(g1), ptr(pt), ptr(tt), 1, 3, 50, 70,
                                                                    float(gs_ss), ptr(ws1), 0.0, 0, s))
    _lib.check(lib.gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(ptr(m2), ptr(pt), ptr(tt), 1, 3, 50, 70, 0.2,
                                                                   ptr(ws2), 0.8, 1, s))
    _lib.check(lib.gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(ptr(g2), ptr(pt), ptr(tt), 1, 3, 50, 70,
                                                                    float(gs_ss), ptr(ws2), float(gs_l1), 1, s))
    torch.cuda.synchronize()
    assert torch.equal(m1, m2)
    assert torch.equal(g1, g2)


@pytest.mark.parametrize("hyper", [(1e-3, 0.9, 0.999, 0.0, 1e-8, 0.0), (1e-2, 0.8, 0.99, 0.01, 1e-6, 0.05)])
# "large": 24.5M elements, above the 256 MiB of traffic from which the launch streams its accesses
# (two float4 per thread, non-temporal), with partial last chunks and one group whose parameter
# is not 16-byte aligned (element-wise path)
@pytest.mark.parametrize("size_set", ["small", "large"])
def test_adam_bit_exact(oracle, hyper, size_set):
    from gsx_amd.backend import Adam
    lr, b1, b2, wd, eps, mg = hyper
    rng = np.random.default_rng(8)
    sizes = [3001, 4 * 1000, 17] if size_set == "small" else [5_250_009, 7_000_012, 5_250_009, 1_750_003, 5_250_009]
    params = [rng.standard_normal(s).astype(np.float32) for s in sizes]
    grads = [rng.standard_normal(s).astype(np.float32) * 0.1 for s in sizes]
    pt = [torch.from_numpy(x.copy()).cuda() for x in params]
    if size_set == "large":
        shifted = torch.empty(sizes[3] + 1, dtype=torch.float32, device="cuda")[1:]
        shifted.copy_(pt[3])
        pt[3] = shifted
    gt = [torch.from_numpy(x).cuda() for x in grads]
    opt = Adam([dict(parameter=p, gradient=g, learning_rate=lr, beta1=b1, beta2=b2, weight_decay=wd, epsilon=eps,
                     max_grad=mg) for p, g in zip(pt, gt)])
    ms = [np.zeros_like(x) for x in params]
    vs = [np.zeros_like(x) for x in params]
    for step in range(1, 4):
        opt.step()
        for k in range(len(sizes)):
            oracle.adam_step(params[k], grads[k], ms[k], vs[k], lr, b1, b2, wd, eps, mg, step)
    torch.cuda.synchronize()
    for k in range(len(sizes)):
        assert np.array_equal(pt[k].cpu().numpy(), params[k])
        assert np.array_equal(opt.groups[k]["m"].cpu().numpy(), ms[k])
        assert np.array_equal(opt.groups[k]["v"].cpu().numpy(), vs[k])


@pytest.mark.parametrize("n,end_bit", [(1, 8), (1000, 16), (100_003, 45), (1_500_000, 45)])
def test_radix_sort_stable(n, end_bit):
    from gsx_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(n)
    # many duplicate keys to exercise stability
    keys = rng.integers(0, 1 << min(end_bit, 20), size=n, dtype=np.uint64) << np.uint64(max(end_bit - 20, 0))
    vals = np.arange(n, dtype=np.uint32)
    k = torch.from_numpy(keys.view(np.int64)).cuda()
    v = torch.from_numpy(vals.view(np.int32)).cuda()
    k2 = torch.empty_like(k)
    v2 = torch.empty_like(v)
    temp = torch.empty(lib.gsx_hip_radix_sort_temp_bytes(n), dtype=torch.uint8, device="cuda")
    in_alt = ctypes.c_int(0)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.gsx_hip_radix_sort_pairs_u64(k.data_ptr(), v.data_ptr(), k2.data_ptr(), v2.data_ptr(), n, 0,
                                                ((end_bit + 7) // 8) * 8, temp.data_ptr(), ctypes.byref(in_alt), s))
    torch.cuda.synchronize()
    ko, vo = (k2, v2) if in_alt.value else (k, v)
    order = np.argsort(keys, kind="stable")
    assert np.array_equal(ko.cpu().numpy().view(np.uint64), keys[order])
    assert np.array_equal(vo.cpu().numpy().view(np.uint32), vals[order])


@pytest.mark.parametrize("n,lo,hi", [(1, 23, 63), (4096, 23, 63), (4097, 5, 45), (1_000_003, 23, 63),
                                     (3_000_000, 20, 60)])
def test_radix_sort_keys_stable(n, lo, hi):
    """Keys-only sort on bits [lo, hi): the low payload (an index) keeps input order among equal
    sort bits, i.e. the result equals a stable sort by the sort bits; duplicates are dense."""
    from gsx_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(n + lo)
    span = hi - lo
    sort_part = rng.integers(0, 1 << min(span, 12), size=n, dtype=np.uint64) << np.uint64(span - min(span, 12))
    payload = rng.permutation(n).astype(np.uint64) & np.uint64((1 << lo) - 1)
    keys = (sort_part << np.uint64(lo)) | payload
    k = torch.from_numpy(keys.view(np.int64)).cuda()
    k2 = torch.empty_like(k)
    temp = torch.empty(lib.gsx_hip_radix_sort_temp_bytes(n), dtype=torch.uint8, device="cuda")
    in_alt = ctypes.c_int(0)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"[case] keys sort n={n} bits=[{lo},{hi})", flush=True)
    _lib.check(lib.gsx_hip_radix_sort_keys_u64(k.data_ptr(), k2.data_ptr(), n, lo, lo + ((span + 7) // 8) * 8,
                                               temp.data_ptr(), ctypes.byref(in_alt), s))
    torch.cuda.synchronize()
    ko = (k2 if in_alt.value else k).cpu().numpy().view(np.uint64)
    order = np.argsort(keys >> np.uint64(lo), kind="stable")
    assert np.array_equal(ko, keys[order])


@pytest.mark.parametrize("n,lo,hi,pairs", [(5000, 4, 16, True), (70_001, 4, 16, False), (9000, 7, 10, True),
                                           (40_000, 0, 21, False), (12_345, 30, 35, True)])
def test_radix_sort_partial_digit_span(n, lo, hi, pairs):
    """A span that is not a whole number of 8-bit digits, with random bits above end_bit and
    below begin_bit: only bits [lo, hi) decide the order (a stable sort by them), all other bits
    travel with the key."""
    from gsx_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(n + hi)
    keys = rng.integers(0, 1 << 62, size=n, dtype=np.uint64) | (rng.integers(0, 2, size=n, dtype=np.uint64) << 63)
    vals = np.arange(n, dtype=np.uint32)
    k = torch.from_numpy(keys.view(np.int64).copy()).cuda()
    v = torch.from_numpy(vals.view(np.int32).copy()).cuda()
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    temp = torch.empty(lib.gsx_hip_radix_sort_temp_bytes(n), dtype=torch.uint8, device="cuda")
    in_alt = ctypes.c_int(0)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"[case] partial-digit sort n={n} bits=[{lo},{hi}) pairs={pairs}", flush=True)
    if pairs:
        _lib.check(lib.gsx_hip_radix_sort_pairs_u64(k.data_ptr(), v.data_ptr(), k2.data_ptr(), v2.data_ptr(), n, lo,
                                                    hi, temp.data_ptr(), ctypes.byref(in_alt), s))
    else:
        _lib.check(lib.gsx_hip_radix_sort_keys_u64(k.data_ptr(), k2.data_ptr(), n, lo, hi, temp.data_ptr(),
                                                   ctypes.byref(in_alt), s))
    torch.cuda.synchronize()
    ko = (k2 if in_alt.value else k).cpu().numpy().view(np.uint64)
    order = np.argsort((keys >> np.uint64(lo)) & np.uint64((1 << (hi - lo)) - 1), kind="stable")
    assert np.array_equal(ko, keys[order])
    if pairs:
        vo = (v2 if in_alt.value else v).cpu().numpy().view(np.uint32)
        assert np.array_equal(vo, vals[order])


def test_scan_exclusive():
    from gsx_amd import _lib
    lib = _lib.load()
    for n in (0, 1, 4095, 4096, 4097, 1_000_003):
        x = np.random.default_rng(n).integers(0, 50, size=max(n, 1), dtype=np.uint32)[:n]
        xi = torch.from_numpy(x.view(np.int32).copy()).cuda() if n else torch.empty(1, dtype=torch.int32,
                                                                                     device="cuda")
        out = torch.empty(n + 1, dtype=torch.int32, device="cuda")
        temp = torch.empty(lib.gsx_hip_scan_temp_bytes(n), dtype=torch.uint8, device="cuda")
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.gsx_hip_scan_exclusive_u32(xi.data_ptr(), out.data_ptr(), n, temp.data_ptr(), s))
        torch.cuda.synchronize()
        ref = np.concatenate([[0], np.cumsum(x, dtype=np.uint64)]).astype(np.uint32)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref)
