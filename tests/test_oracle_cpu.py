"""CPU checks of the oracle restatement, the reference build and the host-side pieces.

These pin the checker itself, so the GPU parity tests mean something:
  - the restatement is bit-identical to the unmodified reference CPU backend compiled from its
    own sources (oracle/_ref), on seeded scenes, for render forward/backward, losses, Adam, ADC;
  - the reference's own known answer (tests/render_runtime.cpp:671-722) and closed forms;
  - the glibc-exact expf restatement used by the kernels against the host libm;
  - the scene generator's pcg32 stream against gsx's own pcg32 (exported by the reference lib).
"""
import ctypes
import math

import numpy as np
import pytest

from gsx_amd import scenes
from oracle.oracle import AdcParams


def _closed_form_scene():
    sc = scenes.Scene(np.array([[0, 0, 4]], np.float32), np.array([[0, 0, 0, 1]], np.float32),
                      np.zeros((1, 3), np.float32), np.zeros(1, np.float32), np.array([[1, 0, 0]], np.float32))
    cam = np.array([1, 1, 0.5, 0.5, 1, 1, 0, 0, 0, 1, 0, 0, 0, 0.1, 10, 0, 0, 0], np.float32)
    return sc, cam


def test_closed_form_render(oracle):
    # tests/render_runtime.cpp:671-722: 1x1 image, f=1, c=0.5, identity pose -> (0.3910474, 0.25, 0.25)
    sc, cam = _closed_form_scene()
    out, t = oracle.render(sc, cam)
    assert abs(out[0, 0, 0] - 0.3910474) <= 1e-5
    assert abs(out[1, 0, 0] - 0.25) <= 1e-5 and abs(out[2, 0, 0] - 0.25) <= 1e-5
    # the same number from first principles: alpha = 0.999-clamped sigmoid(0) * exp(0) = 0.5,
    # colour = SH_C0 * sh0 + 0.5
    sh_c0 = 0.28209479177387814
    assert abs(out[0, 0, 0] - 0.5 * (sh_c0 + 0.5)) <= 1e-6
    assert abs(t[0, 0] - 0.5) <= 1e-7


def test_background_only_transmittance(oracle):
    sc = scenes.cube_scene(0, 10)
    sc.opacity[:] = -20.0  # every Gaussian culled by the opacity logit cut
    cam = scenes.camera(32, 24, 20.0, background=(0.1, 0.2, 0.3))
    out, t = oracle.render(sc, cam)
    assert np.all(t == 1.0)
    assert np.allclose(out[0], 0.1) and np.allclose(out[1], 0.2) and np.allclose(out[2], 0.3)


@pytest.mark.parametrize("deg", [0, 1, 3])
def test_restatement_matches_reference_render(oracle, reference, deg):
    w = scenes.config1(n=6000, width=96, height=72)
    sc = w.scene
    if deg > 0:
        rng = np.random.default_rng(deg)
        sc.sh_degree = deg
        sc.sh1 = (0.2 * rng.standard_normal((sc.count, 3, 3))).astype(np.float32)
        sc.sh2 = (0.2 * rng.standard_normal((sc.count, 5, 3))).astype(np.float32) if deg >= 2 else None
        sc.sh3 = (0.2 * rng.standard_normal((sc.count, 7, 3))).astype(np.float32) if deg >= 3 else None
    cam = w.camera.copy()
    cam[15:18] = (0.2, 0.1, 0.05)
    got, _ = oracle.render(sc, cam)
    ref = reference.render(sc, cam)
    assert np.array_equal(got, ref)
    counter_a = np.zeros(sc.count, np.float32)
    counter_b = np.zeros(sc.count, np.float32)
    oracle.render(sc, cam, visible_counter=counter_a)
    reference.render(sc, cam, train=True, visible_counter=counter_b)
    assert np.array_equal(counter_a, counter_b)
    grad_rgb = np.random.default_rng(11).standard_normal(got.shape).astype(np.float32)
    g_o = oracle.render_backward(sc, cam, grad_rgb)
    _, g_r = reference.render_grad(sc, cam, grad_rgb)
    for k in g_r:
        assert np.array_equal(g_o[k], g_r[k]), k


def test_restatement_matches_reference_cluster_scene(oracle, reference):
    w = scenes.config3(n=20000, width=160, height=90)
    got, _ = oracle.render(w.scene, w.camera)
    assert np.array_equal(got, reference.render(w.scene, w.camera))


@pytest.mark.parametrize("alg", ["l1", "mse", "ssim"])
def test_restatement_matches_reference_losses(oracle, reference, alg):
    rng = np.random.default_rng(3)
    p = rng.random((3, 23, 31), dtype=np.float32)
    t = rng.random((3, 23, 31), dtype=np.float32)
    m_o = rng.random(p.shape, dtype=np.float32)
    g_o = rng.random(p.shape, dtype=np.float32)
    m_r, g_r = m_o.copy(), g_o.copy()
    oracle.loss(alg, p, t, 0.3, m_o, g_o)
    reference.loss(alg, p, t, 0.3, m_r, g_r)
    assert np.array_equal(m_o, m_r)
    assert np.array_equal(g_o, g_r)


def test_ssim_against_independent_float64(oracle):
    """SSIM map from a separate numpy float64 evaluation (scipy-free 2D correlation)."""
    rng = np.random.default_rng(9)
    p = rng.random((1, 20, 24), dtype=np.float32)
    t = rng.random((1, 20, 24), dtype=np.float32)
    x = np.arange(11) - 5
    g = np.exp(-(x ** 2) / (2 * 1.5 ** 2))
    g = g / g.sum()
    w2 = np.outer(g, g)

    def conv(a):
        pad = np.pad(a.astype(np.float64), 5)
        out = np.zeros(a.shape)
        for dy in range(11):
            for dx in range(11):
                out += w2[dy, dx] * pad[dy:dy + a.shape[0], dx:dx + a.shape[1]]
        return out

    a, b = p[0], t[0]
    mu1, mu2 = conv(a), conv(b)
    s1 = conv(a * a.astype(np.float64)) - mu1 ** 2
    s2 = conv(b * b.astype(np.float64)) - mu2 ** 2
    s12 = conv(a.astype(np.float64) * b) - mu1 * mu2
    ssim = ((2 * mu1 * mu2 + 1e-4) * (2 * s12 + 9e-4)) / ((mu1 ** 2 + mu2 ** 2 + 1e-4) * (s1 + s2 + 9e-4))
    expect = (1 - ssim)[5:-5, 5:-5]
    m = np.zeros_like(p)
    oracle.loss("ssim", p, t, 1.0, m, None)
    assert np.abs(m[0, 5:-5, 5:-5] - expect).max() < 2e-6
    assert np.all(m[0, :5] == 0) and np.all(m[0, :, :5] == 0)


def test_ssim_gradient_finite_difference(oracle):
    rng = np.random.default_rng(12)
    p = rng.random((1, 16, 16), dtype=np.float32)
    t = rng.random((1, 16, 16), dtype=np.float32)
    g = np.zeros_like(p)
    m = np.zeros_like(p)
    oracle.loss("ssim", p, t, 1.0, m, g, mean=False)

    def total(pp):
        mm = np.zeros_like(pp)
        oracle.loss("ssim", pp, t, 1.0, mm, None)
        return float(mm.astype(np.float64).sum())

    for (y, x) in [(8, 8), (5, 10), (7, 3)]:
        e = 1e-3
        pp, pm = p.copy(), p.copy()
        pp[0, y, x] += e
        pm[0, y, x] -= e
        fd = (total(pp) - total(pm)) / (2 * e)
        assert abs(fd - g[0, y, x]) <= 2e-2 * max(1.0, abs(fd))


def test_restatement_matches_reference_adam(oracle, reference):
    rng = np.random.default_rng(4)
    p0 = rng.standard_normal(1000).astype(np.float32)
    g = (0.1 * rng.standard_normal(1000)).astype(np.float32)
    hyper = (1e-2, 0.9, 0.999, 0.01, 1e-8, 0.05)
    p_ref = p0.copy()
    reference.adam(p_ref, g, hyper, 5)
    p_o = p0.copy()
    m = np.zeros_like(p0)
    v = np.zeros_like(p0)
    for step in range(1, 6):
        oracle.adam_step(p_o, g, m, v, *hyper, step)
    assert np.array_equal(p_o, p_ref)


def test_adam_textbook(oracle):
    """One step from zero moments: p -= lr * sign-ish(g) as Kingma & Ba (m_hat = g, v_hat = g^2)."""
    g = np.array([0.5, -2.0, 1e-3], np.float32)
    p = np.zeros(3, np.float32)
    m = np.zeros(3, np.float32)
    v = np.zeros(3, np.float32)
    oracle.adam_step(p, g, m, v, 0.1, 0.9, 0.999, 0.0, 1e-8, 0.0, 1)
    expect = -0.1 * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + 1e-8)
    assert np.allclose(p, expect, rtol=1e-5, atol=1e-7)


def _adc_inputs(n, seed):
    sc = scenes.cube_scene(seed, n)
    rng = np.random.default_rng(seed)
    aux = {"grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
           "absgrad_acc": (rng.random(n) * 4e-3).astype(np.float32),
           "visible_counter": rng.integers(0, 4, n).astype(np.float32)}
    fields = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
              "sh0": sc.sh0}
    return fields, aux


@pytest.mark.parametrize("algorithm,step,max_num", [(0, 100, 5000), (1, 200, 5000), (0, 100, 2100), (1, 600, 3000)])
def test_restatement_matches_reference_adc(oracle, reference, algorithm, step, max_num):
    fields, aux = _adc_inputs(2000, 21 + algorithm)
    p = AdcParams(algorithm=algorithm, pruning_opacity_threshold=0.1, opacity_clamp_value=0.3, max_world_scale=0.05,
                  duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01,
                  duplicate_absgrad_threshold=4e-4, scene_scale=1.0, refine_every=100, start_refine=0,
                  end_refine=1000, max_num_gaussians=max_num, reset_every=300, global_step=step, seed=77)
    out_o, _, counts_o = oracle.adc_step({k: v.copy() for k, v in fields.items()}, None,
                                         {k: v.copy() for k, v in aux.items()}, p, max_num)
    out_r, counts_r = reference.adc({k: v.copy() for k, v in fields.items()}, aux, p, max_num)
    assert list(counts_o) == list(counts_r)
    for k in out_r:
        assert np.array_equal(out_o[k].reshape(out_r[k].shape), out_r[k]), k


def test_expf_restatement_matches_libm(oracle):
    """gsx_expf (gsx_amd/csrc/gsx_math.h) == host expf: exhaustive over the blend's power range
    [-4.5, 0] and the sigmoid/exp argument range, strided over all other floats."""
    neg_zero, neg_4_5 = 0x80000000, 0xC0900000
    assert oracle.expf_mismatches(neg_zero, neg_4_5) == 0
    assert oracle.expf_mismatches(0x00000000, 0x42B17218, 3) == 0   # [0, 88.72]
    assert oracle.expf_mismatches(0x80000000, 0xC2D00000, 3) == 0   # [-104, 0]
    assert oracle.expf_mismatches(0x00000000, 0xFFFFFFFF, 977) == 0  # everything else, sampled


@pytest.mark.parametrize("name", ["logf", "sinf", "cosf"])
def test_logf_sincosf_restatements_match_libm(oracle, name):
    """gsx_logf / gsx_sinf / gsx_cosf (gsx_math.h, ARM optimized-routines as glibc ships them) ==
    host libm: every float of the ADC / randn domain [0, 2pi], every 3rd of [-2pi, 0], every
    97th pattern elsewhere (the full 2^32 sweep was run once with zero mismatches)."""
    assert oracle.libm_mismatches(name, 0x00000000, 0x40C90FDB) == 0      # [0, 2pi]
    assert oracle.libm_mismatches(name, 0x80000000, 0xC0C90FDB, 3) == 0   # [-2pi, -0]
    assert oracle.libm_mismatches(name, 0x00000000, 0xFFFFFFFF, 97) == 0


def test_powf_restatement_matches_libm(oracle):
    """gsx_powf == host powf over 4M random pairs (integer and fractional exponents, negative,
    subnormal, zero, inf and NaN bases) and the MCMC exponents 1/k, k + 1 over [0, 1]."""
    assert oracle.powf_mismatches(1234567, 4_000_000, domain=True) == 0


def test_expf_blend_table_matches_libm(oracle):
    """gsx_expf_blend (exponent folded into a 209-entry table, the blend kernels' expf) == host
    expf for every float of its domain [-4.5, 0], -0 and the subnormals included; the endpoints
    are the table's first and last entries."""
    assert oracle.expf_blend_mismatches(0x80000000, 0xC0900000) == 0
    assert oracle.expf_blend_mismatches(0x00000000, 0x00000000) == 0  # +0


def test_scene_pcg32_matches_gsx(reference):
    """The scene generator's uniform/normal streams equal gsx_pcg32_next_float/_next_normal."""
    lib = reference.lib
    lib.gsx_pcg32_init.restype = None
    handle = ctypes.c_void_p()
    lib.gsx_pcg32_init.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint64]
    lib.gsx_pcg32_next_float.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]
    lib.gsx_pcg32_next_normal.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]
    for normal in (False, True):
        lib.gsx_pcg32_init(ctypes.byref(handle), 1234)
        ref = []
        f = ctypes.c_float()
        for _ in range(500):
            (lib.gsx_pcg32_next_normal if normal else lib.gsx_pcg32_next_float)(handle, ctypes.byref(f))
            ref.append(f.value)
        got = scenes.pcg32_stream(1234, 500, normal)
        assert np.array_equal(got, np.array(ref, np.float32))


def _contributing_pixels(rec, bbox, w, h):
    """Per visible Gaussian, the boolean pixel mask of contributions under the CPU's power and
    alpha cuts (render.c:1046-1066), evaluated in float32 in the CPU's operation order."""
    f = np.float32
    masks = []
    for r, b in zip(rec, bbox):
        inv_det = f(r[5])
        inv_a, inv_b, inv_c = f(r[4]) * inv_det, -f(r[3]) * inv_det, f(r[2]) * inv_det
        xs = np.arange(b[0], b[1] + 1, dtype=np.float32)
        ys = np.arange(b[2], b[3] + 1, dtype=np.float32)
        dx = (xs[None, :] + f(0.5)) - f(r[0])
        dy = (ys[:, None] + f(0.5)) - f(r[1])
        power = f(-0.5) * ((inv_a * dx * dx + f(2.0) * inv_b * dx * dy) + inv_c * dy * dy)
        power = np.minimum(power, f(0.0))
        alpha = np.minimum(f(0.999), f(r[13]) * np.exp(power.astype(np.float64)).astype(np.float32))
        m = np.zeros((h, w), bool)
        m[b[2]:b[3] + 1, b[0]:b[1] + 1] = (power >= f(-4.5)) & (alpha >= f(1.0) / f(255.0))
        masks.append(m)
    return masks


def test_tile_restatement_brute_force(oracle):
    """Every tile list holds, in (depth, index) order, a subset of the visible Gaussians whose
    pixel box meets the tile that contains every Gaussian with a contributing pixel in the tile
    (brute force per pixel); the conservative tile test drops only non-contributing instances."""
    w = scenes.config0(n=3000, width=80, height=56)
    keys, vals = oracle.tile_keys(w.scene, w.camera, 16)
    idx, rec, bbox = oracle.preprocess(w.scene, w.camera)
    tiles_x = (80 + 15) // 16
    ranges = oracle.tile_ranges(keys, tiles_x * ((56 + 15) // 16))
    depth = rec[:, 6]
    masks = _contributing_pixels(rec, bbox, 80, 56)
    dropped = 0
    for tile in range(ranges.shape[0]):
        tx, ty = tile % tiles_x, tile // tiles_x
        x0, y0, x1, y1 = tx * 16, ty * 16, tx * 16 + 15, ty * 16 + 15
        hit = (bbox[:, 0] <= x1) & (bbox[:, 1] >= x0) & (bbox[:, 2] <= y1) & (bbox[:, 3] >= y0)
        contributes = np.array([masks[v][y0:y1 + 1, x0:x1 + 1].any() for v in range(len(idx))], bool)
        s, e = ranges[tile]
        got = vals[s:e].astype(np.int64)
        got_set = set(got.tolist())
        assert got_set <= set(idx[hit].tolist())
        assert set(idx[contributes].tolist()) <= got_set
        order = np.lexsort((got, depth[np.searchsorted(idx, got)]))
        assert np.array_equal(order, np.arange(len(got)))  # already in (depth, index) order
        dropped += int(hit.sum()) - len(got)
    assert dropped > 0  # the test is not vacuous on this scene
    assert np.all(keys[1:] >= keys[:-1])


def test_tile_cull_log_accuracy(oracle):
    """The IEEE-only logarithm behind the per-Gaussian cut (tile_cull.h) against numpy float64,
    over the activated-opacity range and far beyond; the cut's 1e-3 slack needs 1e-5."""
    xs = np.concatenate([np.geomspace(1e-30, 1e30, 4001), np.linspace(1 / 255, 1, 4001)]).astype(np.float32)
    got = np.array([oracle.lib.oracle_tile_logf(float(x)) for x in xs], np.float64)
    ref = np.log(xs.astype(np.float64))
    assert np.max(np.abs(got - ref) / np.maximum(1.0, np.abs(ref))) < 1e-6


def test_tile_test_is_conservative_and_effective(oracle):
    """Random and adversarial Gaussians (thin, rotated, far-off centres, low opacity): a tile is
    never dropped when one of its pixel centres passes the CPU's cuts, and most tiles without a
    contribution are dropped."""
    rng = np.random.default_rng(12)
    f = np.float32
    kept_empty = empty = 0
    for case in range(4000):
        sx, sy = np.exp(rng.uniform(-1.0, 6.0, 2))
        th = rng.uniform(0, np.pi)
        c, s = np.cos(th), np.sin(th)
        cov = np.array([[c, -s], [s, c]]) @ np.diag([sx * sx, sy * sy]) @ np.array([[c, s], [-s, c]])
        cov = cov.astype(np.float32) + np.eye(2, dtype=np.float32) * f(0.3)
        a, b, cc = f(cov[0, 0]), f(cov[0, 1]), f(cov[1, 1])
        det = a * cc - b * b
        if not det > 0:
            continue
        inv_det = f(1.0) / det
        inv_a, inv_b, inv_c = cc * inv_det, -b * inv_det, a * inv_det
        op = f(1.0 / (1.0 + np.exp(-rng.normal(0, 3))))
        mx, my = f(rng.uniform(-50, 300)), f(rng.uniform(-50, 300))
        px0, py0 = int(rng.integers(0, 240)), int(rng.integers(0, 240))
        px1, py1 = px0 + int(rng.integers(0, 16)), py0 + int(rng.integers(0, 16))
        kept = oracle.tile_may_contribute(mx, my, inv_a, inv_b, inv_c, op, px0, px1, py0, py1)
        xs = np.arange(px0, px1 + 1, dtype=np.float32)
        ys = np.arange(py0, py1 + 1, dtype=np.float32)
        dx = (xs[None, :] + f(0.5)) - mx
        dy = (ys[:, None] + f(0.5)) - my
        power = np.minimum(f(-0.5) * ((inv_a * dx * dx + f(2.0) * inv_b * dx * dy) + inv_c * dy * dy), f(0.0))
        alpha = np.minimum(f(0.999), op * np.exp(power.astype(np.float64)).astype(np.float32))
        contributes = bool(((power >= f(-4.5)) & (alpha >= f(1.0) / f(255.0))).any())
        if contributes:
            assert kept, (case, mx, my, inv_a, inv_b, inv_c, op, px0, px1, py0, py1)
        else:
            empty += 1
            kept_empty += int(kept)
    assert empty > 1000
    assert kept_empty < 0.1 * empty


def _random_gaussians(seed, count):
    """Gaussians for the brute-force checks of tile_cull.h, with the pixels of their 3-sigma box
    (clipped to 128 x 128) that pass the CPU's power and alpha cuts. Modes: ordinary Gaussians,
    needles up to 400:1 at any angle, huge Gaussians with means far off the image, and opacities
    just above the 1/255 cut. Yields (case, mode, (mx, my, inv_a, inv_b, inv_c, op), box,
    contributes[y, x])."""
    rng = np.random.default_rng(seed)
    f = np.float32
    for case in range(count):
        mode = case % 4
        sx, sy = np.exp(rng.uniform(-1.0, 4.5, 2))
        if mode == 1:
            sx, sy = np.exp(rng.uniform(2.0, 6.0)), np.exp(rng.uniform(-1.0, 0.5))
        if mode == 2:
            sx = np.exp(rng.uniform(5.0, 9.0))
            sy = sx * np.exp(-rng.uniform(0.0, 2.0))
        th = rng.uniform(0, np.pi)
        c, s_ = np.cos(th), np.sin(th)
        cov = np.array([[c, -s_], [s_, c]]) @ np.diag([sx * sx, sy * sy]) @ np.array([[c, s_], [-s_, c]])
        cov = cov.astype(np.float32) + np.eye(2, dtype=np.float32) * f(0.3)
        a, b, cc = f(cov[0, 0]), f(cov[0, 1]), f(cov[1, 1])
        det = a * cc - b * b
        if not det > 0:
            continue
        inv_det = f(1.0) / det
        inv_a, inv_b, inv_c = cc * inv_det, -b * inv_det, a * inv_det
        op = f(1.0 / (1.0 + np.exp(-rng.normal(0, 3))))
        if mode == 3:
            op = f(1.0 / 255.0 * (1.0 + 0.02 * rng.uniform()))
        if not op >= f(1.0 / 255.0):
            continue
        mx, my = f(rng.uniform(-150, 280)), f(rng.uniform(-150, 280))
        if mode == 2 and case % 8 == 2:
            mx = f(rng.uniform(-2e5, 2e5))
        ex, ey = 3.0 * np.sqrt(float(a)), 3.0 * np.sqrt(float(cc))
        x0, x1 = int(max(0, np.floor(mx - ex))), int(min(127, np.ceil(mx + ex)))
        y0, y1 = int(max(0, np.floor(my - ey))), int(min(127, np.ceil(my + ey)))
        if x0 > x1 or y0 > y1:
            continue
        xs = np.arange(x0, x1 + 1, dtype=np.float32)
        ys = np.arange(y0, y1 + 1, dtype=np.float32)
        dx = (xs[None, :] + f(0.5)) - mx
        dy = (ys[:, None] + f(0.5)) - my
        power = np.minimum(f(-0.5) * ((inv_a * dx * dx + f(2.0) * inv_b * dx * dy) + inv_c * dy * dy), f(0.0))
        alpha = np.minimum(f(0.999), op * np.exp(power.astype(np.float64)).astype(np.float32))
        contributes = (power >= f(-4.5)) & (alpha >= f(1.0) / f(255.0))
        yield case, mode, (mx, my, inv_a, inv_b, inv_c, op), (x0, x1, y0, y1), contributes


def test_tile_band_columns_cover_every_contributing_pixel(oracle):
    """The closed-form row runs of the tile test (tile_cull.h) against per-pixel brute force over
    whole boxes: for every 16-row band of the box, every pixel that passes the CPU's cuts lies in
    the band's kept columns."""
    checked = slack = 0
    for case, mode, g, box, contributes in _random_gaussians(31, 1200):
        x0, x1, y0, y1 = box
        for ty in range(y0 // 16, y1 // 16 + 1):
            py0, py1 = max(ty * 16, y0), min(ty * 16 + 15, y1)
            xa, xb = oracle.tile_band_columns(*g, box, py0, py1)
            cols = np.nonzero(contributes[py0 - y0:py1 - y0 + 1].any(axis=0))[0] + x0
            if len(cols):
                assert xa <= cols[0] and cols[-1] <= xb, (case, mode, ty, xa, xb, cols[0], cols[-1])
                checked += 1
                slack += (cols[0] - xa) + (xb - cols[-1])
            assert x0 <= xa or xa > xb
            assert xb <= x1
    assert checked > 1500
    assert slack / checked < 2.0  # the runs hug the contributing columns


def test_contribution_box_covers_every_contributing_pixel(oracle):
    """The blend kernels' per-pixel box (tile_cull.h gsx_contribution_box) against per-pixel brute
    force: every pixel of the 3-sigma box that passes the CPU's cuts lies inside it, it lies inside
    the 3-sigma box, and it hugs the contributing pixels (the rows are found with x and y
    exchanged: a wrong exchange of inv_a and inv_c, which planted in the restatement fails this
    test, gives the transposed ellipse's rows)."""
    checked = 0
    area_box = area_tight = 0
    slack = 0
    for case, mode, g, box, contributes in _random_gaussians(47, 1600):
        x0, x1, y0, y1 = box
        xa, xb, ya, yb = oracle.contribution_box(*g, box)
        rows = np.nonzero(contributes.any(axis=1))[0] + y0
        cols = np.nonzero(contributes.any(axis=0))[0] + x0
        if len(cols):
            assert xa <= cols[0] and cols[-1] <= xb, (case, mode, xa, xb, cols[0], cols[-1])
            assert ya <= rows[0] and rows[-1] <= yb, (case, mode, ya, yb, rows[0], rows[-1])
            checked += 1
            slack += (cols[0] - xa) + (xb - cols[-1]) + (rows[0] - ya) + (yb - rows[-1])
        if xa <= xb and ya <= yb:
            assert x0 <= xa and xb <= x1 and y0 <= ya and yb <= y1
            area_tight += (xb - xa + 1) * (yb - ya + 1)
        area_box += (x1 - x0 + 1) * (y1 - y0 + 1)
    assert checked > 350
    assert slack / checked < 2.0  # measured 0.46 pixels over the four sides
    assert area_tight < 0.7 * area_box  # the corners and the rim of the 3-sigma box go (measured 0.56)


def test_gather_rows(oracle):
    src = np.arange(40, dtype=np.float32).reshape(10, 4)
    idx = np.array([3, 3, 0, 9], np.int32)
    assert np.array_equal(oracle.gather_rows(src, idx), src[idx])
    with pytest.raises(IndexError):
        oracle.gather_rows(src, np.array([10], np.int32))


def test_camera_look_at_convention():
    """look_at yields the documented pose for 'at (0,0,4) looking at the origin'."""
    pose = scenes.look_at((0.0, 0.0, 4.0))
    q = pose[:4]
    # 180 degrees about x up to sign: (1,0,0,0) xyzw
    assert abs(abs(q[0]) - 1.0) < 1e-6 and np.allclose(q[1:], 0, atol=1e-6)
    assert np.allclose(pose[4:], (0, 0, 4), atol=1e-6)
    assert math.isclose(float(np.linalg.norm(scenes.orbit_pose(5)[:4])), 1.0, rel_tol=1e-6)


@pytest.mark.parametrize("name,kw", [("config0", {}), ("config1", dict(n=60_000, width=640, height=360)),
                                     ("config3", dict(n=80_000)), ("config4", dict(n=20_000, width=480, height=270)),
                                     ("config2", dict(n=50_000, size=256))])
def test_tiled_oracle_matches_serial(oracle, name, kw):
    """The tiled full-scene paths (per-tile lists walked per pixel on all host cores) against
    the serial restatement: pixels and final transmittance bit-exact with and without the tile
    test, keys and values equal to oracle_tile_keys'."""
    from gsx_amd import scenes
    w = getattr(scenes, name)(**kw)
    img, t = oracle.render(w.scene, w.camera)
    for cull in (False, True):
        img2, t2 = oracle.render_tiled(w.scene, w.camera, cull=cull)
        assert np.array_equal(img, img2) and np.array_equal(t, t2), cull
    k, v = oracle.tile_keys(w.scene, w.camera)
    k2, v2 = oracle.tile_keys_tiled(w.scene, w.camera)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)
    img3, t3, k3, v3 = oracle.render_and_keys_tiled(w.scene, w.camera)
    assert np.array_equal(img3, img) and np.array_equal(k3, k)
    _check_tiled_backward(oracle, w.scene, w.camera)


# The tiled backward sums each Gaussian's terms in double, the serial one (bit-exact with the
# reference CPU backend) in float in box-raster order; the difference is the CPU's float
# summation error, measured below 4e-5 on these scenes. A dropped term, a wrong suffix or a
# misplaced pixel moves a field by orders of magnitude more.
TILED_BACKWARD_TOL = 1e-4


def _check_tiled_backward(oracle, scene, camera):
    h, w = int(camera[5]), int(camera[4])
    grad_rgb = np.random.default_rng(3).standard_normal((3, h, w)).astype(np.float32)
    ref = oracle.render_backward(scene, camera, grad_rgb)
    got = oracle.render_backward_tiled(scene, camera, grad_rgb)
    assert set(got) == set(ref)
    for k in ref:
        a = ref[k].astype(np.float64).ravel()
        d = np.linalg.norm(got[k].astype(np.float64).ravel() - a) / max(np.linalg.norm(a), 1e-30)
        assert d <= TILED_BACKWARD_TOL, (k, d)
        # the same Gaussians (invisible, or visible with no contribution) get all-zero rows
        rows_ref = (ref[k].reshape(len(ref[k]), -1) == 0).all(axis=1)
        rows_got = (got[k].reshape(len(got[k]), -1) == 0).all(axis=1)
        assert np.array_equal(rows_ref, rows_got), k


def test_tiled_oracle_sh3_and_empty(oracle):
    from gsx_amd import scenes
    w = scenes.config1(n=20_000, width=320, height=180)
    sc = w.scene.copy()
    rng = np.random.default_rng(5)
    sc.sh_degree = 3
    sc.sh1 = (0.2 * rng.standard_normal((sc.count, 3, 3))).astype(np.float32)
    sc.sh2 = (0.2 * rng.standard_normal((sc.count, 5, 3))).astype(np.float32)
    sc.sh3 = (0.2 * rng.standard_normal((sc.count, 7, 3))).astype(np.float32)
    img, t = oracle.render(sc, w.camera)
    img2, t2 = oracle.render_tiled(sc, w.camera)
    assert np.array_equal(img, img2) and np.array_equal(t, t2)
    _check_tiled_backward(oracle, sc, w.camera)
    empty = scenes.Scene(*(np.ascontiguousarray(a[:0]) for a in (sc.mean3d, sc.rotation, sc.logscale, sc.opacity,
                                                                  sc.sh0)))
    cam = w.camera.copy()
    cam[15:18] = (0.1, 0.2, 0.3)
    img_e, t_e = oracle.render_tiled(empty, cam)
    assert np.array_equal(img_e, oracle.render(empty, cam)[0]) and np.all(t_e == 1.0)
    k, v = oracle.tile_keys_tiled(empty, cam)
    assert len(k) == 0 and len(v) == 0
    ge = oracle.render_backward_tiled(empty, cam, np.ones((3, 180, 320), np.float32))
    assert all(a.size == 0 for a in ge.values())
