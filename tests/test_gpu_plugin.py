"""The HIP backend as a gsx backend: the unmodified reference core (gsx front-ends, registry,
tensors, arenas, Gaussian sets, optimizer/ADC plumbing) driven through gsx's public C API with
the HIP plugin in the registry's GPU slot, against the reference CPU backend of the same process
on the same inputs. This mirrors the reference's own backend tests, which run each public
operation on the CUDA backend and on the CPU backend and compare (tests/cuda_render_runtime.cpp,
tests/cuda_loss_runtime.cpp, tests/cuda_optim_runtime.cpp, tests/cuda_adc_runtime.cpp).

Bars: images, visibility counters, L1/MSE maps and gradients, Adam parameters, fills, clamps,
gathers, the pcg32 streams (rand, randint, multinomial), max reductions and layout/u8 image
conversions are bit-identical; render gradients within 1e-3 relative L2; SSIM maps within 1e-5
max-abs and SSIM gradients within 1e-3 relative L2; sums, means, MSE and MAE within 2 ulp of
the exact value (the HIP backend accumulates in float64; the CPU backend's sequential float32
sum is held to its own error bound around the same value); randn, the sRGB curves and every ADC
row (split rows included) are bit-identical too, through the glibc-exact logf / sinf / cosf /
powf restatements of gsx_math.h.
"""
import numpy as np
import pytest

from gsx_amd import scenes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backends():
    from oracle.oracle import Reference
    if not Reference.available(hip=True):
        pytest.skip("oracle/_ref/libgsxref_hip.so was not built (needs the reference tree at build time)")
    cpu, hip = Reference(backend="cpu"), Reference(backend="hip")
    print(f"[plugin] gpu slot device: {hip.device_name()}", flush=True)
    return cpu, hip


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _sh_scene(w, deg, seed):
    sc = w.scene
    if deg > 0:
        rng = np.random.default_rng(seed)
        sc.sh_degree = deg
        sc.sh1 = (0.2 * rng.standard_normal((sc.count, 3, 3))).astype(np.float32)
        sc.sh2 = (0.2 * rng.standard_normal((sc.count, 5, 3))).astype(np.float32) if deg >= 2 else None
        sc.sh3 = (0.2 * rng.standard_normal((sc.count, 7, 3))).astype(np.float32) if deg >= 3 else None
    return sc


def test_registry_gpu_slot_is_the_hip_device(backends):
    _, hip = backends
    name = hip.device_name()
    assert name, "the GPU slot has no device"


@pytest.mark.parametrize("deg", [0, 1, 3])
def test_render_and_visibility_bit_exact(backends, deg):
    cpu, hip = backends
    w = scenes.config1(n=20000, width=160, height=120)
    sc = _sh_scene(w, deg, 40 + deg)
    cam = w.camera.copy()
    cam[15:18] = (0.2, 0.1, 0.05)
    print(f"[case] plugin render deg={deg} n={sc.count}", flush=True)
    assert np.array_equal(hip.render(sc, cam), cpu.render(sc, cam))
    ca = np.full(sc.count, 2.0, np.float32)
    cb = ca.copy()
    img_c = cpu.render(sc, cam, train=True, visible_counter=ca)
    img_h = hip.render(sc, cam, train=True, visible_counter=cb)
    assert np.array_equal(img_h, img_c)
    assert np.array_equal(cb, ca)


@pytest.mark.parametrize("deg", [0, 2, 3])
def test_render_backward(backends, deg):
    cpu, hip = backends
    w = scenes.config1(n=20000, width=160, height=120)
    sc = _sh_scene(w, deg, 50 + deg)
    grad_rgb = np.random.default_rng(deg).standard_normal((3, 120, 160)).astype(np.float32)
    print(f"[case] plugin render_grad deg={deg}", flush=True)
    img_c, g_c = cpu.render_grad(sc, w.camera, grad_rgb)
    img_h, g_h = hip.render_grad(sc, w.camera, grad_rgb)
    assert np.array_equal(img_h, img_c)
    assert set(g_h) == set(g_c)
    for k in g_c:
        assert _rel(g_h[k], g_c[k]) <= 1e-3, k


def _images(seed, shape):
    rng = np.random.default_rng(seed)
    p = rng.random(shape, dtype=np.float32)
    t = np.clip(p + 0.1 * rng.standard_normal(shape).astype(np.float32), 0, 1).astype(np.float32)
    return p, t


@pytest.mark.parametrize("alg", ["l1", "mse", "ssim"])
@pytest.mark.parametrize("mean", [True, False])
@pytest.mark.parametrize("shape", [(3, 48, 64), (2, 3, 33, 47)])
def test_loss(backends, alg, mean, shape):
    cpu, hip = backends
    p, t = _images(7, shape)
    maps = [np.full(shape, 0.5, np.float32) for _ in range(2)]
    grads = [np.full(shape, -0.25, np.float32) for _ in range(2)]
    print(f"[case] plugin loss {alg} mean={mean} {shape}", flush=True)
    cpu.loss(alg, p, t, 0.3, maps[0], grads[0], mean=mean)
    hip.loss(alg, p, t, 0.3, maps[1], grads[1], mean=mean)
    if alg == "ssim":
        assert np.abs(maps[1] - maps[0]).max() <= 1e-5
        assert _rel(grads[1] - (-0.25), grads[0] - (-0.25)) <= 1e-3
    else:
        assert np.array_equal(maps[1], maps[0])
        assert np.array_equal(grads[1], grads[0])


@pytest.mark.parametrize("hyper,steps", [
    ((1e-3, 0.9, 0.999, 0.0, 1e-8, 0.0), 7),
    ((1e-2, 0.8, 0.99, 0.01, 1e-6, 0.05), 3),
])
def test_adam(backends, hyper, steps):
    cpu, hip = backends
    rng = np.random.default_rng(3)
    param = rng.standard_normal(10007).astype(np.float32)
    grad = (0.1 * rng.standard_normal(10007)).astype(np.float32)
    a, b = param.copy(), param.copy()
    cpu.adam(a, grad, hyper, steps)
    hip.adam(b, grad, hyper, steps)
    assert np.array_equal(b, a)


def _adc_inputs(n, seed):
    sc = scenes.cube_scene(seed, n)
    rng = np.random.default_rng(seed)
    fields = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
              "sh0": sc.sh0}
    aux = {"grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
           "absgrad_acc": (rng.random(n) * 4e-3).astype(np.float32),
           "visible_counter": rng.integers(0, 4, n).astype(np.float32)}
    return fields, aux


@pytest.mark.parametrize("algorithm,step,max_num", [(0, 100, 5000), (1, 200, 5000), (0, 100, 2100), (1, 600, 3000),
                                                    (0, 300, 1500)])
def test_adc(backends, algorithm, step, max_num):
    from oracle.oracle import AdcParams
    cpu, hip = backends
    n = 2000
    fields, aux = _adc_inputs(n, 61 + algorithm + step)
    params = AdcParams(algorithm=algorithm, pruning_opacity_threshold=0.1, opacity_clamp_value=0.3,
                       max_world_scale=0.05, duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01,
                       duplicate_absgrad_threshold=4e-4, scene_scale=1.0, refine_every=100, start_refine=0,
                       end_refine=1000, max_num_gaussians=max_num, reset_every=300, global_step=step, seed=5)
    print(f"[case] plugin adc alg={algorithm} step={step} max={max_num}", flush=True)
    out_c, cnt_c = cpu.adc(fields, aux, params, max(n, max_num), optim_probe=True)
    out_h, cnt_h = hip.adc(fields, aux, params, max(n, max_num), optim_probe=True)
    assert np.array_equal(cnt_h, cnt_c)
    assert out_h["mean3d"].shape == out_c["mean3d"].shape
    for k in out_c:
        assert np.array_equal(out_h[k], out_c[k]), k


def test_train_steps(backends):
    cpu, hip = backends
    w = scenes.config2(n=20000, size=128)
    print("[case] plugin image-fit steps", flush=True)
    sc_c, _ = cpu.train_steps(w.scene, w.camera, w.target, 4)
    sc_h, _ = hip.train_steps(w.scene, w.camera, w.target, 4)
    for k in ("mean3d", "rotation", "logscale", "opacity", "sh0"):
        d_c = getattr(sc_c, k).astype(np.float64) - getattr(w.scene, k)
        d_h = getattr(sc_h, k).astype(np.float64) - getattr(w.scene, k)
        assert _rel(d_h, d_c) <= 1e-3, k


# ---- tensor, random and image operations ---------------------------------------------------------

def _terms(op, x, y):
    if op in ("sum", "mean"):
        return x.astype(np.float64)
    d = x - y  # float32, as both backends form it
    return (d * d if op == "mse" else np.abs(d)).astype(np.float64)


@pytest.mark.parametrize("shape,axis", [((5, 3, 7), 1), ((4, 100003), 1), ((3, 40, 50), 0), ((2, 3, 4, 5), 2)])
def test_reduce(backends, shape, axis):
    """The HIP sums accumulate in float64: within 2 ulp of the exact sum of the float32 terms.
    The CPU backend sums sequentially in float32, so it is held to the sequential-sum error
    bound n * 2^-24 * sum|t| around the same exact value, and max is bit-identical."""
    cpu, hip = backends
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape).astype(np.float32)
    x.flat[0] = -5.0
    lead = shape[:axis]
    n = int(np.prod(shape[axis:]))
    for op in ("sum", "mean", "mse", "mae"):
        t = _terms(op, x, y).reshape(lead + (n,))
        exact = t.sum(axis=-1)
        bound = n * 2.0 ** -24 * np.abs(t).sum(axis=-1)
        if op != "sum":
            exact, bound = exact / n, bound / n
        a = hip.reduce(op, x, axis, y=y if op in ("mse", "mae") else None).astype(np.float64)
        b = cpu.reduce(op, x, axis, y=y if op in ("mse", "mae") else None).astype(np.float64)
        ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(a - exact) <= 2 * ulp), op
        assert np.all(np.abs(b - exact) <= bound + 2 * ulp), op
    xm = x.copy()
    xm.flat[3] = np.nan
    assert np.array_equal(hip.reduce("max", xm, axis), cpu.reduce("max", xm, axis), equal_nan=True)
    xm.flat[0] = np.nan
    assert np.array_equal(hip.reduce("max", xm, axis), cpu.reduce("max", xm, axis), equal_nan=True)


def test_reduce_closed_forms(backends):
    """The reference's backend test values (tests/cuda_backend_runtime.cpp:1158-1191): x = 1..24
    as [2, 12], target = x + 1."""
    cpu, hip = backends
    x = np.arange(1, 25, dtype=np.float32).reshape(2, 12)
    y = x + 1.0
    for r in (cpu, hip):
        assert np.array_equal(r.reduce("sum", x, 1), [78.0, 222.0])
        assert np.array_equal(r.reduce("mean", x, 1), [6.5, 18.5])
        assert np.array_equal(r.reduce("max", x, 1), [12.0, 24.0])
        assert np.array_equal(r.reduce("mse", x, 1, y=y), [1.0, 1.0])
        assert np.array_equal(r.reduce("mae", x, 1, y=y), [1.0, 1.0])


@pytest.mark.parametrize("op", ["exp", "sigmoid", "sigmoid_derivative", "abs"])
def test_unary(backends, op):
    cpu, hip = backends
    x = np.random.default_rng(9).standard_normal(70001).astype(np.float32) * 8
    x[:4] = (0.0, -0.0, 88.5, -103.0)
    for inplace in (False, True):
        assert np.array_equal(hip.unary(op, x, inplace), cpu.unary(op, x, inplace)), (op, inplace)


def test_clamp_finite_gather(backends):
    cpu, hip = backends
    rng = np.random.default_rng(10)
    x = rng.standard_normal(50000).astype(np.float32)
    x[7] = np.nan
    assert np.array_equal(hip.clamp(x, -0.5, 0.25), cpu.clamp(x, -0.5, 0.25), equal_nan=True)
    assert hip.check_finite(x) is False and cpu.check_finite(x) is False
    x[7] = np.inf
    assert hip.check_finite(x) is False
    x[7] = 1.0
    assert hip.check_finite(x) is True and cpu.check_finite(x) is True
    rows = rng.standard_normal((1000, 7, 3)).astype(np.float32)
    idx = rng.integers(0, 1000, 1500).astype(np.int32)
    assert np.array_equal(hip.gather(rows, idx), cpu.gather(rows, idx))
    with pytest.raises(RuntimeError):
        hip.gather(rows, np.array([0, 1000], np.int32))


@pytest.mark.parametrize("count", [1, 17, 100003])
def test_random_streams(backends, count):
    cpu, hip = backends
    for seed in (0, 12345, 2**40 + 7):
        assert np.array_equal(hip.random("rand", seed, count), cpu.random("rand", seed, count))
        for bound in (1.0, 7.0, 1000.0, 3.0e9):
            assert np.array_equal(hip.random("randint", seed, count, bound), cpu.random("randint", seed, count, bound))
        assert np.array_equal(hip.random("randn", seed, count, 0.5), cpu.random("randn", seed, count, 0.5))
        cdf = np.cumsum(np.random.default_rng(seed % 1000).random(37)).astype(np.float32)
        assert np.array_equal(hip.random("multinomial", seed, count, cdf=cdf),
                              cpu.random("multinomial", seed, count, cdf=cdf))


def test_image_conversions(backends):
    cpu, hip = backends
    rng = np.random.default_rng(12)
    img = (rng.random((3, 37, 53)) * 1.4 - 0.2).astype(np.float32)
    img[0, 0, :3] = (np.nan, np.inf, -np.inf)
    for kind in ("to_srgb", "to_linear"):
        assert np.array_equal(hip.image(kind, img, 3, 37, 53), cpu.image(kind, img, 3, 37, 53), equal_nan=True), kind
    hwc = rng.random((37, 53, 4)).astype(np.float32)
    assert np.array_equal(hip.image("hwc_to_chw", hwc, 4, 37, 53), cpu.image("hwc_to_chw", hwc, 4, 37, 53))
    chw = rng.random((4, 37, 53)).astype(np.float32)
    assert np.array_equal(hip.image("chw_to_hwc", chw, 4, 37, 53), cpu.image("chw_to_hwc", chw, 4, 37, 53))
    assert np.array_equal(hip.image("to_u8", img, 3, 37, 53), cpu.image("to_u8", img, 3, 37, 53))
    u8 = rng.integers(0, 256, (3, 37, 53)).astype(np.uint8)
    assert np.array_equal(hip.image("from_u8", u8, 3, 37, 53), cpu.image("from_u8", u8, 3, 37, 53))


MCMC_CASES = [  # rows, grow_ratio, max_num, steps, first step, noise_strength, reset_every
    (2500, 0.2, 5000, 1, 100, 50.0, 0),          # relocation + growth in one refine
    (2500, 0.5, 3200, 3, 99, 50.0, 0),           # noise, refine (growth capped by max_num), noise
    (2500, 0.0, 0, 2, 299, 50.0, 300),           # noise then relocation with an opacity reset window
    (2500, 0.3, 4000, 2, 999, 50.0, 0),          # noise stops at end_refine (1000): the refine only
    (2500, 0.25, 4000, 1, 100, 0.0, 0),          # no noise
    (300_000, 0.1, 400_000, 2, 100, 50.0, 0),    # at scale: 36k relocations, 30k appended rows
]


@pytest.mark.parametrize("n,grow,max_num,steps,first,noise,reset_every", MCMC_CASES)
def test_adc_mcmc(backends, n, grow, max_num, steps, first, noise, reset_every):
    """MCMC density control (gsx/src/gsx-cpu/adc/mcmc.c) through gsx_adc_step on both backends:
    relocated and appended rows, counts and the optimizer state they leave (an Adam step on
    normal gradients before and after: cleared moments and restarted step counts change it)
    bit-identical. The checker is the reference CPU backend itself: the C oracle has no MCMC
    restatement."""
    from oracle.oracle import AdcParams
    cpu, hip = backends
    fields, aux = _adc_inputs(n, 77 + steps)
    rng = np.random.default_rng(5)
    dead = rng.random(n) < 0.12
    fields["opacity"] = np.where(dead, -4.0, np.abs(fields["opacity"]) + 0.5).astype(np.float32)
    params = AdcParams(algorithm=2, pruning_opacity_threshold=0.05, opacity_clamp_value=0.3, max_world_scale=0.0,
                       duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01,
                       duplicate_absgrad_threshold=4e-4, scene_scale=1.0, refine_every=100, start_refine=0,
                       end_refine=1000, max_num_gaussians=max_num, reset_every=reset_every, global_step=first,
                       seed=11)
    cap = max(n, max_num)
    print(f"[case] plugin mcmc grow={grow} max={max_num} steps={steps} from={first} noise={noise}", flush=True)
    kw = dict(noise_strength=noise, grow_ratio=grow, steps=steps, optim_probe=True)
    out_c, cnt_c = cpu.adc(fields, aux, params, cap, **kw)
    out_h, cnt_h = hip.adc(fields, aux, params, cap, **kw)
    assert cnt_c[0] == int(dead.sum()) or first % 100 != 0 or steps > 1
    assert np.array_equal(cnt_h, cnt_c)
    assert out_h["mean3d"].shape == out_c["mean3d"].shape
    for k in out_c:
        assert np.array_equal(out_h[k], out_c[k]), k


@pytest.mark.parametrize("dtype", [np.uint8, np.float32])
@pytest.mark.parametrize("prefetch", [0, 1, 3])
def test_dataloader(backends, dtype, prefetch):
    """gsx_dataloader on the HIP backend, synchronous (prefetch 0) and with the async loader of
    the plugin (pinned staging, helper stream, event-ordered slots), against the CPU backend's
    synchronous loader and the expected CHW floats: same order over several shuffled epochs,
    same values (u8 payloads keep their values), same per-sample intrinsics."""
    cpu, hip = backends
    rng = np.random.default_rng(21)
    shape = (7, 45, 61)
    if dtype == np.uint8:
        rgb = rng.integers(0, 256, shape + (3,)).astype(np.uint8)
        alpha = rng.integers(0, 256, shape).astype(np.uint8)
    else:
        rgb = rng.standard_normal(shape + (3,)).astype(np.float32)
        alpha = rng.random(shape).astype(np.float32)
    print(f"[case] plugin dataloader {np.dtype(dtype).name} prefetch={prefetch}", flush=True)
    ref = cpu.dataloader(rgb, alpha, shuffle=True, seed=9, prefetch=0, steps=17)
    got = hip.dataloader(rgb, alpha, shuffle=True, seed=9, prefetch=prefetch, steps=17)
    for a, b in zip(got, ref):
        assert np.array_equal(a, b)
    idx = ref[2]
    assert np.array_equal(ref[0], rgb[idx].transpose(0, 3, 1, 2).astype(np.float32))
    assert np.array_equal(ref[1], alpha[idx].astype(np.float32))
    assert sorted(idx[:7].tolist()) == list(range(7)) and ref[3][-1] == 2


def test_dataloader_full_hd_async(backends):
    """1080p u8 frames through the async loader (prefetch 2): 6 MB payloads per slot."""
    cpu, hip = backends
    rng = np.random.default_rng(22)
    rgb = rng.integers(0, 256, (3, 1080, 1920, 3)).astype(np.uint8)
    ref = cpu.dataloader(rgb, None, shuffle=False, seed=0, prefetch=0, steps=5)
    got = hip.dataloader(rgb, None, shuffle=False, seed=0, prefetch=2, steps=5)
    assert np.array_equal(got[2], [0, 1, 2, 0, 1])
    assert np.array_equal(got[0], ref[0])
