"""The oracle against the golden fixtures of the reference CPU backend, and the reference's own
finite-difference checks (tests/render_runtime.cpp:934-1089) on the oracle and the fixtures.

Bit equality: the oracle restates the CPU backend's float operations in the same order."""
import numpy as np
import pytest

from golden_io import FD_CASES, FD_CHECKS, RENDER_CASES, central_difference, grads_of, load, scene_of


@pytest.mark.parametrize("name", RENDER_CASES + FD_CASES)
def test_oracle_render_matches_golden(oracle, name):
    d = load(name)
    sc = scene_of(d)
    out, _ = oracle.render(sc, d["camera"])
    assert np.array_equal(out, d["out_rgb"])
    counter = np.zeros(sc.count, np.float32)
    oracle.render(sc, d["camera"], visible_counter=counter)
    assert np.array_equal(counter, d["visible_counter"])
    got = oracle.render_backward(sc, d["camera"], d["grad_rgb"])
    for k, ref in grads_of(d).items():
        assert np.array_equal(got[k].reshape(ref.shape), ref), k


@pytest.mark.parametrize("name", FD_CASES)
def test_golden_gradients_match_finite_differences(oracle, name):
    """Pins the fixture (and so the restatement) against the mathematics, with the reference's
    own tolerances; the analytic gradients are the reference's."""
    d = load(name)
    sc = scene_of(d)
    grads = grads_of(d)
    render = lambda s: oracle.render(s, d["camera"])[0]  # noqa: E731
    for field, index, tol in FD_CHECKS[name]:
        numeric = central_difference(render, sc, field, index, d["grad_rgb"])
        analytic = float(grads[field].reshape(-1)[index])
        assert abs(analytic - numeric) <= tol, (field, index, analytic, numeric)


def test_alpha_saturation_scene_is_in_the_saturation_band():
    d = load("fd_alpha_saturation")
    a = 1.0 / (1.0 + np.exp(-float(d["in_opacity"][0])))
    assert 0.99 < a < 0.999  # tests/render_runtime.cpp:1003-1004


@pytest.mark.parametrize("alg", ["l1", "mse", "ssim"])
def test_oracle_loss_matches_golden(oracle, alg):
    d = load("loss")
    m = d[f"{alg}_map_in"].copy()
    g = d[f"{alg}_grad_in"].copy()
    oracle.loss(alg, d["pred"], d["target"], float(d["scale"]), m, g)
    assert np.array_equal(m, d[f"{alg}_map"])
    assert np.array_equal(g, d[f"{alg}_grad"])


def test_oracle_adam_matches_golden(oracle):
    d = load("adam")
    p = d["param"].copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for step in range(1, int(d["steps"]) + 1):
        oracle.adam_step(p, d["grad"], m, v, *[float(x) for x in d["hyper"]], step)
    assert np.array_equal(p, d["param_after"])


@pytest.mark.parametrize("name", ["adc_default", "adc_absgs_reset"])
def test_oracle_adc_matches_golden(oracle, name):
    from oracle.oracle import AdcParams
    d = load(name)
    params = {k[6:]: d[k].item() for k in d if k.startswith("param_")}
    fields = {k[3:]: d[k].copy() for k in d if k.startswith("in_")}
    aux = {k[4:]: d[k].copy() for k in d if k.startswith("aux_")}
    out, _, counts = oracle.adc_step(fields, None, aux, AdcParams(**params), int(params["max_num_gaussians"]))
    assert list(counts) == list(d["counts"])
    for k in fields:
        assert np.array_equal(out[k].reshape(d[f"out_{k}"].shape), d[f"out_{k}"]), k
