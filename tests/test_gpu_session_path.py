"""The session path on the HIP backend: gsx_session_step (gsx/src/gsx-runtime.c:1344-1580), driven
through the unmodified reference core with the HIP plugin in the registry's GPU slot
(oracle/_ref/libgsxref_hip.so), configured as image-fit-demo configures its session
(apps/image_fit_demo.c:1286-1330) at config 2's scale: 1M Gaussians, 1024x1024, one image
served by gsx_dataloader, 0.8 L1 + 0.2 SSIM loss items, Adam over the five SH0 roles, borrowed
train state.

Parity: after the same number of steps the session's parameters equal, bit for bit, those of the
same step sequence driven directly through libgsx_hip.so (render, L1 and SSIM forward and
backward, render backward, Adam). Measurement: the session's time per step with
collect_timings off (no stage synchronisation) and on, and with the async dataloader (prefetch
depth 2), beside the direct step's, written to gpurun_out/session_path_c2.json and printed.
"""
import json
import os
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WARMUP, ITERS = 3, 20


def _direct_steps(w, steps):
    """The session's step sequence through the C-ABI: returns (trained fields, seconds per step
    over the last `steps - WARMUP` steps)."""
    from gsx_amd.backend import Adam, Camera, GaussianTensors, Loss, Renderer
    cam = Camera.from_block(w.camera)
    g = GaussianTensors.from_scene(w.scene)
    grads = g.zeros_like_grads()
    r = Renderer(cam.width, cam.height)
    target = torch.from_numpy(w.target).cuda()
    img = torch.empty_like(target)
    loss_map = torch.empty_like(target)
    grad = torch.empty_like(target)
    l1, ssim = Loss("l1"), Loss("ssim")
    opt = Adam([dict(parameter=g.mean3d, gradient=grads.mean3d, learning_rate=1e-3),
                dict(parameter=g.logscale, gradient=grads.logscale, learning_rate=1e-2),
                dict(parameter=g.rotation, gradient=grads.rotation, learning_rate=1e-2),
                dict(parameter=g.opacity, gradient=grads.opacity, learning_rate=1e-2),
                dict(parameter=g.sh0, gradient=grads.sh0, learning_rate=1e-2)])
    t0 = None
    for i in range(steps):
        if i == WARMUP:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        r.render(cam, g, train=True, out_rgb=img)
        loss_map.zero_()
        grad.zero_()
        l1.forward(img, target, loss_map, 0.8)
        ssim.forward(img, target, loss_map, 0.2)
        l1.backward(grad, 0.8)
        ssim.backward(grad, 0.2)
        r.backward(grad, grads)
        opt.step()
    torch.cuda.synchronize()
    secs = (time.perf_counter() - t0) / (steps - WARMUP)
    return {k: getattr(g, k).cpu().numpy() for k in ("mean3d", "rotation", "logscale", "opacity", "sh0")}, secs


def test_session_path_c2():
    from gsx_amd import scenes
    from oracle.oracle import Reference
    if not Reference.available(hip=True):
        pytest.skip("oracle/_ref/libgsxref_hip.so was not built (needs the reference tree at build time)")
    w = scenes.config2()
    print(f"[case] session path C2 n={w.scene.count} 1024x1024", flush=True)
    hip = Reference(backend="hip")
    sc, secs_off, _ = hip.session_fit(w.scene, w.camera, w.target, WARMUP, ITERS, collect_timings=False)
    print(f"[session] collect_timings off: {1000 * secs_off / ITERS:.3f} ms/step", flush=True)
    _, secs_on, stage_us = hip.session_fit(w.scene, w.camera, w.target, WARMUP, ITERS, collect_timings=True)
    print(f"[session] collect_timings on: {1000 * secs_on / ITERS:.3f} ms/step, last step {list(stage_us)}",
          flush=True)
    _, secs_async, _ = hip.session_fit(w.scene, w.camera, w.target, WARMUP, ITERS, collect_timings=False,
                                       prefetch=2)
    print(f"[session] collect_timings off, async prefetch 2: {1000 * secs_async / ITERS:.3f} ms/step", flush=True)
    direct, secs_direct = _direct_steps(w, WARMUP + ITERS)
    print(f"[direct] {1000 * secs_direct:.3f} ms/step", flush=True)
    for k, v in direct.items():
        assert np.array_equal(getattr(sc, k).reshape(v.shape), v), k
    record = {
        "workload": "config 2 (1M Gaussians, 1024x1024), image-fit-demo's session configuration, SH0, no ADC",
        "steps_timed": ITERS, "warmup": WARMUP,
        "session_ms_per_step_timings_off": round(1000 * secs_off / ITERS, 3),
        "session_ms_per_step_timings_on": round(1000 * secs_on / ITERS, 3),
        "session_ms_per_step_async_prefetch": round(1000 * secs_async / ITERS, 3),
        "direct_abi_ms_per_step": round(1000 * secs_direct, 3),
        "session_last_step_us": dict(zip(("dataloader", "render_forward", "loss_forward", "loss_backward",
                                          "render_backward", "optim", "adc", "total"),
                                         (round(float(x), 1) for x in stage_us))),
        "parameters_equal_after_steps": WARMUP + ITERS,
    }
    out = os.path.join(ROOT, "gpurun_out")
    os.makedirs(out, exist_ok=True)
    with open(os.path.join(out, "session_path_c2.json"), "w") as f:
        json.dump(record, f, indent=1)
    print(f"[session record] {json.dumps(record)}", flush=True)
