#!/usr/bin/env python3
"""Headline benchmark: one gsx training step on one MI355X.

Workload (BASELINE.json metric "fwd+bwd train iters/sec @1M Gaussians 1920x1080"): the
config-3 scene generator at N = 1,000,000 (64 anisotropic clusters + 20% radius-10 shell,
logscale N(-4.5, 0.6), opacity N(0, 1.5), SH0), 1920x1080 pinhole f = 1600, one of 24 orbit
poses (radius 6) per step, seeded blurred-noise targets. One step = TRAIN render forward,
0.8 L1 + 0.2 (1 - SSIM) forward and backward, render backward, Adam over the five parameter
groups (mean3d lr 1e-3, others 1e-2). All inputs are resident in HBM before the timed region.

Printed (rank 0, one JSON line): the train it/s as `value` (K steps with nothing else on the
stream), plus the inference render FPS, the sort bandwidth, a per-kernel table and the roofline
entry of the dominant kernel (both from a replay of the same K steps from the same parameter
and Adam state, with HIP events at every stage boundary), and the CPU baseline (the unmodified gsx CPU backend built from the reference
sources, when present).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(stage, n, visible, instances, tiles, pixels, sort_passes, depth_sort_passes, train=True):
    """Bytes each stage must move at minimum, given this build's data layout (the roofline
    numerators). n Gaussians, visible V, instances I, tiles T, pixels Px, E = 3 Px elements."""
    i = instances
    if stage == "preprocess":
        return 68 * n + (80 if train else 48) * visible
    if stage == "depth_order":
        # depth-key sort (keys only: read for the histogram, read + write to scatter), rank
        # gather (key, count, three index writes), count scan
        return depth_sort_passes * 24 * n + 28 * n + 8 * n
    if stage == "emit":
        return 12 * n + 48 * visible + 12 * i
    if stage == "sort":
        return sort_passes * 24 * i
    if stage == "ranges":
        return 20 * i + 8 * tiles
    if stage == "blend_forward":
        return 52 * i + 20 * pixels + (32 * i if train else 0)
    if stage == "blend_backward":
        return 156 * i + 20 * pixels
    if stage == "instance_reduce":
        return 36 * i + 40 * n
    if stage == "projection_backward":
        return 148 * n
    if stage == "loss_forward":
        return 24 * 3 * pixels
    if stage == "loss_backward":
        return 28 * 3 * pixels
    if stage == "adam":
        return 28 * 14 * n
    return 0


CPU_SAMPLE_STRIDE = 10

STAGE_KERNEL = {"preprocess": "preprocess_kernel", "emit": "emit_kernel", "ranges": "tile_ranges_kernel",
                "blend_forward": "blend_forward_kernel", "blend_backward": "blend_backward_kernel",
                "instance_reduce": "reduce_instance_grads_kernel",
                "projection_backward": "projection_backward_kernel", "loss_forward": "ssim_forward_kernel",
                "loss_backward": "ssim_backward_kernel", "adam": "adam_multi_kernel"}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_metric.txt")
SQ_FILE = os.path.join(ROOT, "profiles", "sq_counters_metric.md")
# Nominal VALU issue peak: 256 CUs x 4 SIMDs x 2.4 GHz, one wave64 instruction per 4 cycles on a
# 16-lane SIMD (some instruction mixes issue faster, so this is a reference, not a hard ceiling).
VALU_PEAK_GINSTR = 256 * 4 * 2.4 / 4.0


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (already scaled by the copy-kernel calibration there), or None."""
    if kernel is None or not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 4 and parts[0] == "traffic" and parts[1] == kernel:
                return int(float(parts[-1]))
    return None


def profiled_valu_instructions(kernel):
    """VALU wave instructions per launch of `kernel` from the committed rocprofv3 SQ_INSTS_VALU
    summary, or None."""
    if kernel is None or not os.path.exists(SQ_FILE):
        return None
    with open(SQ_FILE) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 7 and cells[0] == kernel:
                try:
                    return int(float(cells[6]))
                except ValueError:
                    return None
    return None


def cpu_baseline(scene, camera_block, target, iters):
    """Time the unmodified gsx CPU backend (oracle/_ref) on a bounded sample of the workload:
    every 10th Gaussian of the 1M scene (same distributions) at the full 1920x1080, pose 0.
    The full 1M scene cannot run there: its near-plane Gaussians' pixel boxes cover the image,
    and the CPU backward's contribution scratch exceeds its int32 tensor limit."""
    import numpy as np

    from gsx_amd import scenes
    from oracle.oracle import Reference
    if not Reference.available():
        return None
    sub = scenes.Scene(*(np.ascontiguousarray(a[::CPU_SAMPLE_STRIDE]) for a in
                         (scene.mean3d, scene.rotation, scene.logscale, scene.opacity, scene.sh0)))
    ref = Reference()
    t0 = time.perf_counter()
    _, stages = ref.train_steps(sub, camera_block, target, iters)
    elapsed = time.perf_counter() - t0
    return elapsed, stages, sub.count


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--gaussians", type=int, default=1_000_000)
    ap.add_argument("--width", type=int, default=1920)
    ap.add_argument("--height", type=int, default=1080)
    ap.add_argument("--poses", type=int, default=24)
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run one plain copy kernel of this size first (reference for traffic counters)")
    ap.add_argument("--cpu-baseline-iters", type=int, default=3,
                    help="reference CPU steps to time on the full workload (0 disables)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU scaling (image tile bands "
                                   "per GPU, one gradient all-reduce) is not built", "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch

    from gsx_amd import _lib, scenes
    from gsx_amd.backend import Adam, Camera, GaussianTensors, Renderer, ptr, stream_handle

    lib = _lib.load()
    dev_name = torch.cuda.get_device_name(0)
    log(f"device {dev_name}; generating the metric scene (N={args.gaussians})")
    t0 = time.perf_counter()
    base = scenes.metric_scene(args.gaussians, args.width, args.height, 0)
    cams = []
    targets = []
    for k in range(args.poses):
        pose = scenes.orbit_pose(k)
        block = scenes.camera(args.width, args.height, 1600.0 * args.width / 1920.0, pose=tuple(pose), near=0.01,
                              far=100.0)
        cams.append(Camera.from_block(block))
        tgt = base.target if k == 0 else scenes.target_image(0, 103 + k, args.width, args.height, 2)
        targets.append(torch.from_numpy(tgt).cuda())
    log(f"scene + {args.poses} targets ready in {time.perf_counter() - t0:.1f}s")

    g = GaussianTensors.from_scene(base.scene)
    grads = g.zeros_like_grads()
    renderer = Renderer(args.width, args.height)
    img = torch.empty((3, args.height, args.width), dtype=torch.float32, device="cuda")
    # the loss launchers accumulate (+=) into the loss map and the image gradient, so both start
    # each step at zero: one allocation, cleared by one fill
    loss_and_grad = torch.empty((2,) + tuple(img.shape), dtype=torch.float32, device="cuda")
    loss_map, grad_img = loss_and_grad[0], loss_and_grad[1]
    ssim_ws = torch.empty(3 * img.numel(), dtype=torch.float32, device="cuda")
    opt = Adam([dict(parameter=g.mean3d, gradient=grads.mean3d, learning_rate=1e-3),
                dict(parameter=g.logscale, gradient=grads.logscale, learning_rate=1e-2),
                dict(parameter=g.rotation, gradient=grads.rotation, learning_rate=1e-2),
                dict(parameter=g.opacity, gradient=grads.opacity, learning_rate=1e-2),
                dict(parameter=g.sh0, gradient=grads.sh0, learning_rate=1e-2)])
    numel = img.numel()
    gs_l1 = float(np.float32(0.8) / np.float32(numel))
    gs_ssim = float(np.float32(0.2) / np.float32(numel))
    H, W = args.height, args.width

    ev = {k: [] for k in ("loss_forward", "loss_backward", "adam")}

    def step(i, record=False, borrow=True):
        cam = cams[i % args.poses]
        tgt = targets[i % args.poses]
        st = stream_handle()
        renderer.render(cam, g, train=True, out_rgb=img, borrow_train_state=borrow)
        loss_and_grad.zero_()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)] if record else None
        if record:
            e[0].record()
        # 0.8 L1 + 0.2 (1 - SSIM), fused in one pass each way (bit-identical to separate calls)
        _lib.check(lib.gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(
            ptr(loss_map), ptr(img), ptr(tgt), 1, 3, H, W, 0.2, ptr(ssim_ws), 0.8, 1, st), "loss forward")
        if record:
            e[1].record()
        _lib.check(lib.gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(
            ptr(grad_img), ptr(img), ptr(tgt), 1, 3, H, W, gs_ssim, ptr(ssim_ws), gs_l1, 1, st), "loss backward")
        if record:
            e[2].record()
        renderer.backward(grad_img, grads)
        if record:
            e[3].record()
        opt.step()
        if record:
            e4 = torch.cuda.Event(enable_timing=True)
            e4.record()
            ev["loss_forward"].append((e[0], e[1]))
            ev["loss_backward"].append((e[1], e[2]))
            ev["adam"].append((e[3], e4))

    if args.calibrate_copy_mib > 0:
        nf = args.calibrate_copy_mib * (1 << 20) // 4
        a = torch.ones(nf, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        _lib.check(lib.gsx_hip_copy_f32(ptr(b), ptr(a), nf, stream_handle()), "calibration copy")
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calibrate_copy_mib} MiB read + {args.calibrate_copy_mib} MiB written")
        del a, b

    log(f"warmup {args.warmup} steps")
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # training moves the Gaussians, so pass 2 restarts from this state and replays pass 1's steps
    def opt_state():
        out = []
        for grp in opt.groups:
            out += [grp["parameter"], grp["m"], grp["v"]]
        return out

    snapshot = [t.clone() for t in opt_state()]
    steps_before = [grp["step"] for grp in opt.groups]

    def restore():
        for t, saved in zip(opt_state(), snapshot):
            t.copy_(saved)
        for grp, k in zip(opt.groups, steps_before):
            grp["step"] = k

    def timed_pass(borrow):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(args.warmup + i, borrow=borrow)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    # 1. throughput: K steps with nothing but the work on the stream (the per-stage HIP events
    #    of pass 3 cost about 45 us per step, so they stay out of this loop). The TRAIN state is
    #    borrowed, as gsx's training session requests (apps/image_fit_demo.c:1305): the backward
    #    checks the caller's arrays against the forward's copy before differentiating.
    log(f"timing {args.steps} steps (borrowed train state)")
    elapsed = timed_pass(True)
    it_s = args.steps / elapsed
    # 2. the same K steps from the same state with a cloned TRAIN state (borrow_train_state =
    #    false, the zero-initialised request's choice): no check in the backward
    restore()
    log(f"timing {args.steps} steps (cloned train state)")
    it_s_clone = args.steps / timed_pass(False)
    # 3. per-kernel times: the same K steps from the same state, with HIP events at every stage
    #    boundary, recorded on the launch stream inside the library and around the loss and
    #    Adam launches here
    restore()
    del snapshot
    renderer.set_timing(args.steps)
    log(f"per-stage timing over the same {args.steps} steps")
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(args.warmup + i, record=True)  # the poses of pass 1 again
    torch.cuda.synchronize()
    stage_ms = renderer.timings()
    renderer.set_timing(0)
    for k, pairs in ev.items():
        stage_ms[k] = sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)
    stats = renderer.stats()
    instances = int(stats.instance_count)
    visible = int((torch.zeros(1)).item())  # filled below
    # visible Gaussians of the last pose (tile count > 0), for the byte model
    buf = renderer.buffers()
    tc = torch.empty(args.gaussians, dtype=torch.int32, device="cuda")
    _lib.check(lib.gsx_hip_memcpy_dtod_async(ctypes.c_void_p(tc.data_ptr()), buf.tile_counts, tc.numel() * 4, None))
    torch.cuda.synchronize()
    visible = int((tc > 0).sum().item())
    log(f"train: {it_s:.1f} it/s ({1000.0 / it_s:.3f} ms/step), instances {instances}, visible {visible}")

    # inference forward FPS on the same scene (cycling poses)
    fps_steps = max(args.steps, 20)
    for i in range(3):
        renderer.render(cams[i % args.poses], g, train=False, out_rgb=img)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(fps_steps):
        renderer.render(cams[i % args.poses], g, train=False, out_rgb=img)
    torch.cuda.synchronize()
    fps = fps_steps / (time.perf_counter() - t0)
    log(f"inference forward: {fps:.1f} FPS")

    pixels = H * W
    tiles = int(stats.tile_count)
    kernels = []
    for name, ms in stage_ms.items():
        b = algorithmic_bytes(name, args.gaussians, visible, instances, tiles, pixels, int(stats.sort_passes),
                              int(stats.depth_sort_passes))
        gbps = b / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        kernels.append({"stage": name, "ms": round(ms, 4), "algorithmic_bytes": int(b), "gbps": round(gbps, 1),
                        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)})
    kernels.sort(key=lambda k: -k["ms"])
    dominant = kernels[0]
    sort_entry = next(k for k in kernels if k["stage"] == "sort")
    # the dominant kernel is bound by VALU issue rather than HBM: its wave instructions per launch
    # (committed SQ profile of this workload) over the launch time measured above
    valu_instr = profiled_valu_instructions(STAGE_KERNEL.get(dominant["stage"]))
    valu_issue = None
    if valu_instr is not None and dominant["ms"] > 0:
        rate = valu_instr / (dominant["ms"] * 1e-3) / 1e9
        valu_issue = {"kernel": STAGE_KERNEL.get(dominant["stage"]), "instructions": valu_instr,
                      "achieved": round(rate, 1), "peak": VALU_PEAK_GINSTR, "unit": "G wave-instr/s",
                      "frac": round(rate / VALU_PEAK_GINSTR, 4)}

    result = {
        "metric": "fwd+bwd train iters/sec @1M Gaussians 1920x1080; fwd render FPS; sort GB/s",
        "value": round(it_s, 2),
        "unit": "it/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * elapsed / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded config-3 generator, blurred-noise targets)",
        "config": {"workload": "metric: config-3 generator at N=1M, 1920x1080, f=1600, 24 orbit poses, SH0, "
                               "fwd+bwd+0.8*L1+0.2*(1-SSIM)+Adam",
                   "gaussians": args.gaussians, "width": W, "height": H, "poses": args.poses,
                   "instances_last_pose": instances, "visible_last_pose": visible},
        "train_its_cloned_state": round(it_s_clone, 2),
        "render_fps": round(fps, 1),
        "sort_gbps": sort_entry["gbps"],
        "sort_hbm_frac": sort_entry["hbm_frac"],
        "kernels": kernels,
        "roofline": {"bound": "hbm", "kernel": STAGE_KERNEL.get(dominant["stage"], dominant["stage"]),
                     "achieved": dominant["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": dominant["hbm_frac"], "traffic": measured_traffic(STAGE_KERNEL.get(dominant["stage"])),
                     "algorithmic_bytes": dominant["algorithmic_bytes"], "launch_ms": dominant["ms"]},
        "valu_issue": valu_issue,
        "device": dev_name,
    }

    if args.cpu_baseline_iters > 0:
        log(f"CPU baseline: reference CPU backend, {args.cpu_baseline_iters} step(s) of the full workload, 1 thread")
        block = np.array([1600.0 * W / 1920.0, 1600.0 * W / 1920.0, W / 2.0, H / 2.0, W, H, *scenes.orbit_pose(0),
                          0.01, 100.0, 0, 0, 0], np.float32)
        res = cpu_baseline(base.scene, block, base.target, args.cpu_baseline_iters)
        if res is not None:
            secs, stages, sub_n = res
            result["cpu_baseline"] = {
                "value": round(args.cpu_baseline_iters / secs, 5), "unit": "it/s", "cores": 1, "kind": "reference",
                "sample": f"{args.cpu_baseline_iters} step(s) of the same training step through the unmodified "
                          f"gsx CPU backend (single-threaded by construction) on every {CPU_SAMPLE_STRIDE}th "
                          f"Gaussian of the 1M scene ({sub_n} Gaussians) at the full {W}x{H}, pose 0; the "
                          "full 1M scene exceeds the CPU backend's int32 scratch limit in render backward",
                "seconds_per_step": round(secs / args.cpu_baseline_iters, 3),
                "stage_seconds": {k: round(float(v) / args.cpu_baseline_iters, 3) for k, v in
                                  zip(("render_forward", "loss_forward", "loss_backward", "render_backward",
                                       "adam"), stages)}}
        else:
            result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
