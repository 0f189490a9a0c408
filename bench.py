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
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_bytes(stage, geo, train=True):
    """Minimum HBM bytes of each stage in this build's data layout: every input byte read once and
    every output byte written once, however often the kernel itself touches it (the roofline
    numerators; at or below what the FETCH_SIZE / WRITE_SIZE counters show).
    geo: n Gaussians, Vp past the projection culls (depth-sorted), V of them with at least one
    tile, I instances, T tiles, P pixels, R entries the
    blend must reach (per tile, up to its last contributing entry), U distinct Gaussians among
    them (the touched Gaussians) and It their instances, C transmittance checkpoints the backward
    needs (per pixel, one per 8-entry bucket up to its last contribution), S / D tile- and
    depth-sort passes."""
    n, v, i, t, p = geo["n"], geo["V"], geo["I"], geo["T"], geo["P"]
    vp = geo["Vp"]
    r, u, c = geo["R"], geo["U"], geo["C"]
    if stage == "preprocess":
        # parameters in (SH0: 56 B), the TRAIN snapshot of them out (56 B), tile count + depth key
        # out (12 B); per projected Gaussian its geometry + colour record (48 B) and, TRAIN, the
        # conic-gradient coefficients (32 B)
        return (56 + (56 if train else 0) + 12) * n + (80 if train else 48) * vp
    if stage == "depth_order":
        # depth keys in; the tile counts of the projected ones gathered, their Gaussian and
        # count out in depth order (the intermediate sort passes may stay on chip)
        return 8 * n + 12 * vp
    if stage == "emit":
        # per depth rank: count, Gaussian in, offset out; the geometry record of each Gaussian
        # with tiles in; per instance its tile (4 B) and its Gaussian (4 B) out
        return 12 * vp + 32 * v + 8 * i
    if stage == "sort":
        return sort_bytes(geo["S"], i)
    if stage == "ranges":
        if i >= RANGES_SEARCH_MIN:
            # per tile two binary searches of ceil(log2(I + 1)) 4-byte probes, one range out
            return t * (8 * int(i).bit_length() + 8)
        return 4 * i + 8 * t  # sorted tiles in, one range per tile out
    if stage == "blend_forward":
        # ranges, reached entries' positions + Gaussians in, each reached Gaussian's record once;
        # image (12 B) + final T + last position out; TRAIN: each reached entry's Gaussian and the
        # checkpoints out
        return 8 * t + 8 * r + 48 * u + 20 * p + ((4 * r + 4 * c) if train else 0)
    if stage == "blend_backward":
        # ranges, per pixel the image gradient + final T + last position, the checkpoints, reached
        # entries' positions + Gaussians, each reached Gaussian's record + conic-gradient
        # coefficients once in; a 36-byte partial per reached entry and each tile's cut out; the
        # five parameter gradient sinks zeroed (56 bytes per Gaussian at SH0), which its
        # workgroups store beside their own work
        return 12 * t + 20 * p + 4 * c + 8 * r + 80 * u + 36 * r + 56 * n
    if stage == "instance_reduce":
        # per depth rank its Gaussian, offset and touched flag, the tiles of the touched
        # Gaussians' instances and the reached entries' partials in (the 9-float screen gradients
        # of the touched Gaussians stay in L2 for the projection backward: the counters show no
        # writes, so they are not counted)
        return 9 * vp + 4 * geo["It"] + 36 * r
    if stage == "projection_backward":
        # every Gaussian's touched flag in, the five parameter gradients of the reached Gaussians
        # out (the blend backward has zeroed the others; the reached ones' inputs and screen
        # gradients are read from cache)
        return n + 56 * u
    if stage == "loss_forward":
        # prediction + target in, loss map accumulated (in + out), SSIM workspace (3 floats) out
        return (4 + 4 + 8 + 12) * 3 * p
    if stage == "loss_backward":
        # prediction + target + workspace in, image gradient accumulated (in + out)
        return (4 + 4 + 12 + 8) * 3 * p
    if stage == "adam":
        return 28 * 14 * n  # 14 floats per Gaussian: parameter, m, v in and out, gradient in
    return 0


# instance count from which the ranges come from per-tile binary searches (abi.hip kRangesSearchMin)
RANGES_SEARCH_MIN = 1 << 25


def sort_bytes(passes, instances):
    """Bytes the tile sort moves: per pass each 4-byte tile is read twice (digit counts, then
    scatter) and written once with its 4-byte position; the first pass reads no positions (they
    are the input order), the later ones read them once."""
    if passes <= 0:
        return 0
    return instances * (16 * passes + 4 * (passes - 1))


def render_geometry(lib, renderer, n, width, height):
    """The byte model's per-step quantities, read from the render context's buffers after a
    TRAIN forward + backward (one synchronisation; used between timed steps only)."""
    import torch

    from gsx_amd import _lib
    st = renderer.stats()
    buf = renderer.buffers()
    i_count, t_count, p_count = int(st.instance_count), int(st.tile_count), width * height
    dev = "cuda"

    def pull(ptr_value, count):
        out = torch.empty(count, dtype=torch.int32, device=dev)
        if count > 0:
            _lib.check(lib.gsx_hip_memcpy_dtod_async(ctypes.c_void_p(out.data_ptr()), ptr_value, count * 4, None),
                       "copy render buffer")
        return out

    tc = pull(buf.tile_counts, n)
    rng = pull(buf.tile_ranges, 2 * t_count).view(t_count, 2).long()
    last = pull(buf.last_contributor, p_count).long()
    vals = pull(buf.sorted_values, i_count).long()
    ig = pull(buf.instance_gaussian, i_count).long()
    torch.cuda.synchronize()
    tiles_x = (width + 15) // 16
    pix = torch.arange(p_count, device=dev)
    tile_of = (pix // width // 16) * tiles_x + (pix % width) // 16
    rel = (last - rng[tile_of, 0]).clamp_min(0)
    reach = torch.zeros(t_count, dtype=torch.long, device=dev).scatter_reduce(0, tile_of, rel, "amax")
    r_total = int(reach.sum())
    c_total = int(((rel + 7) // 8).sum())
    u_total = it_total = 0
    if r_total > 0:
        tile_rep = torch.repeat_interleave(torch.arange(t_count, device=dev), reach)
        first = torch.cumsum(reach, 0) - reach
        j = rng[tile_rep, 0] + torch.arange(r_total, device=dev) - first[tile_rep]
        touched = torch.bincount(ig[vals[j]], minlength=n) > 0
        u_total = int(touched.sum())
        it_total = int(tc[touched].long().sum())
    return {"n": n, "Vp": int(st.visible_count), "V": int((tc > 0).sum()), "I": i_count, "T": t_count,
            "P": p_count, "R": r_total,
            "U": u_total, "It": it_total, "C": c_total, "S": int(st.sort_passes), "D": int(st.depth_sort_passes)}


CPU_SAMPLE_STRIDE = 10

STAGE_KERNEL = {"preprocess": "preprocess_kernel", "emit": "emit_kernel", "ranges": "tile_ranges_kernel",
                "blend_forward": "blend_forward_kernel", "blend_backward": "blend_backward_kernel",
                "instance_reduce": "reduce_instance_grads_kernel",
                "projection_backward": "projection_backward_kernel", "loss_forward": "ssim_forward_kernel",
                "loss_backward": "ssim_backward_kernel", "adam": "adam_multi_kernel"}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_metric.txt")
SQ_FILE = os.path.join(ROOT, "profiles", "sq_counters_metric.md")


def _kernel_base(name):
    """A profiled kernel name without its template arguments (ssim_backward_kernel<true> ->
    ssim_backward_kernel): the byte model and the stage map name kernels, not instantiations."""
    return name.split("<", 1)[0]


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (already scaled by the copy-kernel calibration there), or None."""
    if kernel is None or not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 4 and parts[0] == "traffic" and _kernel_base(parts[1]) == kernel:
                return int(float(parts[-1]))
    return None


def profiled_pipe_counters(kernel):
    """VALU busy and LDS bank-conflict percentages of `kernel` (rocprofv3's derived VALUBusy =
    100 SQ_ACTIVE_INST_VALU 4 / SIMDs / GRBM_GUI_ACTIVE and LDSBankConflict = 100
    SQ_LDS_BANK_CONFLICT / GRBM_GUI_ACTIVE / CUs) from the committed SQ summary, or None."""
    if not os.path.exists(SQ_FILE):
        return None
    with open(SQ_FILE) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 3 and _kernel_base(cells[0]) == kernel and cells[1].startswith("pipe"):
                try:
                    return {"valu_busy_pct": float(cells[2]), "lds_bank_conflict_pct": float(cells[3]),
                            "source": os.path.relpath(SQ_FILE, ROOT)}
                except (ValueError, IndexError):
                    return None
    return None


def profiled_valu_instructions(kernel):
    """Wave-level VALU instructions per dispatch of `kernel` (SQ_INSTS_VALU) from the committed SQ
    summary, or None."""
    if not os.path.exists(SQ_FILE):
        return None
    with open(SQ_FILE) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 8 and _kernel_base(cells[0]) == kernel and cells[1] != "pipe":
                try:
                    return int(float(cells[6]))
                except ValueError:
                    return None
    return None


def probe_valu_rate():
    """Wave-level VALU instructions per second of a kernel that does nothing but independent FMAs
    (libgsx_probe.so, 8 waves per SIMD on every SIMD), on this GPU, now; None without the probe."""
    import torch

    from gsx_amd.backend import stream_handle
    path = os.path.join(ROOT, "gsx_amd", "libgsx_probe.so")
    if not os.path.exists(path):
        return None
    plib = ctypes.CDLL(path)
    plib.gsx_probe_valu_fma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    blocks, iters = 2048, 20000
    buf = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    st = stream_handle()
    _probe_check(plib.gsx_probe_valu_fma(blocks, iters, buf.data_ptr(), st))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    _probe_check(plib.gsx_probe_valu_fma(blocks, iters, buf.data_ptr(), st))
    e1.record()
    torch.cuda.synchronize()
    return blocks * 4 * iters * plib.gsx_probe_valu_fma_per_iter() / (e0.elapsed_time(e1) * 1e-3)


def cpu_baseline(scene, camera_block, target, iters):
    """Time the unmodified gsx CPU backend (oracle/_ref) on a bounded sample of the workload:
    every 10th Gaussian of the 1M scene (same distributions) at the full 1920x1080, pose 0, the
    whole step. Then one step of the full 1M scene without the render backward: its near-plane
    Gaussians' pixel boxes cover the image, and the CPU backward's contribution scratch exceeds
    its int32 tensor limit there (gsx-cpu/render.c:1448-1455, gsx-cpu/render.c:167); the render
    forward, both losses and Adam run at full size."""
    import numpy as np

    from gsx_amd import scenes
    from oracle.oracle import Reference
    if not Reference.available():
        return None
    sub = scenes.Scene(*(np.ascontiguousarray(a[::CPU_SAMPLE_STRIDE]) for a in
                         (scene.mean3d, scene.rotation, scene.logscale, scene.opacity, scene.sh0)))
    ref = Reference()
    # the CPU backend runs on this (calling) thread: pin it to one core, as `taskset -c` would,
    # for the timed calls, and restore the mask afterwards
    allowed = sorted(os.sched_getaffinity(0))
    core = allowed[-1]
    os.sched_setaffinity(0, {core})
    try:
        t0 = time.perf_counter()
        _, stages = ref.train_steps(sub, camera_block, target, iters)
        elapsed = time.perf_counter() - t0
        _, full_stages = ref.train_steps(scene, camera_block, target, 1, skip_render_backward=True)
    finally:
        os.sched_setaffinity(0, set(allowed))
    return elapsed, stages, sub.count, full_stages, core, len(allowed)


def host_description():
    """CPU model (/proc/cpuinfo), logical CPUs of the machine and of this process, glibc."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        glibc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        glibc = None
    return {"cpu_model": model, "nproc_machine": os.cpu_count(), "nproc_process": len(os.sched_getaffinity(0)),
            "glibc": glibc}


class TrainRunner:
    """One training step of the metric's sequence (TRAIN render, fused 0.8 L1 + 0.2 (1 - SSIM)
    forward and backward, render backward, Adam over the five SH0 groups) on `gaussians`.
    step(cam, tgt, record=True) also records torch events around the loss and Adam launches
    (their stage times; the render stages are timed by the library's own events)."""

    def __init__(self, lib, gaussians, width, height):
        import numpy as np
        import torch

        from gsx_amd.backend import Adam, Renderer

        self.lib, self.g, self.width, self.height = lib, gaussians, width, height
        self.grads = gaussians.zeros_like_grads()
        self.renderer = Renderer(width, height)
        self.img = torch.empty((3, height, width), dtype=torch.float32, device="cuda")
        # the loss launchers accumulate (+=) into the loss map and the image gradient, so both
        # start each step at zero: one allocation, cleared by one fill
        self.loss_and_grad = torch.empty((2,) + tuple(self.img.shape), dtype=torch.float32, device="cuda")
        self.ssim_ws = torch.empty(3 * self.img.numel(), dtype=torch.float32, device="cuda")
        self.opt = Adam(self.groups_for(gaussians, self.grads))
        self.gs_l1 = float(np.float32(0.8) / np.float32(self.img.numel()))
        self.gs_ssim = float(np.float32(0.2) / np.float32(self.img.numel()))
        self.events = {k: [] for k in ("loss_forward", "loss_backward", "adam")}

    @staticmethod
    def groups_for(g, grads):
        return [dict(parameter=g.mean3d, gradient=grads.mean3d, learning_rate=1e-3),
                dict(parameter=g.logscale, gradient=grads.logscale, learning_rate=1e-2),
                dict(parameter=g.rotation, gradient=grads.rotation, learning_rate=1e-2),
                dict(parameter=g.opacity, gradient=grads.opacity, learning_rate=1e-2),
                dict(parameter=g.sh0, gradient=grads.sh0, learning_rate=1e-2)]

    def step(self, cam, tgt, record=False, borrow=True):
        import torch

        from gsx_amd import _lib
        from gsx_amd.backend import ptr, stream_handle
        lib, h, w = self.lib, self.height, self.width
        loss_map, grad_img = self.loss_and_grad[0], self.loss_and_grad[1]
        st = stream_handle()
        self.renderer.render(cam, self.g, train=True, out_rgb=self.img, borrow_train_state=borrow)
        self.loss_and_grad.zero_()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(5)] if record else None
        if record:
            e[0].record()
        # 0.8 L1 + 0.2 (1 - SSIM), fused in one pass each way (bit-identical to separate calls)
        _lib.check(lib.gsx_hip_loss_ssim_chw_f32_forward_kernel_launch(
            ptr(loss_map), ptr(self.img), ptr(tgt), 1, 3, h, w, 0.2, ptr(self.ssim_ws), 0.8, 1, st), "loss forward")
        if record:
            e[1].record()
        _lib.check(lib.gsx_hip_loss_ssim_chw_f32_backward_kernel_launch(
            ptr(grad_img), ptr(self.img), ptr(tgt), 1, 3, h, w, self.gs_ssim, ptr(self.ssim_ws), self.gs_l1, 1, st),
            "loss backward")
        if record:
            e[2].record()
        self.renderer.backward(grad_img, self.grads)
        if record:
            e[3].record()
        self.opt.step()
        if record:
            e[4].record()
            self.events["loss_forward"].append((e[0], e[1]))
            self.events["loss_backward"].append((e[1], e[2]))
            self.events["adam"].append((e[3], e[4]))

    def stage_pass(self, inputs, first, steps):
        """`steps` steps with HIP events at every stage boundary and the byte model's geometry
        read after each (outside the events): (stage_ms, per-step geometries)."""
        import torch
        for v in self.events.values():
            v.clear()
        self.renderer.set_timing(steps)
        torch.cuda.synchronize()
        geos = []
        for i in range(steps):
            self.step(*inputs[(first + i) % len(inputs)], record=True)
            geos.append(render_geometry(self.lib, self.renderer, self.g.count, self.width, self.height))
        torch.cuda.synchronize()
        stage_ms = self.renderer.timings()
        self.renderer.set_timing(0)
        for k, pairs in self.events.items():
            stage_ms[k] = sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)
        return stage_ms, geos


def stage_table(stage_ms, geos):
    """Per stage: event time, the mean over the same steps of each step's minimum bytes, GB/s
    and fraction of the HBM peak; sorted by time."""
    kernels = []
    for name, ms in stage_ms.items():
        b = sum(algorithmic_bytes(name, gm) for gm in geos) / len(geos)
        gbps = b / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        kernels.append({"stage": name, "ms": round(ms, 4), "algorithmic_bytes": int(b), "gbps": round(gbps, 1),
                        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)})
    kernels.sort(key=lambda k: -k["ms"])
    return kernels


def config_measurement(runner, inputs, warmup, steps):
    """A config's throughput (K steps with nothing else on the stream) and, from K more steps,
    its stage times, minimum bytes per stage, the dominant stage's roofline entry and the step's
    HBM fraction (all stages' minimum bytes over the step time)."""
    ms = 1000.0 * timed_steps(runner.step, inputs, warmup, steps)
    stage_ms, geos = runner.stage_pass(inputs, warmup + steps, steps)
    kernels = stage_table(stage_ms, geos)
    dom = kernels[0]
    step_bytes = sum(k["algorithmic_bytes"] for k in kernels)
    geo_mean = {k: round(sum(gm[k] for gm in geos) / len(geos), 1) for k in geos[0]}
    return {"ms_per_step": round(ms, 3), "it_s": round(1000.0 / ms, 1),
            "stage_ms": {k["stage"]: k["ms"] for k in kernels},
            "kernels": kernels,
            "roofline": {"bound": "hbm", "kernel": STAGE_KERNEL.get(dom["stage"], dom["stage"]),
                         "achieved": dom["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": dom["hbm_frac"],
                         "algorithmic_bytes": dom["algorithmic_bytes"], "launch_ms": dom["ms"]},
            "step_algorithmic_bytes": int(step_bytes),
            "step_hbm_frac": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "mean_per_step": geo_mean}


def timed_steps(step, inputs, warmup, steps):
    import torch
    for i in range(warmup):
        step(*inputs[i % len(inputs)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(*inputs[(warmup + i) % len(inputs)])
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def adc_rows(sc, rng, cap):
    """Density-control rows of a scene in capacity-sized device buffers, with seeded
    statistics (accumulated gradients, absolute gradients, visibility counts) and zero Adam
    moments: (fields, moments, host copies to restore from)."""
    import numpy as np
    import torch
    n = sc.count
    host = {"mean3d": sc.mean3d, "rotation": sc.rotation, "logscale": sc.logscale, "opacity": sc.opacity,
            "sh0": sc.sh0, "grad_acc": (rng.random(n) * 2e-3).astype(np.float32),
            "absgrad_acc": (rng.random(n) * 8e-3).astype(np.float32),
            "visible_counter": rng.integers(0, 20, n).astype(np.float32)}
    d = {k: torch.zeros((cap, ADC_WIDTHS[k]) if ADC_WIDTHS[k] > 1 else (cap,), dtype=torch.float32, device="cuda")
         for k in host}
    src = {k: torch.from_numpy(v.reshape(n, ADC_WIDTHS[k]) if ADC_WIDTHS[k] > 1 else v).cuda()
           for k, v in host.items()}
    moms = {k: (torch.zeros_like(d[k]), torch.zeros_like(d[k])) for k in PARAM_ROLES}
    return d, moms, src


ADC_WIDTHS = {"mean3d": 3, "rotation": 4, "logscale": 3, "opacity": 1, "sh0": 3, "grad_acc": 1, "absgrad_acc": 1,
              "visible_counter": 1}
PARAM_ROLES = ("mean3d", "rotation", "logscale", "opacity", "sh0")
ADC_COMMON = dict(pruning_opacity_threshold=0.05, opacity_clamp_value=0.3, max_world_scale=0.5,
                  duplicate_grad_threshold=2e-4, duplicate_scale_threshold=0.01, scene_scale=4.0, refine_every=100,
                  start_refine=0, end_refine=1000, reset_every=0)


def time_refine(sc, params, cap, seed, reps=3):
    """One density-control refine of `sc`'s rows (moments included), timed `reps` times from
    the same uploaded state after one untimed call; the upload is outside the timed region."""
    import numpy as np
    import torch

    from gsx_amd.backend import DensityControl
    n = sc.count
    d, moms, src = adc_rows(sc, np.random.default_rng(7), cap)
    o = {k: torch.zeros_like(v) for k, v in d.items()}
    om = {k: (torch.zeros_like(a), torch.zeros_like(b)) for k, (a, b) in moms.items()}
    adc = DensityControl({**ADC_COMMON, **params, "max_num_gaussians": cap}, seed=seed)
    times = []
    for rep in range(reps + 1):
        for k in d:
            d[k][:n].copy_(src[k])
        for a, b in moms.values():
            a.zero_()
            b.zero_()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        count, _, counts = adc.step(100, n, 0, d, moms, cap, o, om)
        torch.cuda.synchronize()
        if rep > 0:
            times.append(1000.0 * (time.perf_counter() - t0))
    adc.close()
    return {"rows_before": n, "rows_after": int(count), "ms": round(sum(times) / len(times), 3),
            "counts_pruned_duplicated_grown_reset": [int(c) for c in counts]}


def c4_refine_loop(lib, iters=500, every=100):
    """Config 4 as the config states it: `iters` training steps on the 6M scene at 1080p with an
    ABSGS refine (clone / split / prune, moments included) after every `every`-th step, timed
    end to end. The renderer and Adam run on the current rows of capacity-sized buffers; each
    refine reads seeded accumulated absolute gradients and visibility counts (the CPU backend's
    backward leaves the accumulators to the caller), and its result becomes the next steps'
    Gaussian set and Adam state."""
    import numpy as np
    import torch

    from gsx_amd import scenes
    from gsx_amd.backend import Camera, DensityControl, GaussianTensors
    w = scenes.config4()
    n0 = w.scene.count
    cap = n0 + n0 // 2
    rng = np.random.default_rng(44)
    bufs = [adc_rows(w.scene, rng, cap)[:2], None]
    bufs[1] = ({k: torch.zeros_like(v) for k, v in bufs[0][0].items()},
               {k: (torch.zeros_like(a), torch.zeros_like(b)) for k, (a, b) in bufs[0][1].items()})
    for k in bufs[0][0]:
        src = getattr(w.scene, k, None)
        if src is not None:
            bufs[0][0][k][:n0].copy_(torch.from_numpy(src.reshape(n0, -1) if ADC_WIDTHS[k] > 1 else src))
    adc = DensityControl({**ADC_COMMON, "algorithm": 1, "duplicate_absgrad_threshold": 4e-4,
                          "max_num_gaussians": cap, "start_refine": every, "end_refine": iters + 1}, seed=9)
    cam = Camera.from_block(w.camera)
    tgt = torch.from_numpy(w.target).cuda()
    cur, count = 0, n0
    counts_log = []

    def bind(count, cur):
        f, m = bufs[cur]
        view = lambda t: t[:count]  # noqa: E731
        g = GaussianTensors(*(view(f[k]) for k in PARAM_ROLES))
        runner.g = g
        runner.grads = g.zeros_like_grads()
        runner.opt.groups = [dict(grp, parameter=getattr(g, k), gradient=getattr(runner.grads, k),
                                  m=view(m[k][0]), v=view(m[k][1]))
                             for grp, k in zip(runner.opt.groups, ("mean3d", "logscale", "rotation", "opacity",
                                                                    "sh0"))]

    f0 = bufs[0][0]
    runner = TrainRunner(lib, GaussianTensors(*(f0[k][:n0] for k in PARAM_ROLES)), 1920, 1080)
    bind(count, cur)
    runner.step(cam, tgt)  # warm-up: buffers sized for the first step's instances
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for it in range(1, iters + 1):
        runner.step(cam, tgt)
        if it % every == 0:
            f, m = bufs[cur]
            # the refine's statistics: seeded, as BASELINE config 4 states
            f["absgrad_acc"][:count].uniform_(0.0, 8e-3)
            f["grad_acc"][:count].uniform_(0.0, 2e-3)
            f["visible_counter"][:count].random_(0, 20)
            o, om = bufs[1 - cur]
            new_count, in_out, counts = adc.step(it, count, 0, f, m, cap, o, om)
            counts_log.append([int(c) for c in counts])
            if in_out:
                cur = 1 - cur
            count = new_count
            bind(count, cur)
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    adc.close()
    return {"gaussians_start": n0, "gaussians_end": int(count), "iterations": iters, "refine_every": every,
            "seconds": round(secs, 3), "ms_per_iteration": round(1000.0 * secs / iters, 3),
            "it_s": round(iters / secs, 2), "refine_counts_pruned_duplicated_grown_reset": counts_log}


def extra_workloads(lib, steps, only=None):
    """Throughput of the other BASELINE configs at their stated sizes (one GPU) with per-stage
    times and rooflines, the tile sort's bandwidth on config 4's instances, config 4's
    500-iteration loop with its refines, and density-control refines at 1M and 6M rows."""
    import torch

    out = {}

    def want(name):
        return only is None or only == name

    # config 2: image fit, 1M Gaussians on z = 0, 1024^2, one camera
    if want("c2"):
        out.update(_config2(lib, steps))
    if want("c3"):
        out.update(_config3(lib, steps))
    if want("c4"):
        out.update(_config4(lib, steps))
    if want("c4loop"):
        out["c4_refine_loop"] = c4_refine_loop(lib)
        torch.cuda.empty_cache()
        log(f"config 4 loop: {out['c4_refine_loop']}")
    if want("adc"):
        out.update(_refines())
    if only == "gather32":  # a probe for profiling, not part of the default line
        out["gather32"] = gather32_probe(lib, steps)
    if only == "probes":  # calibration kernels for profiling, not part of the default line
        out["probes"] = calibration_probes()
    return out


def calibration_probes():
    """Kernels of known work from libgsx_probe.so, timed with HIP events on torch's stream:
    - valu_fma: 16 independent FMAs per loop step per lane on the scalar loop counter, at 4 and 8
      waves per SIMD; the time gives the cycles one wave-level VALU instruction occupies a SIMD
      (at the 2.4 GHz peak engine clock), and under rocprofv3 --pmc the counters' reading of a
      kernel that does nothing but VALU work;
    - store_zero: 16-byte zero stores over 56 MB (the metric's five SH0 parameter gradients,
      the projection backward's writes) and 336 MB (config 4's), beside torch's fill of the same
      bytes: the store-only floor of those sizes."""
    import torch

    from gsx_amd.backend import stream_handle
    plib = ctypes.CDLL(os.path.join(ROOT, "gsx_amd", "libgsx_probe.so"))
    plib.gsx_probe_valu_fma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    plib.gsx_probe_store_zero.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    st = stream_handle()
    out = {"engine_clock_ghz_assumed": 2.4, "simds": 1024}

    def timed(fn, reps):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    iters = 20000
    per_iter = plib.gsx_probe_valu_fma_per_iter()
    rows = []
    for waves_per_simd in (4, 8):
        blocks = 256 * waves_per_simd  # 4 waves per workgroup, 4 SIMDs per CU, 256 CUs
        buf = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
        ms = timed(lambda: _probe_check(plib.gsx_probe_valu_fma(blocks, iters, buf.data_ptr(), st)), 3)
        instr = blocks * 4 * iters * per_iter
        cycles = ms * 1e-3 * 2.4e9 * 1024 / instr
        rows.append({"waves_per_simd": waves_per_simd, "blocks": blocks, "iters": iters,
                     "wave_valu_instructions": instr, "ms": round(ms, 4),
                     "simd_cycles_per_wave_instruction": round(cycles, 3)})
        log(f"valu probe: {rows[-1]}")
    out["valu_fma"] = rows
    stores = []
    for mb, label in ((56, "metric projection backward"), (336, "config 4 projection backward")):
        count = mb * 1_000_000 // 4
        buf = torch.empty(count, dtype=torch.float32, device="cuda")
        row = {"bytes": mb * 1_000_000, "sinks_of": label}
        for blocks in (2048, 4096, 16384):
            ms = timed(lambda: _probe_check(plib.gsx_probe_store_zero(buf.data_ptr(), count, blocks, st)), 20)
            row[f"store_zero_{blocks}wg_us"] = round(ms * 1e3, 2)
        ms = timed(lambda: buf.zero_(), 20)
        row["torch_zero_us"] = round(ms * 1e3, 2)
        best = min(v for k, v in row.items() if k.endswith("_us"))
        row["best_gbps"] = round(row["bytes"] / (best * 1e-6) / 1e9, 1)
        stores.append(row)
        log(f"store probe: {row}")
        del buf
    out["store_zero"] = stores
    return out


def _probe_check(rc):
    if rc != 0:
        raise RuntimeError(f"probe launch failed: hipError {rc}")


def gather32_probe(lib, steps, rows=1_000_000, count=579_321):
    """The floor of emission's record reads: gsx_hip_gather_rows_kernel_launch moving `count`
    random 32-byte rows out of `rows` (the metric scene's Gaussians and its projected count, the
    geometry records emission gathers in depth order), `steps` launches timed with HIP events.
    Profiled under FETCH_SIZE / WRITE_SIZE, it shows the bytes a random 32-byte read costs."""
    import numpy as np
    import torch

    from gsx_amd import _lib
    from gsx_amd.backend import ptr, stream_handle
    src = torch.rand((rows, 8), dtype=torch.float32, device="cuda")
    dst = torch.empty((count, 8), dtype=torch.float32, device="cuda")
    idx = torch.from_numpy(np.random.default_rng(5).permutation(rows)[:count].astype(np.int32)).cuda()
    st = stream_handle()
    for _ in range(3):
        _lib.check(lib.gsx_hip_gather_rows_kernel_launch(ptr(src), ptr(dst), 32, count, ptr(idx), rows, None, st),
                   "gather")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        _lib.check(lib.gsx_hip_gather_rows_kernel_launch(ptr(src), ptr(dst), 32, count, ptr(idx), rows, None, st),
                   "gather")
    e1.record()
    torch.cuda.synchronize()
    assert torch.equal(dst, src[idx.long()])
    ms = e0.elapsed_time(e1) / steps
    moved = count * (32 + 32 + 4)  # row read, row written, index read
    return {"rows": rows, "count": count, "row_bytes": 32, "ms": round(ms, 4),
            "algorithmic_bytes": moved, "gbps": round(moved / (ms * 1e-3) / 1e9, 1)}


def _config2(lib, steps):
    import torch

    from gsx_amd import scenes
    from gsx_amd.backend import Camera, GaussianTensors
    out = {}
    w = scenes.config2()
    runner = TrainRunner(lib, GaussianTensors.from_scene(w.scene), 1024, 1024)
    inputs = [(Camera.from_block(w.camera), torch.from_numpy(w.target).cuda())]
    out["c2_image_fit"] = {"gaussians": w.scene.count, "width": 1024, "height": 1024,
                           **config_measurement(runner, inputs, 3, steps),
                           "instances": int(runner.renderer.stats().instance_count)}
    del runner, inputs
    log(f"config 2: {out['c2_image_fit']['it_s']} it/s, stages {out['c2_image_fit']['stage_ms']}")
    return out


def _config3(lib, steps):
    import torch

    from gsx_amd import scenes
    from gsx_amd.backend import Camera, GaussianTensors
    out = {}
    # config 3: 3M Gaussians, 1080p, 24 orbit poses
    base = scenes.config3()
    runner = TrainRunner(lib, GaussianTensors.from_scene(base.scene), 1920, 1080)
    inputs = []
    for k in range(24):
        block = scenes.camera(1920, 1080, 1600.0, pose=tuple(scenes.orbit_pose(k)), near=0.01, far=100.0)
        tgt = base.target if k == 0 else scenes.target_image(0, 103 + k, 1920, 1080, 2)
        inputs.append((Camera.from_block(block), torch.from_numpy(tgt).cuda()))
    out["c3_scene_training"] = {"gaussians": base.scene.count, "width": 1920, "height": 1080, "poses": 24,
                                **config_measurement(runner, inputs, 2, steps)}
    del runner, inputs, base
    log(f"config 3: {out['c3_scene_training']['it_s']} it/s, stages {out['c3_scene_training']['stage_ms']}")
    return out


def _config4(lib, steps):
    import torch

    from gsx_amd import scenes
    from gsx_amd.backend import Camera, GaussianTensors
    out = {}
    # config 4: 6M Gaussians, 1080p, the sort / blend stress
    w = scenes.config4()
    runner = TrainRunner(lib, GaussianTensors.from_scene(w.scene), 1920, 1080)
    inputs = [(Camera.from_block(w.camera), torch.from_numpy(w.target).cuda())]
    c4 = config_measurement(runner, inputs, 1, max(2, steps // 4))
    st = runner.renderer.stats()
    inst = int(st.instance_count)
    moved = sort_bytes(int(st.sort_passes), inst)
    sort_ms = c4["stage_ms"]["sort"]
    out["c4_sort_stress"] = {"gaussians": w.scene.count, "width": 1920, "height": 1080, **c4, "instances": inst,
                             "sort_passes": int(st.sort_passes),
                             "sort_gbps": round(moved / (sort_ms * 1e-3) / 1e9, 1),
                             "sort_hbm_frac": round(moved / (sort_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                             "sort_gkeys_s": round(inst / (sort_ms * 1e-3) / 1e9, 2)}
    del runner, inputs, w
    torch.cuda.empty_cache()
    log(f"config 4: {out['c4_sort_stress']['it_s']} it/s, sort {out['c4_sort_stress']['sort_hbm_frac']} of HBM")
    return out


def _refines():
    import torch

    from gsx_amd import scenes
    out = {}
    # density control: one ABSGS refine (prune + duplicate + split) at 1M rows (the metric
    # scene) and at config 4's 6M, one MCMC refine (relocation + 10% growth) at 1M
    sc1 = scenes.metric_scene().scene
    out["absgs_refine"] = time_refine(sc1, dict(algorithm=1, duplicate_absgrad_threshold=4e-4),
                                      sc1.count + sc1.count // 5, 3)
    out["mcmc_refine"] = time_refine(sc1, dict(algorithm=2, grow_ratio=0.1, noise_strength=50.0,
                                               mean3d_learning_rate=1e-3), sc1.count + sc1.count // 5, 3)
    sc4 = scenes.config4().scene
    out["absgs_refine_c4"] = time_refine(sc4, dict(algorithm=1, duplicate_absgrad_threshold=4e-4),
                                         sc4.count + sc4.count // 5, 3)
    for k in ("absgs_refine", "mcmc_refine", "absgs_refine_c4"):
        log(f"{k}: {out[k]}")
    torch.cuda.empty_cache()
    return out


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
    ap.add_argument("--fps-steps", type=int, default=-1,
                    help="inference renders timed for render_fps (default max(steps, 20); 0 skips them)")
    ap.add_argument("--extra-steps", type=int, default=10,
                    help="timed steps of the config 2/3/4 and density-control lines (0 disables them)")
    ap.add_argument("--only", choices=("c2", "c3", "c4", "c4loop", "adc", "gather32", "probes"), default=None,
                    help="run just one of the config workloads (for profiling) and print its JSON")
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
    if args.calibrate_copy_mib > 0:
        nf = args.calibrate_copy_mib * (1 << 20) // 4
        a = torch.ones(nf, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        _lib.check(lib.gsx_hip_copy_f32(ptr(b), ptr(a), nf, stream_handle()), "calibration copy")
        torch.cuda.synchronize()
        log(f"calibration copy: {args.calibrate_copy_mib} MiB read + {args.calibrate_copy_mib} MiB written")
        del a, b
    if args.only is not None:
        print(json.dumps({"workload": args.only, "device": dev_name,
                          **extra_workloads(lib, args.steps, only=args.only)}), flush=True)
        return
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
    geos = []
    for i in range(args.steps):
        step(args.warmup + i, record=True)  # the poses of pass 1 again
        # the byte model's inputs of this step (buffer reads outside the stage events)
        geos.append(render_geometry(lib, renderer, args.gaussians, W, H))
    torch.cuda.synchronize()
    stage_ms = renderer.timings()
    renderer.set_timing(0)
    for k, pairs in ev.items():
        stage_ms[k] = sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)
    geo_mean = {k: sum(gm[k] for gm in geos) / len(geos) for k in geos[0]}
    instances = geos[-1]["I"]
    visible = geos[-1]["V"]
    log(f"train: {it_s:.1f} it/s ({1000.0 / it_s:.3f} ms/step), instances {instances}, visible {visible}, "
        f"reached {geos[-1]['R']}, distinct reached {geos[-1]['U']} (last pose)")

    # inference forward FPS on the same scene (cycling poses)
    fps_steps = max(args.steps, 20) if args.fps_steps < 0 else args.fps_steps
    fps = None
    if fps_steps > 0:
        for i in range(3):
            renderer.render(cams[i % args.poses], g, train=False, out_rgb=img)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(fps_steps):
            renderer.render(cams[i % args.poses], g, train=False, out_rgb=img)
        torch.cuda.synchronize()
        fps = fps_steps / (time.perf_counter() - t0)
        log(f"inference forward: {fps:.1f} FPS")

    kernels = stage_table(stage_ms, geos)
    dominant = kernels[0]
    sort_entry = next(k for k in kernels if k["stage"] == "sort")
    # the blend kernels are bound by the vector ALU and LDS rather than HBM: rocprofv3's VALU busy
    # and LDS bank-conflict shares from the committed SQ profile of this workload, and the VALU
    # issue rate (the profile's instructions per dispatch over this run's launch time) against the
    # rate of a kernel that does nothing but VALU work, timed now (rocprofv3's VALUBusy assumes 4
    # cycles per wave-level instruction, which part of the blend kernels' instructions undercut,
    # so it reads above 100)
    pipe = {k: profiled_pipe_counters(k) for k in ("blend_forward_kernel", "blend_backward_kernel")}
    probe_rate = probe_valu_rate()
    for k, stage in (("blend_forward_kernel", "blend_forward"), ("blend_backward_kernel", "blend_backward")):
        instr = profiled_valu_instructions(k)
        ms = next((x["ms"] for x in kernels if x["stage"] == stage), None)
        if pipe[k] is not None and instr is not None and ms:
            rate = instr / (ms * 1e-3)
            pipe[k].update({"valu_instructions_per_launch": instr, "valu_issue_g_per_s": round(rate / 1e9, 1)})
            if probe_rate:
                pipe[k].update({"probe_valu_g_per_s": round(probe_rate / 1e9, 1),
                                "valu_issue_vs_probe": round(rate / probe_rate, 3)})

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
                   "instances_last_pose": instances, "visible_last_pose": visible,
                   "mean_per_step": {k: round(v, 1) for k, v in geo_mean.items()}},
        "train_its_cloned_state": round(it_s_clone, 2),
        "render_fps": round(fps, 1) if fps is not None else None,
        "sort_gbps": sort_entry["gbps"],
        "sort_hbm_frac": sort_entry["hbm_frac"],
        # sorted (tile, position) pairs per second over the same steps
        "sort_gkeys_s": round(geo_mean["I"] / (sort_entry["ms"] * 1e-3) / 1e9, 2),
        "kernels": kernels,
        "roofline": {"bound": "hbm", "kernel": STAGE_KERNEL.get(dominant["stage"], dominant["stage"]),
                     "achieved": dominant["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": dominant["hbm_frac"], "traffic": measured_traffic(STAGE_KERNEL.get(dominant["stage"])),
                     "algorithmic_bytes": dominant["algorithmic_bytes"], "launch_ms": dominant["ms"]},
        "blend_pipeline": pipe,
        "device": dev_name,
    }

    if args.extra_steps > 0:
        del renderer, g, grads, opt
        torch.cuda.empty_cache()
        result["workloads"] = extra_workloads(lib, args.extra_steps)

    if args.cpu_baseline_iters > 0:
        log(f"CPU baseline: reference CPU backend, {args.cpu_baseline_iters} step(s) of the full workload, 1 thread")
        block = np.array([1600.0 * W / 1920.0, 1600.0 * W / 1920.0, W / 2.0, H / 2.0, W, H, *scenes.orbit_pose(0),
                          0.01, 100.0, 0, 0, 0], np.float32)
        res = cpu_baseline(base.scene, block, base.target, args.cpu_baseline_iters)
        if res is not None:
            secs, stages, sub_n, full_stages, core, allowed = res
            result["cpu_baseline"] = {
                "value": round(args.cpu_baseline_iters / secs, 5), "unit": "it/s", "cores": 1, "kind": "reference",
                "pinned_core": core, "host": {**host_description(), "nproc_process": allowed},
                "sample": f"{args.cpu_baseline_iters} step(s) of the same training step through the unmodified "
                          f"gsx CPU backend (single-threaded by construction) on every {CPU_SAMPLE_STRIDE}th "
                          f"Gaussian of the 1M scene ({sub_n} Gaussians) at the full {W}x{H}, pose 0; the "
                          "full 1M scene exceeds the CPU backend's int32 scratch limit in render backward",
                "seconds_per_step": round(secs / args.cpu_baseline_iters, 3),
                "stage_seconds": {k: round(float(v) / args.cpu_baseline_iters, 3) for k, v in
                                  zip(("render_forward", "loss_forward", "loss_backward", "render_backward",
                                       "adam"), stages)},
                "full_scene_stage_seconds": {
                    k: round(float(v), 3) for k, v in zip(("render_forward", "loss_forward", "loss_backward",
                                                           "adam"), full_stages[[0, 1, 2, 4]])},
                "full_scene_note": f"one step of the full {base.scene.count}-Gaussian scene at {W}x{H}, pose 0, "
                                   "without the render backward (Adam on zero gradients)"}
        else:
            result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
