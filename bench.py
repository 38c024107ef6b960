#!/usr/bin/env python3
"""Headline benchmark: forward + backward of the splatting hot path on one MI355X.

Workload: 1.18M synthetic gaussians, 979x546 pinhole camera (fx = fy = 580),
128 fp32 feature channels, inputs resident in HBM. One step is what the reference's harness times
(bench/harness.py:59-66, 157-177; README scope "projection, binning and blending of the RGB image plus
the feature image"): normalize(quats) -> project_gaussians -> rasterize(features=F) forward, then
autograd backward of dL/dimage and dL/dfeature_image (both U[0, 1]) through the blend and the
projection. Colours are a leaf, as in the harness, so SH is not in the timed region.

Prints ONE JSON line: the metric (ms per fwd+bwd, lower is better), the fwd / bwd split measured the
harness way (events around each sample, a pause after each, median; bench/harness.py:130-153), per-stage
HIP-event timings taken inside the timed region, the roofline of the dominant kernel (render_backward)
against MI355X HBM (8 TB/s), a CPU baseline: the oracle (oracle/hds_oracle.c, OpenMP) running the same
frame on this host, the median of --cpu-samples runs with its fwd / bwd split and the host (logical
CPUs, usable CPUs, OpenMP threads, CPU model), and the environment (GPU, clocks and power from amd-smi,
source digest). After the headline it times, on the same GPU, the channel sweep (
C = 32, 64, 256, 512 on the headline scene) and configs 0, 1 and 4 (their step, fwd / bwd split, blend
backward span and per-stage means), each with the oracle's CPU figure on the same frame beside it
(config 4's on the 64 tiles its parity test compares, labelled; config 0's also with the dense float64
blend, timed once), reported under 'channel_sweep' and 'other_configs', and one iteration of the reference's
training loop on the headline scene (main.py:159-200, SH and the optimizer step included), reported
under 'training_iteration'.

Like the reference harness, which times only what agrees with its comparison (harness.py:196-208), it
first checks one fwd+bwd step of this frame against the oracle (images and every leaf gradient within
the parity tests' bars) and refuses to time a build that disagrees (exit status 1, value null).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "high-dimensional-splatting_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd+bwd ms at 1.18M gaussians, 979x546, C=128; fraction of HBM roofline"
HBM_PEAK_GBS = 8000.0


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50, help="timed fwd+bwd steps")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, help="BASELINE.json config index (0-4)")
    ap.add_argument("--channels", type=int, default=None, help="override the config's feature width")
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU oracle (its timing and the agreement check it provides)")
    ap.add_argument("--cpu-samples", type=int, default=5,
                    help="oracle fwd+bwd runs per CPU figure (median; config 4's masked frame takes at most 3)")
    ap.add_argument("--no-split", action="store_true", help="skip the separate fwd / bwd median timing")
    ap.add_argument("--breakdown-steps", type=int, default=10,
                    help="steps after the timed region with events around every call and kernel, for the "
                         "per-stage and per-kernel figures")
    ap.add_argument("--frozen-features", action="store_true",
                    help="features without requires_grad: the backward keeps the feature term of the geometry "
                         "gradients but writes no grad_features (reference test_render.py:118-134)")
    ap.add_argument("--rgb-only", action="store_true", help="render RGB without features (features=None)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB device to device once: the plain copy "
                         "kernel whose FETCH_SIZE / WRITE_SIZE calibrate the --pmc traffic figures")
    ap.add_argument("--checkpoint", type=Path, default=None,
                    help="model.pt in the reference's layout (main.py:86-94): render its gaussians instead of the "
                         "synthetic config, with features U[0, 1] as bench/harness.py:46 does (needs --camera)")
    ap.add_argument("--camera", type=Path, default=None,
                    help="JSON camera for --checkpoint (gaussian_splatting.utils.checkpoint.load_camera)")
    ap.add_argument("--loss", choices=("auto", "none", "l1-ssim"), default="auto",
                    help="l1-ssim: the image gradient comes from 0.8 L1 + 0.2 (1 - SSIM) against a U[0, 1] target "
                         "(main.py:179-182), run through the SSIM kernels inside the step; none: dL/dimage U[0, 1] as "
                         "bench/harness.py:49 does; auto: l1-ssim for configs 0 and 4, whose BASELINE definition "
                         "includes the loss, none otherwise")
    ap.add_argument("--bwd-slice", type=int, default=None,
                    help="channels per backward work-group (gaussian_splatting.rasterizer.FEATURE_SLICE_WIDTH)")
    ap.add_argument("--train", choices=("auto", "on", "off"), default="auto",
                    help="also time a training iteration of the reference's loop (main.py:159-200) on the headline "
                         "scene and report it under 'training_iteration'; auto: on for the default run, off under a "
                         "profiler")
    ap.add_argument("--configs", default="auto",
                    help="comma-separated other BASELINE configs timed after the headline on the same GPU (step, "
                         "fwd / bwd split, blend backward span, per-stage ms) and reported under 'other_configs'; "
                         "'auto' = 0,1,4 for config 2 (none under a profiler), none otherwise; 'none' skips them")
    ap.add_argument("--sweep", default="auto",
                    help="comma-separated channel counts of BASELINE config 3 timed after the headline on the same "
                         "scene (fwd / bwd ms, backward roofline) and reported under 'channel_sweep'; 'auto' = "
                         "32,64,256,512 for config 2, none otherwise; 'none' skips it")
    args = ap.parse_args()
    if (args.checkpoint is None) != (args.camera is None):
        ap.error("--checkpoint and --camera go together")
    return args


def checkpoint_workload(checkpoint: Path, camera: Path, channels: int | None):
    """The frame bench/harness.py:33-56 renders: a trained model's activated gaussians (exp scales,
    sigmoid opacities, the raw quats as the leaf) seen from one camera, its SH at the checkpoint's
    active degree, and `channels` (default 128) features U[0, 1] from a seeded generator."""
    import torch

    from gaussian_splatting.utils.checkpoint import load_camera, load_checkpoint
    from tests.scenes import Workload

    ckpt, view = load_checkpoint(checkpoint), load_camera(camera)
    c = 128 if channels is None else channels
    features = torch.rand(ckpt.n, c, generator=torch.Generator().manual_seed(0))
    name = f"checkpoint-{checkpoint.stem}-{view.name or 'view'}-{ckpt.n}-{view.width}x{view.height}-c{c}"
    return Workload(name, ckpt.n, view.width, view.height, view.fx, c, ckpt.means, ckpt.scales,
                    ckpt.params["quats"], ckpt.opacities, ckpt.params["sh_dc"], ckpt.params["sh_rest"], features,
                    w2c=view.world_to_camera, intrinsics=(view.fx, view.fy, view.cx, view.cy),
                    sh_degree=ckpt.active_sh_degree)


def algorithmic_bytes(n: int, n_vis: int, pairs: int, hw: int, c: int) -> dict[str, float]:
    """Minimal unique HBM bytes per stage (fp32), the roofline denominators: each input read once,
    each output written once (gradient outputs counted once, not as zero-fill + read-modify-write).
    Binning: bin_count = the tile counts and their scan (12 B per gaussian); bin_emit = writing the
    pairs (12 B), one read + write of keys and values for a one-pass sort (24 B) and the range build's
    read (8 B), per pair; bin = both, for the one-call tile-order binning."""
    return {
        "project_forward": 44 * n + 28 * n,
        "bin_count": 12 * n,
        "bin_emit": 44 * pairs,
        "bin": 12 * n + 44 * pairs,
        "render": 4 * pairs + 36 * n_vis + 4 * c * n_vis + 20 * hw + 4 * c * hw,
        "render_backward": 20 * hw + 4 * pairs + 36 * n_vis + 4 * c * n_vis + 4 * c * hw + 4 * c * n + 36 * n,
        "project_backward": 60 * n + 40 * n,
    }


class Frame:
    """One frame as the timed step runs it (bench/harness.py:33-66, 157-177): the leaves (means,
    scales, quats, opacities, colours evaluated once from SH under no_grad, features), dL/dimage and
    dL/dfeature_image ~ U[0, 1], and the step's closures: normalize(quats) -> project_gaussians ->
    rasterize, then autograd backward, of 0.8 L1 + 0.2 (1 - SSIM) against the U[0, 1] image
    (main.py:179-182) when loss_mode is "l1-ssim", else of the upstream gradients."""

    def __init__(self, wl, dev, loss_mode: str, rgb_only: bool = False, frozen_features: bool = False):
        import torch

        from gaussian_splatting.rasterizer import project_gaussians
        from gaussian_splatting.utils.sh import eval_sh
        from tests.scenes import upstream, view_dirs

        self.wl, self.rgb_only = wl, rgb_only
        cam = wl.cam
        wl_dev = wl.to(dev)
        self.w2c = wl_dev.world_to_camera.contiguous()
        with torch.no_grad():
            _, _, radii0, _ = project_gaussians(wl_dev.means, wl_dev.scales, wl_dev.quats, wl_dev.opacities, self.w2c,
                                                cam["fx"], cam["fy"], cam["cx"], cam["cy"], wl.width, wl.height)
            self.colors = eval_sh(wl_dev.sh_dc, wl_dev.sh_rest, view_dirs(wl_dev.means, wl_dev.center), wl.sh_degree,
                                  radii0, None)
        self.leaves = {
            "means": wl_dev.means.clone().requires_grad_(True),
            "scales": wl_dev.scales.clone().requires_grad_(True),
            "quats": wl_dev.quats.clone().requires_grad_(True),
            "opacities": wl_dev.opacities[:, 0].clone().requires_grad_(True),
            "colors": self.colors.clone().requires_grad_(True),
            "features": wl_dev.features.clone().requires_grad_(not frozen_features),
        }
        if rgb_only:
            del self.leaves["features"]
        self.grad_image, self.grad_features = upstream(2, wl.height, wl.width, wl.channels, device=dev)
        self.target = self.grad_image if loss_mode == "l1-ssim" else None
        self.state = {}

    def forward(self, retain: bool = False) -> None:
        import torch.nn.functional as F

        from gaussian_splatting.rasterizer import project_gaussians, rasterize

        leaves, cam, W, H = self.leaves, self.wl.cam, self.wl.width, self.wl.height
        means2D, depths, radii, conics = project_gaussians(
            leaves["means"], leaves["scales"], F.normalize(leaves["quats"], dim=-1), leaves["opacities"][:, None],
            self.w2c, cam["fx"], cam["fy"], cam["cx"], cam["cy"], W, H)
        if retain:
            # The rasterizer's own gradients (the agreement gate compares each stage on its inputs).
            means2D.retain_grad()
            conics.retain_grad()
            self.state["means2D"], self.state["conics"] = means2D, conics
            self.state["projected"] = (means2D, depths, radii, conics)
        self.state["out"] = rasterize(means2D, depths, radii, conics, leaves["colors"], leaves["opacities"][:, None],
                                      W, H, features=leaves.get("features"))

    def backward(self) -> None:
        import torch

        from gaussian_splatting.utils.loss import l1_loss, ssim

        out = self.state["out"]
        image = out if self.rgb_only else out[0]
        if self.target is not None:
            # main.py:179-182: 0.8 L1 + 0.2 (1 - SSIM), the SSIM on the fused HIP kernels.
            loss = 0.8 * l1_loss(image, self.target) + 0.2 * (1.0 - ssim(image, self.target))
            if self.rgb_only:
                loss.backward()
            else:
                torch.autograd.backward([loss, out[1]], [None, self.grad_features])
        elif self.rgb_only:
            torch.autograd.backward(out, self.grad_image)
        else:
            torch.autograd.backward(out, [self.grad_image, self.grad_features])

    def reset(self) -> None:
        for leaf in self.leaves.values():
            leaf.grad = None

    def step(self) -> None:
        self.reset()
        self.forward()
        self.backward()


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the rasterizer path has no multi-GPU mode in this build (it would "
              "shard over feature channels, with one all-reduce of the geometry gradients). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    import torch.nn.functional as F

    from gaussian_splatting.rasterizer import _get_rasterizer, project_gaussians
    from gaussian_splatting.rasterizer._native import KernelProfile, StageTimer
    from tests.scenes import synthetic_config

    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.checkpoint is not None:
        wl = checkpoint_workload(args.checkpoint, args.camera, args.channels)
    else:
        wl = synthetic_config(args.config, channels=args.channels)
    cam = wl.cam
    W, H, C, N = wl.width, wl.height, wl.channels, wl.n
    print(f"[bench] {wl.name}: N={N} {W}x{H} C={C}", file=sys.stderr, flush=True)
    # With the loss, the U[0, 1] image drawn as dL/dimage is the target and dL/dimage comes from the loss.
    loss_mode = args.loss if args.loss != "auto" else ("l1-ssim" if args.config in (0, 4) and args.checkpoint is None
                                                        else "none")
    frame = Frame(wl, dev, loss_mode, rgb_only=args.rgb_only, frozen_features=args.frozen_features)
    leaves, state, w2c = frame.leaves, frame.state, frame.w2c
    colors, grad_image, grad_features, target = frame.colors, frame.grad_image, frame.grad_features, frame.target
    forward, backward, reset, step = frame.forward, frame.backward, frame.reset, frame.step

    if args.bwd_slice:
        import gaussian_splatting.rasterizer as rasterizer_module

        rasterizer_module.FEATURE_SLICE_WIDTH = args.bwd_slice
    ext = _get_rasterizer()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    # Agreement gate and CPU baseline: the oracle runs the same frame; one GPU step must agree with it.
    cpu, agreement = None, None
    if not args.no_cpu_baseline and not args.rgb_only and not args.frozen_features:
        reset()
        forward(retain=True)
        backward()
        torch.cuda.synchronize()
        gpu_out = {"image": state["out"][0], "feature_image": state["out"][1],
                   "means2D": state["means2D"].grad, "conics": state["conics"].grad,
                   **{name: leaf.grad for name, leaf in leaves.items()}}
        gpu_out = {k: v.detach().cpu().numpy() for k, v in gpu_out.items()}
        # The rasterizer's own inputs, for the oracle's forward on identical inputs.
        gpu_out["rasterizer_inputs"] = [t.detach().cpu().numpy() for t in state.pop("projected")] + [
            leaves["colors"].detach().cpu().numpy(), leaves["opacities"].detach().cpu().numpy()]
        state.pop("means2D"), state.pop("conics")
        cpu, want = cpu_baseline(wl, colors, grad_image, grad_features, args.cpu_samples, loss_target=target)
        agreement = agree(gpu_out, want)
        print(f"[bench] agreement with the oracle: {agreement}", file=sys.stderr, flush=True)
        if not agreement["passed"]:
            print(json.dumps({"metric": METRIC, "value": None, "unit": "ms", "n_gpus": 1,
                              "error": "disagrees with the oracle; not timed", "agreement": agreement}), flush=True)
            return 1

    # Timed region: exactly `steps` fwd+bwd steps between two device synchronisations. The library
    # records HIP events around the blend backward's kernels only (the roofline's duration): every
    # recorded launch adds two timed events to its stream, a few microseconds each, which around every
    # kernel and call of the step added about 0.19 ms to it.
    step_events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(args.steps)]
    torch.cuda.synchronize()
    with KernelProfile(only=BACKWARD_KERNELS) as kprof:
        t0 = time.perf_counter()
        for start, end in step_events:
            start.record()
            step()
            end.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3
    kernels = kprof.summary()
    step_ms = [s.elapsed_time(e) for s, e in step_events]
    ms_per_step = wall_ms / args.steps
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step wall, median {statistics.median(step_ms):.3f}",
          file=sys.stderr, flush=True)

    # Breakdown, after the timed region: a few more steps with events around every library call
    # (stages) and every kernel, for the per-stage and per-kernel figures of the JSON line.
    timer = StageTimer()
    ext.timer = timer
    with KernelProfile() as breakdown_prof:
        for _ in range(args.breakdown_steps):
            step()
        torch.cuda.synchronize()
    ext.timer = None
    stages = timer.summary()
    breakdown_kernels = breakdown_prof.summary()

    # Counts the roofline needs: visible gaussians and tile-gaussian pairs of this frame.
    with torch.no_grad():
        m2, d, r, c = project_gaussians(leaves["means"], leaves["scales"], F.normalize(leaves["quats"], dim=-1),
                                        leaves["opacities"][:, None], w2c, cam["fx"], cam["fy"], cam["cx"],
                                        cam["cy"], W, H)
        n_vis = int((r > 0).sum())
        pairs = int(ext.bin(m2, d, r, c, None, leaves["opacities"][:, None], W, H)[0].numel())
    hw = W * H
    alg = algorithmic_bytes(N, n_vis, pairs, hw, C)
    stage_report = {}
    for name, row in stages.items():
        entry = {"launches_per_step": row["launches"] / max(args.breakdown_steps, 1), "mean_ms": round(row["mean_ms"], 4)}
        if name in alg and row["mean_ms"] > 0:
            gbs = alg[name] / (row["mean_ms"] * 1e-3) / 1e9
            entry.update({"algorithmic_MB": round(alg[name] / 1e6, 2), "achieved_GBs": round(gbs, 1),
                          "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        stage_report[name] = entry

    split = {}
    if not args.no_split:
        split = harness_split(forward, backward, reset, min(args.steps, 20))

    # Roofline of the blend backward: one hds_render_backward call runs its two kernels (back-to-front
    # geometry/colour gradients, front-to-back feature gradients) side by side on two streams. The
    # duration is the pair's span, first start to last end, from the HIP events the library records
    # on each kernel's own stream over the timed region (rocprofv3's kernel trace gives the same
    # span); the per-kernel means, each longer than when run alone, are reported beside it.
    bwd_names, bwd_ms = backward_span(kernels, kprof.timeline)
    achieved = alg["render_backward"] / (bwd_ms * 1e-3) / 1e9
    roofline = {"kernel": " + ".join(bwd_names) + (" (side by side, one hds_render_backward call)"
                                                   if len(bwd_names) > 1 else ""),
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic_per_step(bwd_names, wl.name + ("-rgb-only" if args.rgb_only else "")),
                "algorithmic_bytes": int(alg["render_backward"]), "ms_per_call": round(bwd_ms, 4),
                "kernel_mean_ms": {k: round(kernels[k]["mean_ms"], 4) for k in bwd_names}}
    kernel_report = {k: {"launches_per_step": round(v["launches"] / max(args.breakdown_steps, 1), 2),
                         "mean_ms": round(v["mean_ms"], 4)}
                     for k, v in sorted(breakdown_kernels.items(), key=lambda kv: -kv[1]["total_ms"])}
    total_alg = sum(alg.values())
    step_frac = total_alg / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS

    sweep_channels = ([32, 64, 256, 512] if args.config == 2 and args.checkpoint is None and not args.rgb_only
                      else []) if args.sweep == "auto" else ([] if args.sweep == "none"
                                                             else [int(c) for c in args.sweep.split(",")])
    channel_sweep = None
    if sweep_channels:
        # Free the headline's feature buffers before the wider ones.
        leaves.pop("features", None)
        state.clear()
        del grad_features
        frame.grad_features = None
        torch.cuda.empty_cache()
        channel_sweep = measure_sweep(wl, leaves, w2c, sweep_channels, n_vis, pairs, args)

    # Under a profiler "auto" times no other config, so a trace or counter run covers the headline only.
    other = ([0, 1, 4] if args.config == 2 and args.checkpoint is None and not args.rgb_only
             and not args.frozen_features and not _profiled() else []) if args.configs == "auto" else (
        [] if args.configs == "none" else [int(c) for c in args.configs.split(",")])
    other_configs = None
    if other:
        torch.cuda.empty_cache()
        other_configs = [measure_config(index, args) for index in other]

    train = (args.train == "on" or (args.train == "auto" and args.config == 2 and args.checkpoint is None
                                     and not args.rgb_only and not args.frozen_features and not _profiled()))
    training_iteration = None
    if train:
        torch.cuda.empty_cache()
        training_iteration = measure_training_iteration(args.config)

    line = {
        "metric": METRIC, "value": round(ms_per_step, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": wl.name + ("-rgb-only" if args.rgb_only else "")
                   + ("-frozen-features" if args.frozen_features else ""), "gaussians": N, "width": W, "height": H,
                   "channels": 0 if args.rgb_only else C,
                   "visible": n_vis, "pairs": pairs, "parallelism": "single-gpu",
                   "loss": "0.8 L1 + 0.2 (1 - SSIM)" if target is not None else "none (dL/dimage U[0, 1])"},
        "step_ms_median": round(statistics.median(step_ms), 4), **split,
        "step_hbm_frac": round(step_frac, 4), "step_algorithmic_MB": round(total_alg / 1e6, 1),
        "roofline": roofline, "breakdown_steps": args.breakdown_steps, "stages": stage_report,
        "kernels": kernel_report, "cpu_baseline": cpu,
        "agreement": agreement, "channel_sweep": channel_sweep, "other_configs": other_configs,
        "training_iteration": training_iteration,
        "environment": environment(),
    }
    print(json.dumps(line), flush=True)
    if args.calibrate_copy_mib > 0:
        n_floats = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n_floats, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] calibration copy: {n_floats * 4} bytes read and written", file=sys.stderr, flush=True)
    return 0


# The blend backward's kernels: the only launches the library times inside the timed region.
BACKWARD_KERNELS = ("backward_geometry_kernel", "backward_features_kernel")


def backward_span(kernels: dict, timeline) -> tuple[list[str], float]:
    """The blend backward's kernels in the timed region and the mean duration of one
    hds_render_backward call: with two kernels side by side on two streams, their span (first start
    to last end); with one, its mean."""
    names = [k for k in BACKWARD_KERNELS if k in kernels]
    if len(names) == 2:
        return names, concurrent_span_ms(timeline, *names)
    return names, kernels[names[0]]["mean_ms"]


def harness_split(fn_fwd, fn_bwd, reset, samples: int) -> dict:
    """bench/harness.py:130-177's method: events around the forward alone, and around the backward
    alone with an untimed forward before each sample, a pause of 1.5x the sample after each, median /
    min / max, GPU clock and power before and after."""
    import torch

    def time_ms(fn, before=None):
        time.sleep(0.5)
        start_state = gpu_state()
        times = []
        for _ in range(samples):
            if before:
                before()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            e.synchronize()
            times.append(s.elapsed_time(e))
            time.sleep(max(0.01, 1.5 * times[-1] / 1000))
        return times, start_state, gpu_state()

    fwd, fwd_start, _ = time_ms(lambda: (reset(), fn_fwd()))
    bwd, _, bwd_end = time_ms(fn_bwd, before=lambda: (reset(), fn_fwd()))
    return {"fwd_ms_median": round(statistics.median(fwd), 4), "bwd_ms_median": round(statistics.median(bwd), 4),
            "fwd_ms_min_max": [round(min(fwd), 4), round(max(fwd), 4)],
            "bwd_ms_min_max": [round(min(bwd), 4), round(max(bwd), 4)],
            "gpu_state_split_start": fwd_start, "gpu_state_split_end": bwd_end}


def measure_sweep(wl, leaves: dict, w2c, channels_list, n_vis: int, pairs: int, args) -> list[dict]:
    """the headline scene's gaussians with C feature channels ~ N(0, 1) (seed 1, as
    tests/scenes.py draws them) and dL/dimage, dL/dF ~ U[0, 1] (seed 2), for each C: the fwd+bwd step
    (a few warm-up steps, then HIP events around each timed step), the harness fwd / bwd split, the
    blend backward's roofline over the span of its kernels and, unless --no-cpu-baseline, the CPU
    oracle's median fwd+bwd on the same frame."""
    import torch
    import torch.nn.functional as F

    from gaussian_splatting.rasterizer import project_gaussians, rasterize
    from gaussian_splatting.rasterizer._native import KernelProfile
    from tests.scenes import upstream

    dev = leaves["means"].device
    cam = wl.cam
    W, H, N = wl.width, wl.height, wl.n
    out = []
    for c in channels_list:
        print(f"[bench] channel sweep: C={c}", file=sys.stderr, flush=True)
        feats = torch.randn(N, c, generator=torch.Generator().manual_seed(1)).to(dev).requires_grad_(True)
        grad_image, grad_features = upstream(2, H, W, c, device=dev)
        holder = {}
        sweep_leaves = [leaves[k] for k in ("means", "scales", "quats", "opacities", "colors")] + [feats]

        def forward():
            m2, d, r, con = project_gaussians(leaves["means"], leaves["scales"], F.normalize(leaves["quats"], dim=-1),
                                              leaves["opacities"][:, None], w2c, cam["fx"], cam["fy"], cam["cx"],
                                              cam["cy"], W, H)
            holder["out"] = rasterize(m2, d, r, con, leaves["colors"], leaves["opacities"][:, None], W, H,
                                      features=feats)

        def backward():
            torch.autograd.backward(holder["out"], [grad_image, grad_features])

        def reset():
            for leaf in sweep_leaves:
                leaf.grad = None

        for _ in range(3):
            reset(), forward(), backward()
        steps = min(args.steps, 20)
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        torch.cuda.synchronize()
        with KernelProfile(only=BACKWARD_KERNELS) as kprof:
            for start, end in events:
                start.record()
                reset(), forward(), backward()
                end.record()
            torch.cuda.synchronize()
        step_ms = [s.elapsed_time(e) for s, e in events]
        names, bwd_ms = backward_span(kprof.summary(), kprof.timeline)
        alg = algorithmic_bytes(N, n_vis, pairs, W * H, c)["render_backward"]
        gbs = alg / (bwd_ms * 1e-3) / 1e9
        split = harness_split(forward, backward, reset, min(args.steps, 10))
        out.append({"channels": c, "step_ms_median": round(statistics.median(step_ms), 4),
                    "fwd_ms_median": split["fwd_ms_median"], "bwd_ms_median": split["bwd_ms_median"],
                    "render_backward_ms": round(bwd_ms, 4), "render_backward_algorithmic_MB": round(alg / 1e6, 1),
                    "render_backward_GBs": round(gbs, 1), "render_backward_hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        if not args.no_cpu_baseline:
            x = oracle_inputs(wl, leaves["colors"], grad_image, grad_features, features=feats)
            out[-1]["cpu_baseline"] = cpu_timing(
                x, args.cpu_samples, f"median of {args.cpu_samples} full fwd+bwd frames of the headline scene at "
                                     f"C={c} (same inputs) on the C oracle, OpenMP")[0]
            del x
        del feats, grad_image, grad_features, holder
        torch.cuda.empty_cache()
    return out


def measure_training_iteration(index: int, iterations: int = 20, warmup: int = 5) -> dict:
    """One iteration of the reference's training loop (main.py:159-200) on config `index`'s scene: the
    model's activations (exp scales, normalised quats, sigmoid opacities), projection, eval_sh with the
    fused SH Adam (utils/sh.py:59-109), rasterize with the features, 0.8 L1 + 0.2 (1 - SSIM) plus an L1
    term on the feature image against U[0, 1] targets, backward, the densification statistics from
    means2D.grad (utils/gaussian.py:143-160) and fused torch Adam over the other parameters. Returns the
    mean ms per iteration over `iterations` after `warmup`, timed with CUDA events."""
    import torch
    import torch.nn.functional as F

    from gaussian_splatting.rasterizer import project_gaussians, rasterize
    from gaussian_splatting.utils.densification import DensificationStats
    from gaussian_splatting.utils.loss import l1_loss, ssim
    from gaussian_splatting.utils.sh import eval_sh
    from tests.scenes import synthetic_config

    dev = torch.device("cuda:0")
    wl = synthetic_config(index).to(dev)
    cam, W, H = wl.cam, wl.width, wl.height
    print(f"[bench] training iteration on {wl.name}", file=sys.stderr, flush=True)
    model = {"means": wl.means, "scales": torch.log(wl.scales), "quats": wl.quats,
             "opacities": torch.logit(wl.opacities.clamp(1e-4, 1 - 1e-4)), "sh_dc": wl.sh_dc, "sh_rest": wl.sh_rest,
             "features": wl.features}
    model = {k: v.detach().clone().contiguous().requires_grad_(True) for k, v in model.items()}
    # Learning rates of the reference's config (config.py); they set no cost.
    lrs = {"means": 1.6e-4, "scales": 5e-3, "quats": 1e-3, "opacities": 5e-2, "sh_dc": 2.5e-3, "sh_rest": 1.25e-4,
           "features": 2.5e-3}
    optimizer = torch.optim.Adam([{"params": [model[k]], "lr": lrs[k], "name": k} for k in model], eps=1e-15,
                                 fused=True)
    g = torch.Generator(device=dev).manual_seed(2)
    gt = torch.rand(H, W, 3, device=dev, generator=g)
    gt_features = torch.rand(H, W, wl.channels, device=dev, generator=g)
    centre = wl.center
    stats = DensificationStats(wl.n, dev)

    def iteration():
        opac = torch.sigmoid(model["opacities"])
        means2D, depths, radii, conics = project_gaussians(
            model["means"], torch.exp(model["scales"]), F.normalize(model["quats"], dim=-1), opac,
            wl.world_to_camera, cam["fx"], cam["fy"], cam["cx"], cam["cy"], W, H)
        means2D.retain_grad()
        dirs = F.normalize(model["means"] - centre, dim=-1)
        colors = eval_sh(model["sh_dc"], model["sh_rest"], dirs, wl.sh_degree, radii, optimizer)
        image, feature_image = rasterize(means2D, depths, radii, conics, colors, opac, W, H,
                                         features=model["features"])
        loss = 0.8 * l1_loss(image, gt) + 0.2 * (1 - ssim(image, gt)) + l1_loss(feature_image, gt_features)
        loss.backward()
        with torch.no_grad():
            stats.add(means2D.grad, radii, W, H)
            optimizer.step()
            optimizer.zero_grad(set_to_none=True)

    for _ in range(warmup):
        iteration()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iterations):
        iteration()
    end.record()
    torch.cuda.synchronize()
    parameters = sum(v.numel() for v in model.values())
    return {"workload": wl.name, "ms": round(start.elapsed_time(end) / iterations, 4), "iterations": iterations,
            "warmup": warmup, "parameters": parameters,
            "scope": "activations, projection, eval_sh + fused SH Adam, rasterize (RGB + features), "
                     "0.8 L1 + 0.2 (1 - SSIM) + L1(features), backward, densification statistics, fused Adam"}


def measure_config(index: int, args) -> dict:
    """Another BASELINE config on the same GPU after the headline (0, 1 and 4 by default): its fwd+bwd
    step as the headline's runs (with the 0.8 L1 + 0.2 (1 - SSIM) loss for configs 0 and 4, whose
    BASELINE definition includes it), timed the same way, the harness fwd / bwd split, the blend
    backward's span and HBM fraction, and the per-stage means of a short breakdown pass. It has no
    oracle gate of its own: the -m gpu tests compare these configs with the oracle. Unless
    --no-cpu-baseline, the CPU oracle's median fwd+bwd of the same frame goes beside it: for config 4
    on the 64 tiles its parity test compares (the oracle's sort cannot take its ~94M pairs in
    seconds), labelled; for config 0 also the dense float64 blend, timed once."""
    import torch

    from gaussian_splatting.rasterizer import _get_rasterizer
    from gaussian_splatting.rasterizer._native import KernelProfile, StageTimer
    from tests.scenes import synthetic_config

    dev = torch.device("cuda:0")
    wl = synthetic_config(index)
    print(f"[bench] config {index}: {wl.name}", file=sys.stderr, flush=True)
    frame = Frame(wl, dev, "l1-ssim" if index in (0, 4) else "none")
    for _ in range(3):
        frame.step()
    steps = min(args.steps, 20)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    with KernelProfile(only=BACKWARD_KERNELS) as kprof:
        for start, end in events:
            start.record()
            frame.step()
            end.record()
        torch.cuda.synchronize()
    step_ms = [s.elapsed_time(e) for s, e in events]
    _, bwd_ms = backward_span(kprof.summary(), kprof.timeline)
    ext = _get_rasterizer()
    timer = StageTimer()
    ext.timer = timer
    for _ in range(5):
        frame.step()
    ext.timer = None
    stages = {name: round(row["mean_ms"], 4) for name, row in timer.summary().items()}
    split = harness_split(frame.forward, frame.backward, frame.reset, min(args.steps, 10))
    # Visible gaussians and pairs of this frame, for the backward's algorithmic bytes.
    import torch.nn.functional as F

    from gaussian_splatting.rasterizer import project_gaussians

    with torch.no_grad():
        lv, cam = frame.leaves, wl.cam
        m2, d, r, c = project_gaussians(lv["means"], lv["scales"], F.normalize(lv["quats"], dim=-1),
                                        lv["opacities"][:, None], frame.w2c, cam["fx"], cam["fy"], cam["cx"],
                                        cam["cy"], wl.width, wl.height)
        n_vis = int((r > 0).sum())
        values, ranges = ext.bin(m2, d, r, c, None, lv["opacities"][:, None], wl.width, wl.height)[:2]
        pairs, ranges = int(values.numel()), ranges.cpu().numpy()
        del values
    alg = algorithmic_bytes(wl.n, n_vis, pairs, wl.width * wl.height, wl.channels)["render_backward"]
    gbs = alg / (bwd_ms * 1e-3) / 1e9
    out = {"config": index, "workload": wl.name, "gaussians": wl.n, "width": wl.width, "height": wl.height,
           "channels": wl.channels, "visible": n_vis, "pairs": pairs,
           "loss": "0.8 L1 + 0.2 (1 - SSIM)" if frame.target is not None else "none (dL/dimage U[0, 1])",
           "step_ms_median": round(statistics.median(step_ms), 4), "fwd_ms_median": split["fwd_ms_median"],
           "bwd_ms_median": split["bwd_ms_median"], "render_backward_ms": round(bwd_ms, 4),
           "render_backward_GBs": round(gbs, 1), "render_backward_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
           "stages_ms": stages}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = config_cpu_baseline(wl, frame, index, ranges, args.cpu_samples)
    del frame
    torch.cuda.empty_cache()
    return out


def config_cpu_baseline(wl, frame, index: int, ranges, samples: int) -> dict:
    """The CPU oracle on a config's frame (same inputs as the GPU's): the median of `samples` full
    fwd+bwd frames, with the loss when the GPU step has it; config 4 on the 64 tiles of its parity test
    (tests/scenes.py tile_selection on the GPU binning's list lengths), at most 3 samples, without the
    loss (its SSIM would run on a frame rendered only there); config 0 adds the dense float64 blend."""
    from tests.scenes import tile_selection

    x = oracle_inputs(wl, frame.colors, frame.grad_image, frame.grad_features)
    if index == 4:
        mask = tile_selection(ranges, (wl.width + 15) // 16)
        samples = max(1, min(samples, 3))
        record, _ = cpu_timing(x, samples, f"median of {samples} fwd+bwd of {wl.name} restricted to {int(mask.sum())} "
                                           f"of {mask.size} tiles (the 16 longest lists + 48 at random, seed 0): "
                                           "projection of every gaussian, binning and blend fwd+bwd on those "
                                           "tiles; dL/dimage U[0, 1], no SSIM; C oracle, OpenMP",
                               tile_mask=mask)
        record["tile_masked"] = True
        return record
    target = None if frame.target is None else frame.target.detach().cpu().numpy()
    record, _ = cpu_timing(x, samples, f"median of {samples} full fwd+bwd frames of {wl.name} (same inputs"
                                       + (", 0.8 L1 + 0.2 (1 - SSIM)" if target is not None else "")
                                       + ") on the C oracle, OpenMP", loss_target=target)
    if index == 0:
        record["dense_fp64"] = dense_fp64_timing(x)
    return record


def concurrent_span_ms(timeline, first: str, second: str) -> float:
    """Mean over calls of (later end - earlier start) of two kernels launched together: each `first`
    launch is paired with the `second` launch that starts nearest to it."""
    a = [(t0, t1) for name, t0, t1 in timeline if name == first]
    b = [(t0, t1) for name, t0, t1 in timeline if name == second]
    spans = []
    for s0, e0 in a:
        s1, e1 = min(b, key=lambda se: abs(se[0] - s0))
        spans.append(max(e0, e1) - min(s0, s1))
    return sum(spans) / len(spans)


TRAFFIC_FILE = ROOT / "profiles" / "render_backward_headline_c128_pmc.md"


def source_digest() -> str:
    """sha256 (first 16 hex digits) of the HIP sources and the public header."""
    digest = hashlib.sha256()
    for path in sorted((ROOT / "high-dimensional-splatting_amd" / "csrc").glob("*")) + [ROOT / "include" / "hds_rasterizer.h"]:
        digest.update(path.read_bytes())
    return digest.hexdigest()[:16]


def traffic_per_step(kernel_names, workload: str) -> int | None:
    """HBM bytes the named kernels move per step, from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a copy kernel of known size); None unless that
    summary was taken on this workload with this build (its "workload:" and "source:" header lines)
    and covers every one of the kernels."""
    if not TRAFFIC_FILE.exists():
        return None
    text = TRAFFIC_FILE.read_text()
    header = {}
    for line in text.splitlines():
        for key in ("workload:", "source:"):
            if line.strip().lower().startswith(key):
                header[key] = line.split(":", 1)[1].strip().strip("`")
    if header.get("workload:") != workload or header.get("source:") != source_digest():
        return None
    per_kernel = {}
    for line in text.splitlines():
        # rows of the form "| kernel | ... | traffic_bytes |" with the bytes in the last column
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 2 and cells[0] in kernel_names and cells[-1].isdigit():
            per_kernel[cells[0]] = int(cells[-1])
    if not kernel_names or any(k not in per_kernel for k in kernel_names):
        return None
    return sum(per_kernel[k] for k in kernel_names)


def oracle_inputs(wl, colors, grad_image, grad_features, features=None) -> dict:
    """The frame's inputs as the CPU oracle takes them (numpy float32 copies of the GPU's leaves and
    upstream gradients; features default to the workload's)."""
    import numpy as np

    np_ = lambda t: t.detach().cpu().numpy()  # noqa: E731
    return {"wl": wl, "means": np_(wl.means), "scales": np_(wl.scales),
            "quats": np_(wl.quats / wl.quats.norm(dim=-1, keepdim=True)), "opacities": np_(wl.opacities),
            "features": np_(wl.features if features is None else features), "colors": np_(colors),
            "grad_image": np_(grad_image), "grad_features": np_(grad_features),
            "w2c": np_(wl.world_to_camera).astype(np.float32)}


def oracle_frame(x: dict, loss_target=None, tile_mask=None):
    """One fwd+bwd of the frame on the C oracle (OpenMP): projection, binning, blend forward, then
    (with loss_target, dL/dimage of 0.8 L1 + 0.2 (1 - SSIM) against it from the oracle's SSIM instead
    of the given dL/dimage) blend backward and projection backward. With tile_mask the binning, and
    so the blend, covers only the selected tiles. Returns the forward's and backward's seconds and the
    outputs."""
    import numpy as np

    import oracle

    cam, wl = x["wl"].cam, x["wl"]
    W, H = wl.width, wl.height
    bg = np.zeros(3, np.float32)
    t0 = time.perf_counter()
    m2, d, r, c = oracle.project_forward(x["means"], x["scales"], x["quats"], x["opacities"], x["w2c"], cam["fx"],
                                         cam["fy"], cam["cx"], cam["cy"], W, H)
    _, values, ranges = oracle.bin_gaussians(m2, d, r, c, x["opacities"], W, H, tile_mask=tile_mask)
    image, T, nc, fimg = oracle.render_forward(W, H, ranges, values, m2, c, x["opacities"], x["colors"], bg,
                                               x["features"])
    t1 = time.perf_counter()
    gi = x["grad_image"]
    if loss_target is not None:
        # d/dimage of 0.8 mean|image - target| + 0.2 (1 - mean SSIM): sign / numel, and the SSIM
        # backward with dL/dmean = -0.2 (utils/loss.py:57-96 there).
        gi = (0.8 * np.sign(image - loss_target) / image.size).astype(np.float32)
        _, d_mu, d_aa, d_ab = oracle.ssim_forward(image, loss_target)
        gi += oracle.ssim_backward(-0.2, image, loss_target, d_mu, d_aa, d_ab)
    dm, dc, dcol, dop, df = oracle.render_backward(W, H, ranges, values, m2, c, x["opacities"], x["colors"], bg, T, nc,
                                                   gi, x["features"], x["grad_features"])
    dmeans, dscales, dq = oracle.project_backward(dm, dc, x["means"], x["scales"], x["quats"], x["w2c"], cam["fx"],
                                                  cam["fy"], cam["cx"], cam["cy"], W, H)
    t2 = time.perf_counter()
    return t1 - t0, t2 - t1, {"image": image, "feature_image": fimg, "means2D": dm, "conics": dc, "colors": dcol,
                              "opacities": dop, "features": df, "means": dmeans, "scales": dscales, "quats": dq}


def host() -> dict:
    """The host the CPU figures ran on: logical CPUs, the ones this process may use, the OpenMP
    thread count the oracle ran with, and the CPU model."""
    import oracle

    return {"nproc": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0)), "omp_threads": oracle.num_threads(),
            "cpu": _cpu_model()}


def cpu_timing(x: dict, samples: int, sample: str, loss_target=None, tile_mask=None):
    """`samples` oracle fwd+bwd runs of the frame: the median total, forward and backward (ms), every
    sample's total, and the host. Returns the record and the last run's outputs."""
    import oracle

    totals, fwds, bwds, out = [], [], [], None
    for i in range(samples):
        fwd, bwd, out = oracle_frame(x, loss_target=loss_target, tile_mask=tile_mask)
        fwds.append(fwd * 1e3), bwds.append(bwd * 1e3), totals.append((fwd + bwd) * 1e3)
        print(f"[bench] cpu baseline {x['wl'].name}: sample {i + 1}/{samples} {totals[-1]:.0f} ms",
              file=sys.stderr, flush=True)
    return ({"value": round(statistics.median(totals), 1), "unit": "ms", "cores": oracle.num_threads(),
             "kind": "port", "fwd_ms": round(statistics.median(fwds), 1), "bwd_ms": round(statistics.median(bwds), 1),
             "samples": samples, "samples_ms": [round(t, 1) for t in totals], "statistic": "median",
             "sample": sample, **host()}, out)


def cpu_baseline(wl, colors, grad_image, grad_features, samples: int, loss_target=None):
    """The CPU oracle (OpenMP, all usable host threads) on the same frame, `samples` times (median;
    fwd = projection + binning + blend forward, bwd = loss gradient + blend backward + projection
    backward). Returns the baseline record and the oracle's outputs in the leaves' shapes (for the
    agreement gate)."""
    import numpy as np
    import torch

    import oracle

    x = oracle_inputs(wl, colors, grad_image, grad_features)
    target = None if loss_target is None else loss_target.detach().cpu().numpy()
    print(f"[bench] cpu baseline: oracle fwd+bwd of the full frame, {samples} samples", file=sys.stderr, flush=True)
    record, out = cpu_timing(x, samples, f"median of {samples} full fwd+bwd frames of {wl.name} (same inputs) on "
                                         "the C oracle, OpenMP", loss_target=target)
    cam = wl.cam
    means, scales, quats, w2c, feats = x["means"], x["scales"], x["quats"], x["w2c"], x["features"]

    def normalize_backward(d_unit):
        # The quats leaf goes through F.normalize before the projection: its gradient, on the CPU.
        q = wl.quats.detach().clone().requires_grad_(True)
        torch.nn.functional.normalize(q, dim=-1).backward(torch.from_numpy(np.ascontiguousarray(d_unit)))
        return q.grad.numpy()

    def forward_stage(m2_, d_, r_, c_, col_, op_):
        # The oracle's binning and blend forward on the GPU projection's outputs (identical inputs).
        _, values_, ranges_ = oracle.bin_gaussians(m2_, d_, r_, c_, op_, cam["width"], cam["height"])
        out_ = oracle.render_forward(cam["width"], cam["height"], ranges_, values_, m2_, c_, op_, col_,
                                     np.zeros(3, np.float32), feats)
        return out_[0], out_[3]

    def projection_stage(grad_means2D, grad_conics):
        # The oracle's projection backward (and the normalize chain) on given upstream gradients.
        pm, ps, pq = oracle.project_backward(grad_means2D, grad_conics, means, scales, quats, w2c, cam["fx"],
                                             cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
        return {"means": pm, "scales": ps, "quats": normalize_backward(pq)}

    want = {"image": out["image"], "feature_image": out["feature_image"], "means2D": out["means2D"],
            "conics": out["conics"], "opacities": np.asarray(out["opacities"]).reshape(-1), "colors": out["colors"],
            "features": out["features"],
            "chain": {"means": out["means"], "scales": out["scales"], "quats": normalize_backward(out["quats"])},
            "projection_stage": projection_stage, "forward_stage": forward_stage}
    return record, want


def dense_fp64_timing(x: dict) -> dict:
    """The dense float64 formulation (tests/dense_reference.py, the formulation of the reference's
    tests/oracle.py:9-77: every pixel against every visible gaussian, torch autograd for the backward)
    timed once on the frame's blend: the oracle's projection (not timed), then the blend of colours and
    features as one [N, 3 + C] value per gaussian, forward and backward of dL/dimage and
    dL/dfeature_image."""
    import numpy as np
    import torch

    import oracle
    from tests.dense_reference import dense_blend_grad

    wl, cam = x["wl"], x["wl"].cam
    m2, d, r, c = oracle.project_forward(x["means"], x["scales"], x["quats"], x["opacities"], x["w2c"], cam["fx"],
                                         cam["fy"], cam["cx"], cam["cy"], wl.width, wl.height)
    values = torch.from_numpy(np.concatenate([x["colors"], x["features"]], axis=1))
    upstream = torch.from_numpy(np.concatenate([x["grad_image"], x["grad_features"]], axis=-1))
    print(f"[bench] dense fp64 blend of {wl.name}, once", file=sys.stderr, flush=True)
    _, _, fwd, bwd = dense_blend_grad(*(torch.from_numpy(a) for a in (m2, d, r, c)), values,
                                      torch.from_numpy(x["opacities"]), wl.width, wl.height, upstream)
    return {"value": round((fwd + bwd) * 1e3, 1), "unit": "ms", "fwd_ms": round(fwd * 1e3, 1),
            "bwd_ms": round(bwd * 1e3, 1), "samples": 1, "kind": "dense fp64 (tests/dense_reference.py)",
            "torch_threads": torch.get_num_threads(),
            "sample": f"one dense float64 blend fwd+bwd of {wl.name} (RGB + {wl.channels} features as one "
                      f"{3 + wl.channels}-wide value, {int((r > 0).sum())} visible gaussians x {wl.width * wl.height} "
                      "pixels), the formulation of the reference's tests/oracle.py; projection not timed"}


# Largest gradient error allowed by the gate, relative to max|want|: the parity tests' bar, from the
# reference's assert_grads_close (tests/test_render.py:45-58 there).
GATE_MAX_REL = 2e-3


def agree(got: dict, want: dict) -> dict:
    """The parity tests' bars on this frame, stage by stage, each stage on identical inputs:
      - the blend forward on the GPU projection's outputs: the RGB image bit for bit (both sides take
        alpha from hds_gauss_alpha and blend with the same fused multiply-adds), the feature image by
        max / 99th percentile error;
      - the rasterizer's gradients (means2D, conics, colors, opacities, features) against the oracle's
        rasterizer on the same projected inputs;
      - the projection backward (means, scales and the quats leaf through normalize) against the
        oracle's projection backward fed the GPU's own means2D / conics gradients;
    each gradient with < 0.1% of values outside rtol 1e-3 and the largest error within GATE_MAX_REL
    of max|want|. The end-to-end leaf errors (the oracle's projection backward on the oracle's own
    rasterizer gradients) are reported under "chain" without a bar: composing the two stages
    amplifies their ~1e-6 relative differences by the conditioning of the conic -> quaternion map of
    elongated gaussians."""
    import numpy as np

    from tests.tolerances import grad_error, image_error

    report, passed = {}, True
    want_image, want_fimg = want["forward_stage"](*got["rasterizer_inputs"])
    differ = int(np.sum(got["image"] != want_image))
    report["image"] = {"values_differing": differ}
    passed &= differ == 0
    worst, p99 = image_error(got["feature_image"], want_fimg)
    report["feature_image"] = {"max": worst, "p99": p99}
    passed &= worst < 1e-3 and p99 < 5e-4
    for name in ("means2D", "conics", "colors", "opacities", "features"):
        outside, rel = grad_error(got[name].reshape(want[name].shape), want[name])
        report[name] = {"outside": outside, "max_rel": rel}
        passed &= outside < 1e-3 and rel <= GATE_MAX_REL
    stage = want["projection_stage"](got["means2D"], got["conics"])
    report["chain"] = {}
    for name in ("means", "scales", "quats"):
        outside, rel = grad_error(got[name].reshape(stage[name].shape), stage[name])
        report[name] = {"outside": outside, "max_rel": rel}
        passed &= outside < 1e-3 and rel <= GATE_MAX_REL
        outside, rel = grad_error(got[name].reshape(want["chain"][name].shape), want["chain"][name])
        report["chain"][name] = {"outside": outside, "max_rel": rel}
    report["passed"] = bool(passed)
    return report


def _profiled() -> bool:
    """True under rocprofv3, whose tool library is loaded into child processes too: amd-smi (a
    script started through env) is then not run, so no child re-executes after GPU initialisation."""
    return any(k.startswith(("ROCPROF_", "ROCPROFILER_")) for k in os.environ)


def gpu_state() -> dict:
    """Mean GFX clock (MHz) over the XCDs and socket power (W) of GPU 0 from amd-smi; {} if unavailable
    or under a profiler (the reference harness reads clocks and power capping from nvidia-smi,
    harness.py:117-128)."""
    if _profiled():
        return {}
    try:
        out = subprocess.run(["amd-smi", "metric", "-g", "0", "--clock", "--power", "--json"], capture_output=True,
                             text=True, timeout=20, check=True).stdout
        data = json.loads(out)
        data = data["gpu_data"] if isinstance(data, dict) and "gpu_data" in data else data
        data = data[0] if isinstance(data, list) else data
        clocks = [v["clk"]["value"] for k, v in data.get("clock", {}).items()
                  if k.startswith("gfx") and isinstance(v.get("clk"), dict)]
        power = data.get("power", {}).get("socket_power", {})
        return {"gfx_clock_mhz": round(sum(clocks) / len(clocks), 1) if clocks else None,
                "socket_power_w": power.get("value") if isinstance(power, dict) else None}
    except Exception:  # noqa: BLE001 - a missing or differently shaped amd-smi only drops the record
        return {}


def environment() -> dict:
    """GPU, software and a digest of the HIP sources, like the reference's golden-test environment
    record (tests/test_golden.py:34-35)."""
    import torch

    name = torch.cuda.get_device_name(0)
    try:
        if _profiled():
            raise RuntimeError("amd-smi is not run under a profiler")
        out = subprocess.run(["amd-smi", "static", "-g", "0", "--asic", "--json"], capture_output=True, text=True,
                             timeout=20, check=True).stdout
        data = json.loads(out)
        data = data["gpu_data"] if isinstance(data, dict) and "gpu_data" in data else data
        data = data[0] if isinstance(data, list) else data
        name = data["asic"]["market_name"]
    except Exception:  # noqa: BLE001 - torch's device name stands in
        pass
    return {"gpu": name, "torch": torch.__version__, "hip": torch.version.hip, "source": source_digest(),
            **gpu_state()}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
