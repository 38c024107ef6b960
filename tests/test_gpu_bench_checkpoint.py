"""bench.py on a trained-model checkpoint: the reference harness's use (bench/harness.py:216-235).

A model.pt in the reference's layout (written here from a seeded scene) and a camera turned 30 degrees
off the world axes go through bench.py's --checkpoint / --camera path in this process: the agreement
gate (one fwd+bwd step against the CPU oracle on the same frame) must pass and the JSON line must carry
the checkpoint's frame.
"""
import json
import math
import sys

import pytest
import torch

from gaussian_splatting.utils.checkpoint import CameraView, save_camera, save_checkpoint

pytestmark = pytest.mark.gpu


def test_bench_times_a_checkpoint_frame_that_agrees_with_the_oracle(tmp_path, monkeypatch, capsys):
    import bench

    n = 20_000
    g = torch.Generator().manual_seed(3)
    params = {
        "means": (torch.rand(n, 3, generator=g) * 2 - 1) * 1.5,
        "scales": torch.randn(n, 3, generator=g) * 0.5 - 4.0,
        "quats": torch.randn(n, 4, generator=g) * 2,
        "opacities": torch.randn(n, 1, generator=g),
        "sh_dc": torch.randn(n, 1, 3, generator=g) * 0.5,
        "sh_rest": torch.randn(n, 15, 3, generator=g) * 0.05,
    }
    save_checkpoint(tmp_path / "model.pt", params, 3, 7000, 24.0)
    a = math.radians(30)
    w2c = torch.eye(4)
    w2c[:3, :3] = torch.tensor([[math.cos(a), 0.0, math.sin(a)], [0.0, 1.0, 0.0], [-math.sin(a), 0.0, math.cos(a)]])
    w2c[:3, 3] = torch.tensor([0.1, -0.2, 4.0])
    save_camera(tmp_path / "cam.json", CameraView(w2c, 230.0, 225.0, 131.0, 94.5, 256, 192, "turned"))

    monkeypatch.setattr(sys, "argv", ["bench.py", "--checkpoint", str(tmp_path / "model.pt"), "--camera",
                                      str(tmp_path / "cam.json"), "--channels", "32", "--steps", "3", "--warmup", "1",
                                      "--no-split"])
    print("[test] bench.py --checkpoint (20k gaussians, 256x192, C=32)", file=sys.stderr, flush=True)
    rc = bench.main()
    line = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert rc == 0, line
    assert line["agreement"]["passed"], line["agreement"]
    cfg = line["config"]
    assert (cfg["gaussians"], cfg["width"], cfg["height"], cfg["channels"]) == (n, 256, 192, 32)
    assert cfg["workload"].startswith("checkpoint-model-turned")
    assert 0 < cfg["visible"] <= n and cfg["pairs"] > 0
    assert line["value"] > 0


def test_bench_times_another_config_with_its_loss():
    """bench.py's other-config pass (configs 0, 1 and 4 after the headline): config 0 runs its step with
    the L1 + SSIM loss and reports the step, the harness split, the blend backward and the stages, and
    beside them the CPU oracle's median fwd+bwd of the same frame and the dense float64 blend."""
    import argparse

    import bench

    print("[test] bench.measure_config(0)", file=sys.stderr, flush=True)
    out = bench.measure_config(0, argparse.Namespace(steps=3, no_cpu_baseline=False, cpu_samples=2))
    cpu = out["cpu_baseline"]
    assert cpu["samples"] == 2 and len(cpu["samples_ms"]) == 2 and cpu["value"] > 0 and cpu["kind"] == "port"
    assert cpu["fwd_ms"] > 0 and cpu["bwd_ms"] > 0 and cpu["nproc"] >= 1 and "SSIM" in cpu["sample"]
    assert cpu["dense_fp64"]["samples"] == 1 and cpu["dense_fp64"]["value"] > 0
    assert out["config"] == 0 and out["workload"].startswith("cpu-plumbing-10k")
    assert out["loss"].startswith("0.8 L1")
    assert out["gaussians"] == 10_000 and out["channels"] == 32
    assert 0 < out["visible"] <= out["gaussians"] and out["pairs"] > 0
    for key in ("step_ms_median", "fwd_ms_median", "bwd_ms_median", "render_backward_ms"):
        assert out[key] > 0, key
    stages = set(out["stages_ms"])
    # The binning is one stage in tile order ("bin"), two with the global depth sort.
    assert {"bin"} <= stages or {"bin_count", "bin_emit"} <= stages
    assert {"render", "render_backward", "ssim_forward", "ssim_backward"} <= stages


def test_bench_times_a_training_iteration():
    """bench.py's training-iteration pass (the reference's loop: projection, eval_sh with the fused SH
    Adam, rasterize, the loss, backward, densification statistics, Adam) runs on config 0's scene and
    reports its time and parameter count."""
    import bench

    print("[test] bench.measure_training_iteration(0)", file=sys.stderr, flush=True)
    out = bench.measure_training_iteration(0, iterations=2, warmup=1)
    assert out["workload"].startswith("cpu-plumbing-10k") and out["iterations"] == 2
    assert out["ms"] > 0
    assert out["parameters"] == 10_000 * (3 + 3 + 4 + 1 + 3 + 45 + 32)
