"""bench.py's CPU baseline leg on the CPU (no GPU): the oracle's median fwd+bwd of a frame with its
split and host record, a config's figure with the loss, and the dense float64 blend of config 0
(BASELINE.md's CPU plan); the agreement gate's reference outputs come back in the leaves' shapes."""
from __future__ import annotations

import statistics
import types

import numpy as np
import torch

import bench
from tests.scenes import synthetic_config, upstream

KEYS = {"value", "unit", "cores", "kind", "sample", "samples", "samples_ms", "fwd_ms", "bwd_ms", "statistic",
        "nproc", "usable_cpus", "omp_threads", "cpu"}


def test_cpu_baseline_is_a_median_with_its_split_and_host():
    wl = synthetic_config(0)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3))
    grad_image, grad_features = upstream(2, wl.height, wl.width, wl.channels)
    record, want = bench.cpu_baseline(wl, colors, grad_image, grad_features, 3)
    assert KEYS <= set(record) and record["kind"] == "port" and record["unit"] == "ms"
    assert record["samples"] == 3 and len(record["samples_ms"]) == 3
    assert record["value"] == round(statistics.median(record["samples_ms"]), 1)
    assert 0 < record["fwd_ms"] and 0 < record["bwd_ms"] and record["nproc"] >= record["usable_cpus"] >= 1
    assert record["cores"] == record["omp_threads"] >= 1
    n, c = wl.n, wl.channels
    assert want["image"].shape == (wl.height, wl.width, 3) and want["feature_image"].shape == (wl.height, wl.width, c)
    assert want["means2D"].shape == (n, 2) and want["conics"].shape == (n, 3) and want["colors"].shape == (n, 3)
    assert want["opacities"].shape == (n,) and want["features"].shape == (n, c)
    assert {k: v.shape for k, v in want["chain"].items()} == {"means": (n, 3), "scales": (n, 3), "quats": (n, 4)}
    assert np.isfinite(want["chain"]["quats"]).all() and np.abs(want["features"]).max() > 0


def test_config_figure_carries_the_loss_and_the_dense_float64_blend():
    wl = synthetic_config(0)
    grad_image, grad_features = upstream(2, wl.height, wl.width, wl.channels)
    frame = types.SimpleNamespace(colors=torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)),
                                  grad_image=grad_image, grad_features=grad_features, target=grad_image)
    record = bench.config_cpu_baseline(wl, frame, 0, None, 2)
    assert KEYS <= set(record) and record["samples"] == 2 and "SSIM" in record["sample"]
    dense = record["dense_fp64"]
    assert dense["samples"] == 1 and dense["value"] > 0 and dense["fwd_ms"] > 0 and dense["bwd_ms"] > 0
    assert dense["kind"].startswith("dense fp64") and f"{3 + wl.channels}-wide" in dense["sample"]
