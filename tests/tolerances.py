"""Agreement bars shared by the GPU parity tests and bench.py's agreement gate.

Images: the reference's assert_image_close (tests/test_render.py:33-38 there): max error and 99th
percentile of the absolute difference. Gradients: assert_grads_close (test_render.py:45-58 there):
rtol 1e-3 with an absolute floor of 1e-4 x max|want|, fewer than 0.1% of the values outside, and the
largest error at most 2e-3 x max|want|.
"""
from __future__ import annotations

import math

import numpy as np


def image_error(got, want) -> tuple[float, float]:
    """(max, 99th percentile) of |got - want|."""
    diff = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).ravel()
    if diff.size == 0:
        return 0.0, 0.0
    p99 = np.partition(diff, max(0, math.ceil(0.99 * diff.size) - 1))[max(0, math.ceil(0.99 * diff.size) - 1)]
    return float(diff.max()), float(p99)


def assert_image_close(got, want, max_error=2e-3, max_perc_99=1e-4):
    worst, p99 = image_error(got, want)
    assert worst < max_error and p99 < max_perc_99, f"max {worst:.2e}, 99th {p99:.2e}"


def grad_error(got, want, chunk: int = 1 << 24) -> tuple[float, float]:
    """(share of values outside rtol 1e-3 / atol 1e-4 max, max error / max|want|).

    Evaluated in float64 over chunks of `chunk` values, so gradients of hundreds of millions of
    values (1.18M gaussians x 512 channels) need no full-size float64 temporaries. A NaN or infinite
    value on either side makes the max error infinite (and counts as outside), so it can never hide
    in the share of values allowed outside the tolerance."""
    got, want = np.asarray(got).reshape(-1), np.asarray(want).reshape(-1)
    if want.size == 0:
        return 0.0, 0.0
    assert got.size == want.size, (got.size, want.size)
    scale = 0.0
    for i in range(0, want.size, chunk):
        w = np.abs(want[i:i + chunk])
        finite = np.isfinite(w)
        if finite.any():
            scale = max(scale, float(w[finite].max()))
    bad, worst = 0, 0.0
    for i in range(0, want.size, chunk):
        g, w = got[i:i + chunk].astype(np.float64), want[i:i + chunk].astype(np.float64)
        nonfinite = ~(np.isfinite(g) & np.isfinite(w))
        if nonfinite.any():
            worst = math.inf
        bad += int(np.count_nonzero(~np.isclose(g, w, rtol=1e-3, atol=1e-4 * scale) | nonfinite))
        if not nonfinite.all():
            worst = max(worst, float(np.abs(g[~nonfinite] - w[~nonfinite]).max()))
    return bad / want.size, worst / scale if scale > 0 else worst


def assert_grads_close(names, grads, wants):
    for name, got, want in zip(names, grads, wants):
        got, want = np.asarray(got), np.asarray(want)
        assert got.shape == want.shape, f"{name}: shape {got.shape} vs {want.shape}"
        outside, rel = grad_error(got, want)
        assert outside < 1e-3, f"{name}: {outside:.2%} outside tolerance"
        assert rel <= 2e-3, f"{name}: max error {rel:.2e} of max |want|"
