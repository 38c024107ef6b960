"""Densification statistics of GaussianModel (the reference's utils/gaussian.py:133-160).

`DensificationStats` holds the per-gaussian bookkeeping the reference keeps on its GaussianModel
(max_radii2D [N], means2D_grad_accum [N, 1], denom [N, 1]; `_reset_stats`, gaussian.py:133-141) and
`add` is `add_densification_stats` (gaussian.py:143-160): for the gaussians a view rendered, the
largest screen radius, the accumulated norm of the pixel-space means2D gradient rescaled to
normalised device units, and the count. One HIP kernel per call instead of the reference's torch
operations, and no host synchronisation (the reference's boolean indexing waits for the device).
"""
from __future__ import annotations

import torch

from gaussian_splatting.rasterizer import _get_rasterizer


class DensificationStats:
    """The densification bookkeeping of `n` gaussians on `device`."""

    def __init__(self, n: int, device: torch.device | str) -> None:
        self.reset(n, device)

    def reset(self, n: int, device: torch.device | str | None = None) -> None:
        """Zeroes the statistics, sized for the current population (gaussian.py:133-141)."""
        device = self.max_radii2D.device if device is None else device
        self.max_radii2D = torch.zeros(n, device=device)
        self.means2D_grad_accum = torch.zeros(n, 1, device=device)
        self.denom = torch.zeros(n, 1, device=device)

    def add(self, means2D_grad: torch.Tensor, radii: torch.Tensor, width: int, height: int) -> None:
        """add_densification_stats (gaussian.py:143-160).

        Args:
            means2D_grad: [N, 2] gradient of the loss with respect to the 2D centers, in pixels.
            radii: [N] footprint radii in pixels, 0 for gaussians this view did not render.
            width: Image width in pixels.
            height: Image height in pixels.
        """
        _get_rasterizer().densification_stats(means2D_grad, radii, width, height, self.max_radii2D,
                                              self.means2D_grad_accum, self.denom)

    def mean_grads(self) -> torch.Tensor:
        """[N] mean accumulated gradient per gaussian, the quantity densify_and_prune thresholds
        (gaussian.py:173)."""
        return torch.nan_to_num(self.means2D_grad_accum / self.denom.clamp_min(1)).squeeze(-1)
