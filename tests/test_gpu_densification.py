"""Densification statistics (the reference's GaussianModel.add_densification_stats,
utils/gaussian.py:143-160) on the HIP kernel against the reference's torch formula.

The expected values restate gaussian.py:154-158 with torch on the CPU; a hand-solved case pins
that restatement (a gradient of (3, 4) / (W/2, H/2) has norm 5 after the rescale).
"""
import pytest
import torch

from gaussian_splatting.utils.densification import DensificationStats

pytestmark = pytest.mark.gpu

DEV = "cuda"


def reference_add(max_radii2D, accum, denom, grad, radii, width, height):
    """gaussian.py:154-158 (torch, CPU)."""
    visible = radii > 0
    max_radii2D = torch.where(visible, torch.maximum(max_radii2D, radii), max_radii2D)
    scale = torch.tensor([0.5 * width, 0.5 * height])
    accum = accum.clone()
    denom = denom.clone()
    accum[visible] += (grad * scale)[visible].norm(dim=-1, keepdim=True)
    denom[visible] += 1
    return max_radii2D, accum, denom


def test_hand_solved_gaussian():
    stats = DensificationStats(3, DEV)
    grad = torch.tensor([[3.0 / 40, 4.0 / 30], [1.0, 1.0], [0.0, -2.0 / 30]], device=DEV)
    radii = torch.tensor([2.5, 0.0, 7.0], device=DEV)
    stats.add(grad, radii, 80, 60)
    stats.add(grad, radii, 80, 60)
    torch.cuda.synchronize()
    assert torch.allclose(stats.means2D_grad_accum.squeeze(-1).cpu(), torch.tensor([10.0, 0.0, 4.0]), rtol=1e-6)
    assert torch.equal(stats.denom.squeeze(-1).cpu(), torch.tensor([2.0, 0.0, 2.0]))
    assert torch.equal(stats.max_radii2D.cpu(), torch.tensor([2.5, 0.0, 7.0]))
    assert torch.allclose(stats.mean_grads().cpu(), torch.tensor([5.0, 0.0, 2.0]), rtol=1e-6)


@pytest.mark.parametrize("n", [1, 1000, 300_001])
def test_matches_the_reference_over_several_views(n):
    g = torch.Generator().manual_seed(n)
    stats = DensificationStats(n, DEV)
    want = (torch.zeros(n), torch.zeros(n, 1), torch.zeros(n, 1))
    for view in range(4):
        grad = torch.randn(n, 2, generator=g) * 1e-3
        radii = torch.where(torch.rand(n, generator=g) < 0.3, torch.zeros(n), torch.rand(n, generator=g) * 20)
        if n > 2:
            radii[:2] = torch.tensor([float("nan"), -1.0])  # culled either way
        w, h = 979 + view, 546
        stats.add(grad.to(DEV), radii.to(DEV), w, h)
        want = reference_add(*want, grad, radii, w, h)
    torch.cuda.synchronize()
    assert torch.equal(stats.max_radii2D.cpu(), want[0])
    assert torch.equal(stats.denom.cpu(), want[2])
    torch.testing.assert_close(stats.means2D_grad_accum.cpu(), want[1], rtol=2e-6, atol=0.0)
