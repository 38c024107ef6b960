"""The reference's training iteration (main.py:159-200) running on this library's operators.

One iteration: project the gaussians for a camera, colour them with eval_sh (whose backward steps
sh_dc / sh_rest with Adam inside the kernel), rasterize, score with 0.8 L1 + 0.2 (1 - SSIM), backward,
accumulate the densification statistics from means2D.grad (utils/gaussian.py:143-160, on this
library's fused kernel, checked against the reference's torch formula), then optimizer.step() on the
other parameters. The targets are renders of a known scene from four cameras orbiting it; the
trained model starts from a perturbed copy. What is checked is the integration, not a convergence
rate: every gradient is finite, means2D.grad is non-zero on the visible gaussians and zero on the
culled ones, the fused SH Adam and torch's Adam both move their parameters, and the loss falls well
below where it started (80 iterations at 128x128: about 0.05 -> 0.01, PSNR +9 dB).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from gaussian_splatting.rasterizer import project_gaussians, rasterize
from gaussian_splatting.utils.densification import DensificationStats
from gaussian_splatting.utils.loss import l1_loss, psnr, ssim
from gaussian_splatting.utils.sh import eval_sh, rgb_to_sh

pytestmark = pytest.mark.gpu

DEV = "cuda"
W = H = 128
FOCAL = 0.8 * W
LAMBDA_DSSIM = 0.2  # config.py:16


def orbit_cameras(count: int, distance: float = 5.0) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """(world_to_camera [4, 4], camera centre [3]) for cameras around the y axis, all facing the origin."""
    cams = []
    for k in range(count):
        a = 2 * math.pi * k / count * 0.25  # a quarter turn in total keeps every view on the scene's front
        rot = torch.tensor([[math.cos(a), 0.0, math.sin(a)], [0.0, 1.0, 0.0], [-math.sin(a), 0.0, math.cos(a)]])
        w2c = torch.eye(4)
        w2c[:3, :3] = rot
        w2c[2, 3] = distance
        centre = -rot.T @ w2c[:3, 3]
        cams.append((w2c.to(DEV), centre.to(DEV)))
    return cams


def scene(seed: int, n: int, channels: int) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    params = {
        "means": (torch.rand(n, 3, generator=g) * 2 - 1) * torch.tensor([1.2, 1.2, 0.6]),
        "scales": torch.randn(n, 3, generator=g) * 0.3 - 3.0,  # log-scales
        "quats": torch.randn(n, 4, generator=g),
        "opacities": torch.randn(n, 1, generator=g) + 1.0,  # logits
        "sh_dc": rgb_to_sh(torch.rand(n, 3, generator=g))[:, None, :],
        "sh_rest": 0.02 * torch.randn(n, 15, 3, generator=g),
    }
    if channels:
        params["features"] = torch.randn(n, channels, generator=g)
    return {k: v.to(DEV).contiguous() for k, v in params.items()}


def render(p: dict, cam, degree: int, optimizer=None):
    """main.py:14-40 with the model's activations (exp scales, normalised quats, sigmoid opacities)."""
    w2c, centre = cam
    opac = torch.sigmoid(p["opacities"])
    means2D, depths, radii, conics = project_gaussians(p["means"], torch.exp(p["scales"]), F.normalize(p["quats"], dim=-1),
                                                       opac, w2c, FOCAL, FOCAL, W / 2, H / 2, W, H)
    if means2D.requires_grad:
        means2D.retain_grad()
    dirs = F.normalize(p["means"] - centre, dim=-1)
    colors = eval_sh(p["sh_dc"], p["sh_rest"], dirs, degree, radii, optimizer)
    out = rasterize(means2D, depths, radii, conics, colors, opac, W, H, features=p.get("features"))
    image, feature_image = out if isinstance(out, tuple) else (out, None)
    return image, feature_image, means2D, radii


@pytest.mark.parametrize("channels", [0, 32])
def test_training_iterations_reduce_the_loss(channels):
    cams = orbit_cameras(4)
    truth = scene(0, 1500, channels)
    with torch.no_grad():
        targets = [render(truth, cam, 3)[:2] for cam in cams]

    model = {k: v.clone() for k, v in truth.items()}
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        model["means"] += 0.05 * torch.randn(model["means"].shape, generator=g).to(DEV)
        model["scales"] += 0.3 * torch.randn(model["scales"].shape, generator=g).to(DEV)
        model["opacities"].zero_()
        model["sh_dc"].copy_(rgb_to_sh(torch.full((1500, 3), 0.5)).to(DEV)[:, None, :])
        if channels:
            model["features"].mul_(0.0)
    for v in model.values():
        v.requires_grad_(True)
    lrs = {"means": 1e-3, "scales": 5e-3, "quats": 1e-3, "opacities": 5e-2, "sh_dc": 1e-2, "sh_rest": 5e-4,
           "features": 5e-2}
    optimizer = torch.optim.Adam([{"params": [model[k]], "lr": lrs[k], "name": k} for k in model], eps=1e-15,
                                 fused=True)
    stats = DensificationStats(1500, DEV)
    ref_accum, ref_denom = torch.zeros(1500, 1, device=DEV), torch.zeros(1500, 1, device=DEV)
    sh_before = model["sh_dc"].detach().clone()
    means_before = model["means"].detach().clone()

    def loss_of(image, feature_image, target):
        gt_image, gt_features = target
        loss = (1 - LAMBDA_DSSIM) * l1_loss(image, gt_image) + LAMBDA_DSSIM * (1 - ssim(image, gt_image))
        if feature_image is not None:
            loss = loss + l1_loss(feature_image, gt_features)
        return loss

    with torch.no_grad():
        start = sum(float(loss_of(*render(model, cam, 3)[:2], t)) for cam, t in zip(cams, targets)) / len(cams)
        start_psnr = sum(float(psnr(render(model, cam, 3)[0], t[0])) for cam, t in zip(cams, targets)) / len(cams)

    for it in range(80):
        k = it % len(cams)
        image, feature_image, means2D, radii = render(model, cams[k], 3, optimizer)
        loss = loss_of(image, feature_image, targets[k])
        loss.backward()
        with torch.no_grad():
            assert torch.isfinite(loss)
            grad2d = means2D.grad
            assert grad2d is not None and torch.isfinite(grad2d).all()
            visible = radii > 0
            # Densification statistics (utils/gaussian.py:143-160): norms of the screen-space gradient.
            stats.add(grad2d, radii, W, H)
            scale = torch.tensor([0.5 * W, 0.5 * H], device=DEV)
            ref_accum[visible] += (grad2d * scale)[visible].norm(dim=-1, keepdim=True)
            ref_denom[visible] += 1
            assert float(ref_accum.max()) > 0.0
            assert float(grad2d[~visible].abs().sum()) == 0.0
            for name, p in model.items():
                if name.startswith("sh_"):
                    assert p.grad is None, "eval_sh steps sh_dc / sh_rest itself and leaves no gradient"
                else:
                    assert p.grad is not None and torch.isfinite(p.grad).all(), name
            optimizer.step()
            optimizer.zero_grad(set_to_none=True)

    with torch.no_grad():
        end = sum(float(loss_of(*render(model, cam, 3)[:2], t)) for cam, t in zip(cams, targets)) / len(cams)
        end_psnr = sum(float(psnr(render(model, cam, 3)[0], t[0])) for cam, t in zip(cams, targets)) / len(cams)
    torch.testing.assert_close(stats.means2D_grad_accum, ref_accum, rtol=1e-5, atol=0.0)
    assert torch.equal(stats.denom, ref_denom)
    assert not torch.equal(model["sh_dc"].detach(), sh_before), "the fused SH Adam did not step sh_dc"
    assert not torch.equal(model["means"].detach(), means_before), "torch's Adam did not step the means"
    print(f"loss {start:.4f} -> {end:.4f}, PSNR {start_psnr:.2f} -> {end_psnr:.2f} dB")
    assert end < 0.6 * start, (start, end)
    assert end_psnr > start_psnr + 3.0, (start_psnr, end_psnr)
