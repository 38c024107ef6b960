"""One training iteration on the GPU against the same iteration composed from the CPU oracle.

The iteration is the reference's (main.py:159-200 there) at BASELINE config 0 (10k gaussians,
128x128, fx = fy = 140): the model's activations (exp scales, normalised quats, sigmoid opacities),
project_gaussians, eval_sh at degree 3 with its Adam step fused into the backward, rasterize,
loss = 0.8 L1 + 0.2 (1 - SSIM) against a U[0, 1] target, backward, then Adam on the other parameter
groups with the reference's learning rates (config.py:7-15 there). With 32 feature channels the
feature image joins the loss through an L1 term against a U[0, 1] feature target.

The GPU side runs this library's operators and torch's fused Adam; the CPU side runs the oracle's
stages (tests/oracle_autograd.py) and torch's plain Adam. Both start from identical parameters and
an identical Adam state (step 5, seeded first and second moments, as when training resumes), so
that the step is a smooth function of the gradients (a first Adam step is lr * sign(g), which flips
on gradients that sit at zero). Compared with assert_grads_close: every leaf gradient, means2D.grad
(which densification reads), the parameter updates of every group including sh_dc / sh_rest, and
the first and second moments of every group.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tests.oracle_autograd as orc
from gaussian_splatting.rasterizer import project_gaussians, rasterize
from gaussian_splatting.utils.loss import l1_loss, ssim
from gaussian_splatting.utils.sh import eval_sh
from tests.scenes import synthetic_config
from tests.tolerances import assert_grads_close

pytestmark = pytest.mark.gpu

DEV = "cuda"
LRS = {"means": 0.00016, "scales": 0.005, "quats": 0.001, "opacities": 0.025, "sh_dc": 0.0025,
       "sh_rest": 0.0025 / 20, "features": 0.0025}
LAMBDA_DSSIM = 0.2


def raw_params(channels: int) -> dict[str, torch.Tensor]:
    """Config 0's gaussians as the model stores them: log-scales, raw quats, opacity logits (CPU)."""
    wl = synthetic_config(0, channels=max(channels, 32))
    params = {"means": wl.means, "scales": torch.log(wl.scales), "quats": wl.quats * 1.7,
              "opacities": torch.logit(wl.opacities), "sh_dc": wl.sh_dc, "sh_rest": wl.sh_rest}
    if channels:
        params["features"] = wl.features
    return {k: v.contiguous() for k, v in params.items()}


def iteration(params, state, targets, cam, gpu: bool):
    """One training iteration; returns (leaf grads, means2D.grad, parameter updates, moments)."""
    dev = DEV if gpu else "cpu"
    leaves = {k: v.clone().to(dev).requires_grad_(True) for k, v in params.items()}
    groups = [{"params": [leaves[k]], "lr": LRS[k], "name": k} for k in leaves]
    adam = torch.optim.Adam(groups, eps=1e-15, fused=gpu, foreach=False if not gpu else None)
    for k, p in leaves.items():
        m, v = state[k]
        adam.state[p] = {"step": torch.tensor(5.0, device=dev), "exp_avg": m.clone().to(dev),
                         "exp_avg_sq": v.clone().to(dev)}
    w2c = torch.eye(4, device=dev)
    scales = torch.exp(leaves["scales"])
    quats = F.normalize(leaves["quats"], dim=-1)
    opac = torch.sigmoid(leaves["opacities"])
    if gpu:
        means2D, depths, radii, conics = project_gaussians(leaves["means"], scales, quats, opac, w2c, cam["fx"],
                                                           cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
    else:
        means2D, depths, radii, conics = orc.OracleProject.apply(leaves["means"], scales, quats, opac, w2c, cam)
    means2D.retain_grad()
    dirs = F.normalize(leaves["means"], dim=-1)  # the camera sits at the origin
    sh = eval_sh if gpu else orc.OracleEvalSH.apply
    colors = sh(leaves["sh_dc"], leaves["sh_rest"], dirs, 3, radii, adam)
    render = rasterize if gpu else orc.rasterize
    if gpu:
        out = render(means2D, depths, radii, conics, colors, opac, cam["width"], cam["height"],
                     features=leaves.get("features"))
    else:
        out = render(means2D, depths, radii, conics, colors, opac, cam["width"], cam["height"],
                     features=leaves.get("features"))
    image, fimg = out if isinstance(out, tuple) else (out, None)
    gt_image, gt_features = (t.to(dev) for t in targets)
    ssim_fn = ssim if gpu else orc.OracleSSIM.apply
    loss = (1 - LAMBDA_DSSIM) * l1_loss(image, gt_image) + LAMBDA_DSSIM * (1 - ssim_fn(image, gt_image))
    if fimg is not None:
        loss = loss + l1_loss(fimg, gt_features)
    loss.backward()
    grads = {k: p.grad.detach().cpu().clone() for k, p in leaves.items() if p.grad is not None}
    assert set(grads) == set(leaves) - {"sh_dc", "sh_rest"}, "eval_sh steps the SH groups itself"
    with torch.no_grad():
        adam.step()
    # The SH groups were stepped during the backward already: updates are taken from the start.
    updates = {k: p.detach().cpu() - params[k] for k, p in leaves.items()}
    moments = {k: (adam.state[p]["exp_avg"].cpu(), adam.state[p]["exp_avg_sq"].cpu()) for k, p in leaves.items()}
    return grads, means2D.grad.detach().cpu(), updates, moments, loss.item()


@pytest.mark.parametrize("channels", [0, 32])
def test_training_iteration_matches_the_oracle(channels):
    params = raw_params(channels)
    wl = synthetic_config(0)
    cam = wl.cam
    g = torch.Generator().manual_seed(2)
    targets = (torch.rand(cam["height"], cam["width"], 3, generator=g),
               torch.rand(cam["height"], cam["width"], max(channels, 1), generator=g))
    # Moments on the scale of each group's gradients (from a dry run's gradient magnitude, so both
    # sides start from the same smooth regime): v ~ (0.5 .. 2) * mean|g|^2, m ~ N(0, 0.5) * mean|g|.
    zero_state = {k: (torch.zeros_like(v), torch.full_like(v, 1.0)) for k, v in params.items()}
    dry, _, _, _, _ = iteration(params, zero_state, targets, cam, gpu=True)
    gs = torch.Generator().manual_seed(4)
    state = {}
    for k, v in params.items():
        scale = float(dry[k].abs().mean()) if k in dry else 1e-3
        scale = scale if scale > 0 else 1e-3
        state[k] = (0.5 * scale * torch.randn(v.shape, generator=gs),
                    scale * scale * (0.5 + 1.5 * torch.rand(v.shape, generator=gs)))

    got = iteration(params, state, targets, cam, gpu=True)
    want = iteration(params, state, targets, cam, gpu=False)
    assert math.isclose(got[4], want[4], rel_tol=1e-4), (got[4], want[4])
    names = sorted(got[0])
    assert_grads_close([f"grad {k}" for k in names], [got[0][k].numpy() for k in names], [want[0][k].numpy() for k in names])
    assert_grads_close(["means2D.grad"], [got[1].numpy()], [want[1].numpy()])
    names = sorted(params)
    assert_grads_close([f"update {k}" for k in names], [got[2][k].numpy() for k in names],
                       [want[2][k].numpy() for k in names])
    assert_grads_close([f"exp_avg {k}" for k in names], [got[3][k][0].numpy() for k in names],
                       [want[3][k][0].numpy() for k in names])
    assert_grads_close([f"exp_avg_sq {k}" for k in names], [got[3][k][1].numpy() for k in names],
                       [want[3][k][1].numpy() for k in names])
    # The SH groups did move, through the fused kernel on the GPU and the oracle on the CPU.
    assert float(got[2]["sh_dc"].abs().max()) > 0 and float(got[2]["sh_rest"].abs().max()) > 0
    assert np.isfinite(got[4])
