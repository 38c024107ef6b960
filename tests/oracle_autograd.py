"""The CPU oracle as torch autograd functions on CPU tensors. TEST INFRASTRUCTURE ONLY.

Composes the oracle's stages (oracle/hds_oracle.c) the way the library's Python layer composes its
HIP calls, so that a whole training iteration of the reference (main.py:159-200 there: projection,
eval_sh with its Adam-fused backward, rasterize, 0.8 L1 + 0.2 (1 - SSIM), backward, Adam) can run on
the CPU and be compared with the same iteration on the GPU. Every forward and backward below is an
oracle call; torch supplies only the chain rule, the activations and torch.optim.Adam.
"""
from __future__ import annotations

import numpy as np
import torch

import oracle

_NEAR, _LOW_PASS, _FOV = 0.2, 0.3, 1.3  # projection.py:3-5 there


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().numpy()


class OracleProject(torch.autograd.Function):
    """project_gaussians (projection.py:39-96 there): means2D, depths, radii, conics; the backward
    gives means, scales and quats, never depths or radii."""

    @staticmethod
    def forward(ctx, means, scales, quats, opacities, w2c, cam):
        m2, d, r, c = oracle.project_forward(_np(means), _np(scales), _np(quats), _np(opacities), _np(w2c),
                                             cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"],
                                             _NEAR, _LOW_PASS, _FOV)
        ctx.save_for_backward(means, scales, quats, w2c)
        ctx.cam = cam
        depths, radii = torch.from_numpy(d), torch.from_numpy(r)
        ctx.mark_non_differentiable(depths, radii)
        return torch.from_numpy(m2), depths, radii, torch.from_numpy(c)

    @staticmethod
    def backward(ctx, g_m2, g_d, g_r, g_c):
        means, scales, quats, w2c = ctx.saved_tensors
        cam = ctx.cam
        g_m2 = torch.zeros(means.shape[0], 2) if g_m2 is None else g_m2
        g_c = torch.zeros(means.shape[0], 3) if g_c is None else g_c
        dm, ds, dq = oracle.project_backward(_np(g_m2), _np(g_c), _np(means), _np(scales), _np(quats), _np(w2c),
                                             cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"],
                                             _NEAR, _LOW_PASS, _FOV)
        return torch.from_numpy(dm), torch.from_numpy(ds), torch.from_numpy(dq), None, None, None


def _adam_slot(optimizer: torch.optim.Adam, name: str):
    """The named group's parameter and Adam state, created as torch's Adam creates it, with this step
    counted (utils/sh.py:89-109 there)."""
    group = next(g for g in optimizer.param_groups if g["name"] == name)
    param = group["params"][0]
    state = optimizer.state[param]
    if not state:
        state["step"] = torch.zeros((), dtype=torch.float32)
        state["exp_avg"] = torch.zeros_like(param)
        state["exp_avg_sq"] = torch.zeros_like(param)
    state["step"] += 1
    return param, group, state


class OracleEvalSH(torch.autograd.Function):
    """eval_sh with the SH Adam step fused into the backward (utils/sh.py:26-86 there): returns only
    grad_dirs and steps sh_dc / sh_rest and their moments in place."""

    @staticmethod
    def forward(ctx, sh_dc, sh_rest, dirs, degree, radii, optimizer):
        ctx.save_for_backward(dirs, radii)
        ctx.degree, ctx.optimizer = degree, optimizer
        return torch.from_numpy(oracle.eval_sh(_np(sh_dc), _np(sh_rest), _np(dirs), degree, _np(radii)))

    @staticmethod
    def backward(ctx, grad_rgb):
        dirs, radii = ctx.saved_tensors
        dc, dc_group, dc_state = _adam_slot(ctx.optimizer, "sh_dc")
        rest, rest_group, rest_state = _adam_slot(ctx.optimizer, "sh_rest")
        beta1, beta2 = dc_group["betas"]
        arrays = [t.data.numpy() for t in (dc, rest, dc_state["exp_avg"], dc_state["exp_avg_sq"],
                                           rest_state["exp_avg"], rest_state["exp_avg_sq"])]
        grad_dirs = oracle.eval_sh_backward_adam(_np(grad_rgb), arrays[0], arrays[1], _np(dirs), ctx.degree,
                                                 _np(radii), arrays[2], arrays[3], arrays[4], arrays[5],
                                                 float(dc_state["step"]), float(rest_state["step"]), dc_group["lr"],
                                                 rest_group["lr"], beta1, beta2, dc_group["eps"])
        return None, None, torch.from_numpy(grad_dirs), None, None, None


class OracleRasterize(torch.autograd.Function):
    """rasterize (rasterizer/__init__.py:57-211 there): binning, front-to-back blend of RGB and
    optional features, and the back-to-front replay backward."""

    @staticmethod
    def forward(ctx, means2D, depths, radii, conics, colors, opacities, features, width, height):
        m2, d, r, c, col, op = (_np(t) for t in (means2D, depths, radii, conics, colors, opacities))
        feats = None if features is None else _np(features)
        _, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, width, height)
        bg = np.zeros(3, np.float32)
        image, T, nc, fimg = oracle.render_forward(width, height, ranges, values, m2, c, op, col, bg, feats)
        ctx.saved = (values, ranges, m2, c, op, col, bg, T, nc, feats)
        ctx.size = (width, height)
        if features is None:
            return torch.from_numpy(image)
        return torch.from_numpy(image), torch.from_numpy(fimg)

    @staticmethod
    def backward(ctx, grad_image, grad_features=None):
        values, ranges, m2, c, op, col, bg, T, nc, feats = ctx.saved
        width, height = ctx.size
        gf = None
        if feats is not None:
            gf = np.zeros((height, width, feats.shape[1]), np.float32) if grad_features is None else _np(grad_features)
        dm, dc, dcol, dop, df = oracle.render_backward(width, height, ranges, values, m2, c, op, col, bg, T, nc,
                                                       _np(grad_image), feats, gf)
        g_feat = None if df is None else torch.from_numpy(df)
        return (torch.from_numpy(dm), None, None, torch.from_numpy(dc), torch.from_numpy(dcol),
                torch.from_numpy(dop.reshape(-1, 1)), g_feat, None, None)


class OracleSSIM(torch.autograd.Function):
    """Mean SSIM of [H, W, 3] images with the 11-tap sigma 1.5 window (utils/loss.py:57-89 there)."""

    @staticmethod
    def forward(ctx, rendered, gt):
        ssim_map, d_mu, d_aa, d_ab = oracle.ssim_forward(_np(rendered), _np(gt))
        ctx.saved = (_np(rendered), _np(gt), d_mu, d_aa, d_ab)
        return torch.tensor(float(np.mean(ssim_map, dtype=np.float64)), dtype=torch.float32)

    @staticmethod
    def backward(ctx, grad_mean):
        a, b, d_mu, d_aa, d_ab = ctx.saved
        return torch.from_numpy(oracle.ssim_backward(float(grad_mean), a, b, d_mu, d_aa, d_ab)), None


def rasterize(means2D, depths, radii, conics, colors, opacities, width, height, features=None):
    return OracleRasterize.apply(means2D, depths, radii, conics, colors, opacities, features, width, height)
