"""Photometric losses: L1, PSNR and SSIM with a fused HIP forward/backward (reference utils/loss.py)."""
from __future__ import annotations

from functools import lru_cache

import torch
import torch.nn.functional as F

from gaussian_splatting.rasterizer import _get_rasterizer

C1 = 0.01 ** 2
C2 = 0.03 ** 2


def l1_loss(rendered: torch.Tensor, gt: torch.Tensor) -> torch.Tensor:
    """Mean absolute error between a render and its ground truth."""
    return (rendered - gt).abs().mean()


def psnr(rendered: torch.Tensor, gt: torch.Tensor) -> torch.Tensor:
    """Peak signal to noise ratio in dB, for images in [0, 1]."""
    return -10.0 * torch.log10(((rendered - gt) ** 2).mean())


@lru_cache(maxsize=4)
def _window(size: int, sigma: float, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    """[3, 1, size, size] normalised Gaussian window for grouped conv2d (utils/loss.py:38-54)."""
    coords = torch.arange(size, device=device, dtype=dtype) - (size - 1) / 2
    g = torch.exp(-coords ** 2 / (2 * sigma ** 2))
    g = g / g.sum()
    return (g[:, None] * g[None, :]).expand(3, 1, size, size).contiguous()


class FusedSSIM(torch.autograd.Function):
    """Mean SSIM with one HIP kernel each way (utils/loss.py:57-89)."""

    @staticmethod
    def forward(ctx, rendered: torch.Tensor, gt: torch.Tensor) -> torch.Tensor:
        ssim_map, d_mu, d_aa, d_ab = _get_rasterizer().ssim_forward(rendered, gt)
        ctx.save_for_backward(rendered, gt, d_mu, d_aa, d_ab)
        return ssim_map.mean()

    @staticmethod
    def backward(ctx, grad_mean: torch.Tensor):
        rendered, gt, d_mu, d_aa, d_ab = ctx.saved_tensors
        grad = _get_rasterizer().ssim_backward(grad_mean.reshape(1).contiguous(), rendered, gt, d_mu, d_aa, d_ab)
        return grad, None


def ssim(rendered: torch.Tensor, gt: torch.Tensor, size: int = 11, sigma: float = 1.5) -> torch.Tensor:
    """Mean structural similarity over every pixel and channel of [H, W, 3] images, 1 when identical.

    GPU float32 inputs with the default 11-tap, sigma 1.5 window always run the fused HIP kernels (and
    raise if the library is missing). Other windows, dtypes or devices take the reference's own general
    conv2d formulation (utils/loss.py:110-133), as the reference does.
    """
    if rendered.is_cuda and rendered.dtype == torch.float32 and size == 11 and sigma == 1.5:
        return FusedSSIM.apply(rendered.contiguous(), gt.detach().contiguous())

    a = rendered.permute(2, 0, 1).unsqueeze(0)
    b = gt.permute(2, 0, 1).unsqueeze(0)
    window = _window(size, sigma, a.device, a.dtype)

    def blur(t: torch.Tensor) -> torch.Tensor:
        return F.conv2d(t, window, padding=size // 2, groups=3)

    mu_a, mu_b = blur(a), blur(b)
    mu_a2, mu_b2, mu_ab = mu_a * mu_a, mu_b * mu_b, mu_a * mu_b
    var_a = blur(a * a) - mu_a2
    var_b = blur(b * b) - mu_b2
    cov = blur(a * b) - mu_ab
    numerator = (2 * mu_ab + C1) * (2 * cov + C2)
    denominator = (mu_a2 + mu_b2 + C1) * (var_a + var_b + C2)
    return (numerator / denominator).mean()
