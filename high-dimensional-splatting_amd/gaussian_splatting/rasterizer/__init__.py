"""Tile-binned alpha blending of projected gaussians into RGB and C-channel feature images.

Mirrors gaussian_splatting/rasterizer/__init__.py of the reference: the same `rasterize` signature and
return values, the `RasterizeGaussians` autograd node, the `FEATURE_SLICE_WIDTH` knob and
`_get_rasterizer()`, which here returns the ctypes binding of the HIP library instead of a JIT-built
CUDA extension. The forward renders RGB and features in one tile walk. The backward runs two tile
kernels side by side: a back-to-front replay for the geometry gradients (means2D, conics, opacities,
colours), and a front-to-back replay that contracts the blend weights with dL/dF for the feature
gradients.
"""
from __future__ import annotations

from typing import Any

import torch

from gaussian_splatting.rasterizer._native import HipRasterizer, black_background, default_slice_width
from gaussian_splatting.rasterizer.projection import project_gaussians  # noqa: F401

_rasterizer_module: Any | None = None

# Channels each feature backward work-group owns (32, 64 or 128, dividing C). None picks
# min(C, 128), as the reference does: every slice replays the tile walk and issues its own geometry
# atomics, so the widest slice is fastest, and dL/dF for 128 channels still fits the registers of two
# waves per SIMD.
FEATURE_SLICE_WIDTH: int | None = None


def _get_rasterizer() -> HipRasterizer:
    """Loads the HIP library on first use and caches the binding (rasterizer/__init__.py:15-54).

    Returns:
        An object exposing the reference extension's ten functions (rasterize, rasterize_backward,
        rasterize_features, rasterize_features_backward, eval_sh, eval_sh_backward_adam, ssim_forward,
        ssim_backward, project_gaussians, project_gaussians_backward) and the fused bin / render /
        render_backward calls.
    """
    global _rasterizer_module
    if _rasterizer_module is None:
        _rasterizer_module = HipRasterizer()
    return _rasterizer_module


class RasterizeGaussians(torch.autograd.Function):
    """Autograd node wrapping the HIP tile binning and alpha blend (rasterizer/__init__.py:57-165)."""

    @staticmethod
    def forward(ctx, means2D, depths, radii, conics, colors, opacities, background, features, image_width,
                image_height, grad_enabled=False):
        """Bins, then renders the image (and the feature image when features are given) in one walk.

        Returns:
            [H, W, 3] image, followed by the [H, W, D] feature image when features are given.
        """
        ext = _get_rasterizer()
        width, height = int(image_width), int(image_height)
        means2D = means2D.contiguous()
        # Training (features need a gradient and the caller records a graph): the render's work-groups
        # zero the backward's gradient buffers beside their walk. Inside forward grad mode is always
        # off, so the caller's mode comes in as grad_enabled.
        ctx.prezeroed, clear = None, None
        if features is not None and ctx.needs_input_grad[7] and grad_enabled:
            clear, ctx.prezeroed = ext.gradient_buffers(means2D.shape[0], int(features.shape[1]), means2D.device)
        # The render is enqueued before the host reads the pair count (the reference's one
        # blocking read, forward.cu:321-325), so the GPU does not idle during that read.
        bins = ext.bin_async(means2D, depths.contiguous(), radii.contiguous(), conics.contiguous(),
                             colors.contiguous(), opacities.contiguous(), width, height)
        if features is not None:
            features = features.contiguous()
        background = background.contiguous()
        conic, color_opacity, tile_ranges = bins.conic4, bins.color_opacity4, bins.tile_ranges
        image, feature_image, final_T, n_contrib = ext.render(
            means2D, conic, color_opacity, bins.values, tile_ranges, width, height, background, features,
            clear=clear)
        # A render again after a rebin: the buffers were already cleared (on this stream) by the first.
        if ext.resolve(bins):
            image, feature_image, final_T, n_contrib = ext.render(
                means2D, conic, color_opacity, bins.values, tile_ranges, width, height, background, features)
        values_sorted = bins.values
        ctx.image_size = (width, height)
        ctx.save_for_backward(means2D, conic, color_opacity, values_sorted, tile_ranges, final_T, n_contrib,
                              background, features)
        if features is None:
            return image
        return image, feature_image

    @staticmethod
    def backward(ctx, grad_image, grad_features=None):
        """Gradients of the blend for RGB and features from one library call (two kernels side by side).

        Returns:
            Gradients for means2D, conics, colors, opacities and features; None for depths, radii,
            background and the image size.
        """
        means2D, conic, color_opacity, values_sorted, tile_ranges, final_T, n_contrib, background, features = (
            ctx.saved_tensors)
        width, height = ctx.image_size
        # Frozen features still shape the geometry gradients, so the feature term runs whenever any of
        # means2D, conics, opacities or features needs a gradient (rasterizer/__init__.py:150-152).
        feature_term = (features is not None and grad_features is not None
                        and any(ctx.needs_input_grad[i] for i in (0, 3, 5, 7)))
        # One marker range (a roctx range on ROCm) for what the reference marks as rasterize_backward and
        # rasterize_features_backward (rasterizer/__init__.py:135, 153): here both are one call.
        with torch.cuda.nvtx.range("rasterize_backward"):
            g_means, g_conics, g_colors, g_opac, g_feat = _get_rasterizer().render_backward(
                means2D, conic, color_opacity, values_sorted, tile_ranges, final_T, n_contrib, width, height,
                grad_image=grad_image.contiguous(), background=background,
                features=features if feature_term else None,
                grad_feature_image=grad_features.contiguous() if feature_term else None,
                slice_width=(FEATURE_SLICE_WIDTH or default_slice_width(features.shape[1])) if feature_term else None,
                want_feature_grad=feature_term and ctx.needs_input_grad[7], prezeroed=ctx.prezeroed)
        ctx.prezeroed = None
        return g_means, None, None, g_conics, g_colors, g_opac, None, g_feat, None, None, None


def rasterize(
    means2D: torch.Tensor,
    depths: torch.Tensor,
    radii: torch.Tensor,
    conics: torch.Tensor,
    colors: torch.Tensor,
    opacities: torch.Tensor,
    image_width: int,
    image_height: int,
    background: torch.Tensor | None = None,
    features: torch.Tensor | None = None,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Alpha blends projected gaussians into an image, front to back, on 16x16 pixel tiles.

    Same contract as the reference's rasterize (rasterizer/__init__.py:168-211).

    Args:
        means2D: [N, 2] centers in pixels.
        depths: [N] camera space depths, used to sort.
        radii: [N] footprint radii in pixels, 0 for culled gaussians.
        conics: [N, 3] inverse 2D covariances as (xx, xy, yy).
        colors: [N, 3] RGB.
        opacities: [N, 1] in (0, 1).
        image_width: Output width in pixels.
        image_height: Output height in pixels.
        background: [3] RGB shown wherever the gaussians do not cover, black by default.
        features: [N, D] channels blended with the same weights over a zero background, with D one of
            32, 64, 128, 256 or 512. None renders RGB only.

    Returns:
        [H, W, 3] rendered image, or (image, [H, W, D] feature image) when features are given.
    """
    n = means2D.shape[0]
    assert means2D.shape == (n, 2)
    assert depths.shape == (n,) and radii.shape == (n,)
    assert conics.shape == (n, 3) and colors.shape == (n, 3)
    assert opacities.shape == (n, 1)
    if background is None:
        background = black_background(means2D.device) if means2D.is_cuda else torch.zeros(3, dtype=means2D.dtype)
    assert background.shape == (3,)
    assert features is None or (features.ndim == 2 and features.shape[0] == n)
    return RasterizeGaussians.apply(means2D, depths, radii, conics, colors, opacities, background, features,
                                    image_width, image_height, torch.is_grad_enabled())
