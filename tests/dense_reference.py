"""Independent float64 formulations used to pin the CPU oracle (test infrastructure, CPU only).

These are different algorithms from the oracle's, not restatements of it:
  - `dense_blend` evaluates every pixel against every visible gaussian with a cumulative product of
    (1 - alpha) over the depth-sorted list (the formulation of the reference's tests/oracle.py:9-77):
    no tiles, no per-tile sort, no early-exit loop; torch autograd through it gives the backward.
  - `project_torch` is the EWA projection written with torch matrix products in float64 (the
    reference's projection.py describes the same math), differentiated by autograd.
  - `ssim_torch` is textbook SSIM with a 2D conv2d window (reference utils/loss.py:110-133).
  - `sh_closed_form` is the real SH basis of degrees 0-3 written term by term (reference
    tests/test_sh.py:13-49), and `sh_numeric` is the basis from its Legendre definition, which pins
    the constants independently.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

MIN_ALPHA = 1.0 / 255.0
MAX_ALPHA = 0.99
MIN_TRANSMITTANCE = 1e-4


def _sorted_visible(means2D, depths, radii, conics, colors, opacities):
    """The visible gaussians in blend order, as float64: means, conics, colours, opacities."""
    f64 = torch.float64
    # Equal depths keep index order; the kernels sort the float bits of the depth, which for the
    # positive depths used here orders like the values.
    order = torch.sort(depths, stable=True).indices
    order = order[radii[order] > 0]
    return order, means2D[order].to(f64), conics[order].to(f64), colors[order].to(f64), opacities[order, 0].to(f64)


def _pixel_centres(width, height):
    ys, xs = torch.meshgrid(torch.arange(height), torch.arange(width), indexing="ij")
    return torch.stack([xs, ys], dim=-1).reshape(-1, 2).to(torch.float64) + 0.5


def _blend_pixels(px, mean, conic, color, opacity, background):
    """[P, D] blend of the pixel centres px against every gaussian of the sorted visible list."""
    d = px[:, None] - mean
    dx, dy = d[..., 0], d[..., 1]
    m = dx * (conic[:, 0] * dx + conic[:, 1] * dy) + dy * (conic[:, 1] * dx + conic[:, 2] * dy)
    alpha = (opacity * torch.exp(-0.5 * m)).clamp(max=MAX_ALPHA)
    alpha = torch.where(alpha >= MIN_ALPHA, alpha, torch.zeros_like(alpha))
    post = torch.cumprod(1 - alpha, dim=1)
    pre = torch.cat([torch.ones_like(post[:, :1]), post[:, :-1]], dim=1)
    w = alpha * pre
    # A gaussian that would push T below the floor ends the pixel: it and everything behind it
    # are dropped (post is monotone, so the mask is a prefix).
    w = torch.where(post >= MIN_TRANSMITTANCE, w, torch.zeros_like(w))
    remaining = 1 - w.sum(dim=1, keepdim=True)
    return w @ color + background * remaining


def dense_blend(means2D, depths, radii, conics, colors, opacities, width, height, background=None):
    """[H, W, D] blend of every pixel against every visible gaussian, float64 torch (autograd-able)."""
    background = torch.zeros(colors.shape[1], dtype=torch.float64) if background is None else background.double()
    _, mean, conic, color, opacity = _sorted_visible(means2D, depths, radii, conics, colors, opacities)
    pixels = _pixel_centres(width, height)
    chunk = max(1, 2 ** 22 // max(1, mean.shape[0]))
    out = [_blend_pixels(px, mean, conic, color, opacity, background) for px in pixels.split(chunk)]
    return torch.cat(out).reshape(height, width, colors.shape[1])


def dense_blend_grad(means2D, depths, radii, conics, colors, opacities, width, height, grad_image,
                     chunk: int | None = None):
    """Forward and backward of dense_blend with upstream gradient grad_image [H, W, D], one pixel
    chunk at a time (`chunk` pixels, by default as many as keep one [pixels, gaussians] float64 array
    at 32 MiB; each chunk's autograd graph is freed before the next, so memory stays at one chunk's). Pixels are independent, so the chunks' gradients add up to the full frame's. Returns the
    [H, W, D] image and the float64 gradients of means2D [N, 2], conics [N, 3], colors [N, D] and
    opacities [N, 1] (zero for culled gaussians), plus the forward's and backward's seconds."""
    import time

    f64 = torch.float64
    leaves = [t.detach().to(f64).requires_grad_(True) for t in (means2D, conics, colors, opacities)]
    order, *_ = _sorted_visible(means2D, depths, radii, conics, colors, opacities)
    background = torch.zeros(colors.shape[1], dtype=f64)
    pixels = _pixel_centres(width, height)
    upstream = grad_image.reshape(-1, colors.shape[1]).to(f64)
    chunk = chunk or max(1, 2 ** 22 // max(1, order.numel()))
    out, t_fwd, t_bwd = [], 0.0, 0.0
    for start in range(0, pixels.shape[0], chunk):
        t0 = time.perf_counter()
        mean, conic, color, opacity = (leaves[0][order], leaves[1][order], leaves[2][order], leaves[3][order, 0])
        img = _blend_pixels(pixels[start:start + chunk], mean, conic, color, opacity, background)
        t1 = time.perf_counter()
        img.backward(upstream[start:start + chunk])
        t_bwd += time.perf_counter() - t1
        t_fwd += t1 - t0
        out.append(img.detach())
    grads = {name: leaf.grad for name, leaf in zip(("means2D", "conics", "colors", "opacities"), leaves)}
    return torch.cat(out).reshape(height, width, colors.shape[1]), grads, t_fwd, t_bwd


def quat_to_rotmat(q):
    w, x, y, z = q.unbind(-1)
    return torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y),
    ], dim=-1).reshape(-1, 3, 3)


def project_torch(means, scales, quats, w2c, fx, fy, cx, cy, width, height, near=0.2, low_pass=0.3, fov=1.3):
    """EWA projection with matrix algebra: returns means2D [N,2], depths [N], conics [N,3], cov2D [N,2,2]."""
    R, t = w2c[:3, :3], w2c[:3, 3]
    p = means @ R.T + t
    z = p[:, 2].clamp(min=near)
    z_inv = 1.0 / (z + 1e-6)
    lim_x, lim_y = fov * 0.5 * width / fx, fov * 0.5 * height / fy
    jx = (p[:, 0] * z_inv).clamp(-lim_x, lim_x) * z
    jy = (p[:, 1] * z_inv).clamp(-lim_y, lim_y) * z
    zero = torch.zeros_like(z)
    J = torch.stack([
        torch.stack([fx * z_inv, zero, -fx * jx * z_inv * z_inv], -1),
        torch.stack([zero, fy * z_inv, -fy * jy * z_inv * z_inv], -1)], -2)
    M = quat_to_rotmat(quats) * scales[:, None, :]
    T = J @ R @ M
    cov = T @ T.transpose(1, 2) + low_pass * torch.eye(2, dtype=means.dtype)
    det = cov[:, 0, 0] * cov[:, 1, 1] - cov[:, 0, 1] ** 2
    conic = torch.stack([cov[:, 1, 1] / det, -cov[:, 0, 1] / det, cov[:, 0, 0] / det], -1)
    u = fx * p[:, 0] / z + cx
    v = fy * p[:, 1] / z + cy
    return torch.stack([u, v], -1), p[:, 2], conic, cov


def ssim_torch(a, b, size=11, sigma=1.5):
    """Mean SSIM of [H, W, 3] images with a zero-padded 2D Gaussian window (conv2d)."""
    coords = torch.arange(size, dtype=a.dtype) - (size - 1) / 2
    g = torch.exp(-coords ** 2 / (2 * sigma ** 2))
    g = g / g.sum()
    window = (g[:, None] * g[None, :]).expand(3, 1, size, size).contiguous()
    A, B = a.permute(2, 0, 1)[None], b.permute(2, 0, 1)[None]
    blur = lambda t: F.conv2d(t, window, padding=size // 2, groups=3)  # noqa: E731
    mu_a, mu_b = blur(A), blur(B)
    va, vb, cov = blur(A * A) - mu_a ** 2, blur(B * B) - mu_b ** 2, blur(A * B) - mu_a * mu_b
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    return ((2 * mu_a * mu_b + c1) * (2 * cov + c2) / ((mu_a ** 2 + mu_b ** 2 + c1) * (va + vb + c2))).mean()


def sh_closed_form(sh, dirs, degree, radii):
    """[N, 3] colour from sh [N, 16, 3], written term by term in the 3DGS sign convention."""
    x, y, z = (dirs[:, i:i + 1] for i in range(3))
    xx, yy, zz, xy, yz, xz = x * x, y * y, z * z, x * y, y * z, x * z
    terms = [0.28209479177387814 + 0 * x]
    if degree >= 1:
        terms += [-0.4886025119029199 * y, 0.4886025119029199 * z, -0.4886025119029199 * x]
    if degree >= 2:
        terms += [1.0925484305920792 * xy, -1.0925484305920792 * yz, 0.31539156525252005 * (2 * zz - xx - yy),
                  -1.0925484305920792 * xz, 0.5462742152960396 * (xx - yy)]
    if degree >= 3:
        terms += [-0.5900435899266435 * y * (3 * xx - yy), 2.890611442640554 * xy * z,
                  -0.4570457994644658 * y * (4 * zz - xx - yy), 0.3731763325901154 * z * (2 * zz - 3 * xx - 3 * yy),
                  -0.4570457994644658 * x * (4 * zz - xx - yy), 1.445305721320277 * z * (xx - yy),
                  -0.5900435899266435 * x * (xx - 3 * yy)]
    rgb = 0.5 + sum(term * sh[:, j] for j, term in enumerate(terms))
    return torch.where(radii[:, None] > 0, rgb.clamp_min(0), torch.zeros_like(rgb))


def sh_numeric(dirs: np.ndarray, degree: int) -> np.ndarray:
    """Real SH basis [N, (degree+1)^2] from the associated Legendre definition (no hard-coded constants).

    Y_l^m = sqrt((2l+1)/(4 pi) (l-|m|)!/(l+|m|)!) P_l^|m|(cos theta) * {sqrt2 cos(m phi), 1, sqrt2 sin(|m| phi)},
    ordered m = -l..l and with the 3DGS sign convention (-1)^m folded in, so it can be compared with
    the kernels' constants term by term.
    """
    x, y, z = dirs[:, 0], dirs[:, 1], dirs[:, 2]
    theta = np.arccos(np.clip(z, -1, 1))
    phi = np.arctan2(y, x)
    cols = []
    for l in range(degree + 1):
        for m in range(-l, l + 1):
            am = abs(m)
            norm = math.sqrt((2 * l + 1) / (4 * math.pi) * math.factorial(l - am) / math.factorial(l + am))
            # Associated Legendre without the Condon-Shortley phase, by recurrence.
            p = _assoc_legendre(l, am, np.cos(theta))
            if m > 0:
                val = math.sqrt(2) * norm * p * np.cos(m * phi)
            elif m < 0:
                val = math.sqrt(2) * norm * p * np.sin(am * phi)
            else:
                val = norm * p
            cols.append(((-1) ** am) * val)
    return np.stack(cols, axis=1)


def _assoc_legendre(l: int, m: int, x: np.ndarray) -> np.ndarray:
    pmm = np.ones_like(x)
    if m > 0:
        somx2 = np.sqrt(np.maximum(0.0, 1 - x * x))
        fact = 1.0
        for _ in range(m):
            pmm = pmm * fact * somx2
            fact += 2.0
    if l == m:
        return pmm
    pmmp1 = x * (2 * m + 1) * pmm
    if l == m + 1:
        return pmmp1
    pll = pmmp1
    for ll in range(m + 2, l + 1):
        pll = ((2 * ll - 1) * x * pmmp1 - (ll + m - 1) * pmm) / (ll - m)
        pmm, pmmp1 = pmmp1, pll
    return pll
