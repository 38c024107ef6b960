"""Seeded synthetic scenes for tests and the bench. Generated on the CPU with torch.Generator, then
moved to the device, so the CPU oracle and the GPU see identical bits.

`gaussians()` follows the reference's property-test scenes (tests/scenes.py:12-30 there: means in a
4x3x4 box 1-5 units in front of an identity camera, focal 0.8*W); `synthetic_config()` builds the
five BASELINE.json workloads (seeds: geometry 0, features 1, targets / upstream gradients 2).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F


def gaussians(seed: int, n: int, channels: int = 3, device: str | torch.device = "cpu") -> dict[str, torch.Tensor]:
    """Random 3D gaussians in front of an identity camera: means, scales, quats, opacities, colors."""
    g = torch.Generator().manual_seed(seed)
    rand = lambda *shape: torch.rand(*shape, generator=g)  # noqa: E731
    means = rand(n, 3) * torch.tensor([4.0, 3.0, 4.0]) + torch.tensor([-2.0, -1.5, 1.0])
    scales = torch.exp(rand(n, 3) * 3 - 4.5)
    quats = F.normalize(torch.randn(n, 4, generator=g), dim=-1)
    opacities = rand(n, 1) * 0.95 + 0.04
    colors = rand(n, channels)
    out = {"means": means, "scales": scales, "quats": quats, "opacities": opacities, "colors": colors}
    return {k: v.to(device) for k, v in out.items()}


def camera(width: int, height: int) -> dict:
    """The reference tests' camera: focal 0.8*W, principal point at the centre."""
    focal = 0.8 * width
    return {"fx": focal, "fy": focal, "cx": width / 2, "cy": height / 2, "width": width, "height": height}


@dataclass
class Workload:
    name: str
    n: int
    width: int
    height: int
    focal: float
    channels: int
    means: torch.Tensor
    scales: torch.Tensor
    quats: torch.Tensor
    opacities: torch.Tensor
    sh_dc: torch.Tensor
    sh_rest: torch.Tensor
    features: torch.Tensor
    w2c: torch.Tensor | None = None  # [4, 4] world-to-camera; the identity when None
    intrinsics: tuple[float, float, float, float] | None = None  # (fx, fy, cx, cy); centred `focal` when None
    sh_degree: int = 3

    @property
    def cam(self) -> dict:
        fx, fy, cx, cy = self.intrinsics or (self.focal, self.focal, self.width / 2, self.height / 2)
        return {"fx": fx, "fy": fy, "cx": cx, "cy": cy, "width": self.width, "height": self.height}

    @property
    def world_to_camera(self) -> torch.Tensor:
        return torch.eye(4, device=self.means.device) if self.w2c is None else self.w2c

    @property
    def center(self) -> torch.Tensor:
        """Camera position in world space: -R^T t."""
        m = self.world_to_camera
        return -(m[:3, :3].T @ m[:3, 3])

    def to(self, device) -> "Workload":
        fields = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return Workload(**fields)


# (name, N, W, H, f, C, x half-range, y half-range, z range, log-scale mean, std, opacity logit mean, std)
CONFIGS = [
    ("cpu-plumbing-10k-128x128-c32", 10_000, 128, 128, 140.0, 32, 1.0, 1.0, (2.0, 6.0), -3.5, 0.5, 0.0, 1.5),
    ("mid-200k-979x546-c32", 200_000, 979, 546, 580.0, 32, 5.0, 3.0, (2.0, 12.0), -4.5, 0.7, 0.0, 1.5),
    ("headline-1.18M-979x546-c128", 1_180_000, 979, 546, 580.0, 128, 5.0, 3.0, (2.0, 12.0), -5.0, 0.8, 0.0, 1.5),
    ("sweep-1.18M-979x546", 1_180_000, 979, 546, 580.0, 128, 5.0, 3.0, (2.0, 12.0), -5.0, 0.8, 0.0, 1.5),
    ("stress-4M-1920x1080-c256", 4_000_000, 1920, 1080, 1100.0, 256, 5.0, 3.0, (2.0, 12.0), -4.0, 1.2, 1.0, 1.0),
]


def synthetic_config(index: int, channels: int | None = None, n: int | None = None) -> Workload:
    """BASELINE.json config `index` (0-4) on the CPU: identity world-to-camera, principal point at the centre."""
    name, n_cfg, w, h, f, c, hx, hy, (z0, z1), ls_mu, ls_sd, op_mu, op_sd = CONFIGS[index]
    n = n_cfg if n is None else n
    c = c if channels is None else channels
    g = torch.Generator().manual_seed(0)
    means = torch.empty(n, 3)
    means[:, 0] = (torch.rand(n, generator=g) * 2 - 1) * hx
    means[:, 1] = (torch.rand(n, generator=g) * 2 - 1) * hy
    means[:, 2] = z0 + torch.rand(n, generator=g) * (z1 - z0)
    scales = torch.exp(ls_mu + ls_sd * torch.randn(n, 3, generator=g))
    quats = F.normalize(torch.randn(n, 4, generator=g), dim=-1)
    opacities = torch.sigmoid(op_mu + op_sd * torch.randn(n, 1, generator=g))
    sh_dc = 0.5 * torch.randn(n, 1, 3, generator=g)
    sh_rest = 0.05 * torch.randn(n, 15, 3, generator=g)
    gf = torch.Generator().manual_seed(1)
    features = torch.randn(n, c, generator=gf)
    if c != CONFIGS[index][5]:
        name = name.rsplit("-c", 1)[0] + f"-c{c}"  # the name states the channel count actually used
    return Workload(name, n, w, h, f, c, means, scales, quats, opacities, sh_dc, sh_rest, features)


def upstream(seed: int, height: int, width: int, channels: int, device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """dL/dimage and dL/dfeature_image ~ U[0, 1] (bench/harness.py:49-50 uses the same)."""
    g = torch.Generator().manual_seed(seed)
    grad_image = torch.rand(height, width, 3, generator=g)
    grad_features = torch.rand(height, width, channels, generator=g)
    return grad_image.to(device), grad_features.to(device)


def view_dirs(means: torch.Tensor, center: torch.Tensor | None = None) -> torch.Tensor:
    """normalize(mean - camera centre): the directions eval_sh takes (utils/gaussian.py:110 there)."""
    center = torch.zeros(3, device=means.device) if center is None else center
    return F.normalize(means - center, dim=-1)


def flat_scene(means2D: list, depths: list, sigmas: list, opacities: list, device="cpu", seed: int | None = None):
    """Round gaussians placed directly in pixels (reference test_render.py:137-152): radii 1, conics
    sigma^-2 I, colours U[0, 1] from a generator seeded with n."""
    n = len(depths)
    sigma = torch.tensor(sigmas, dtype=torch.float32)
    g = torch.Generator().manual_seed(n if seed is None else seed)
    out = (
        torch.tensor(means2D, dtype=torch.float32).reshape(n, 2),
        torch.tensor(depths, dtype=torch.float32),
        torch.ones(n),
        torch.stack([sigma ** -2, torch.zeros_like(sigma), sigma ** -2], dim=-1).reshape(n, 3),
        torch.rand(n, 3, generator=g),
        torch.tensor(opacities, dtype=torch.float32)[:, None],
    )
    return tuple(t.to(device) for t in out)


def tiles(width: int, height: int) -> int:
    return math.ceil(width / 16) * math.ceil(height / 16)


def tile_selection(ranges: np.ndarray, tiles_x: int, seed: int = 0, longest: int = 16, random: int = 48) -> np.ndarray:
    """Mask of the `longest` tiles with the longest lists plus `random` other tiles drawn with `seed`."""
    lens = ranges[:, 1] - ranges[:, 0]
    order = np.argsort(-lens, kind="stable")
    mask = np.zeros(lens.size, bool)
    mask[order[:longest]] = True
    rest = np.flatnonzero(~mask)
    mask[np.random.default_rng(seed).choice(rest, random, replace=False)] = True
    return mask


def pixel_mask(tile_mask: np.ndarray, width: int, height: int) -> np.ndarray:
    """[H, W] bool: the pixels of the selected 16x16 tiles."""
    tiles_x = (width + 15) // 16
    grid = tile_mask.reshape(-1, tiles_x)
    full = np.repeat(np.repeat(grid, 16, axis=0), 16, axis=1)
    return full[:height, :width]
