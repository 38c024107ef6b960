"""The reference's training checkpoint (`model.pt`, gaussian_splatting/main.py:86-94).

A checkpoint is a torch-saved dict: "params" (name -> CPU tensor: means [N,3], scales [N,3] as
log-scales, quats [N,4] unnormalised (w, x, y, z), opacities [N,1] as logits, sh_dc [N,1,3], sh_rest
[N,K,3]), "active_sh_degree", "iteration" and "test_psnr". `load_checkpoint` reads one with torch's
weights-only loader (nothing in the file is executed) and exposes the activated tensors the way the
reference's GaussianModel does (utils/gaussian.py:64-98: exp scales, normalised quats, sigmoid
opacities), which is what the reference's bench harness feeds the rasterizer (bench/harness.py:25-30).
`save_checkpoint` writes the same layout.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch
import torch.nn.functional as F

PARAM_SHAPES = {"means": (3,), "scales": (3,), "quats": (4,), "opacities": (1,), "sh_dc": (1, 3)}


@dataclass
class Checkpoint:
    params: dict[str, torch.Tensor]
    active_sh_degree: int
    iteration: int
    test_psnr: float

    @property
    def n(self) -> int:
        return self.params["means"].shape[0]

    @property
    def means(self) -> torch.Tensor:
        return self.params["means"]

    @property
    def scales(self) -> torch.Tensor:
        return torch.exp(self.params["scales"])

    @property
    def quats(self) -> torch.Tensor:
        return F.normalize(self.params["quats"], dim=-1)

    @property
    def opacities(self) -> torch.Tensor:
        return torch.sigmoid(self.params["opacities"])


def load_checkpoint(path: str | Path, device: torch.device | str = "cpu") -> Checkpoint:
    """Reads a model.pt (weights only) and moves its parameters to `device` as contiguous float32.

    Raises:
        ValueError: a missing key or a parameter of the wrong shape.
    """
    state = torch.load(Path(path), map_location="cpu", weights_only=True)
    for key in ("params", "active_sh_degree"):
        if key not in state:
            raise ValueError(f"{path}: not a model.pt checkpoint (no {key!r})")
    params = state["params"]
    n = params["means"].shape[0] if "means" in params else -1
    for name, tail in PARAM_SHAPES.items():
        if name not in params or tuple(params[name].shape) != (n, *tail):
            got = tuple(params[name].shape) if name in params else None
            raise ValueError(f"{path}: parameter {name!r} has shape {got}, expected ({n}, {', '.join(map(str, tail))})")
    rest = params.get("sh_rest")
    if rest is None or rest.dim() != 3 or rest.shape[0] != n or rest.shape[2] != 3 or rest.shape[1] not in (0, 3, 8, 15):
        raise ValueError(f"{path}: parameter 'sh_rest' must be [N, (degree+1)^2 - 1, 3]")
    degree = int(state["active_sh_degree"])
    if not 0 <= degree <= 3 or (degree + 1) ** 2 - 1 > rest.shape[1]:
        raise ValueError(f"{path}: active_sh_degree {degree} needs more SH coefficients than the file holds")
    moved = {k: v.to(device=device, dtype=torch.float32).contiguous() for k, v in params.items()}
    return Checkpoint(moved, degree, int(state.get("iteration", 0)), float(state.get("test_psnr", float("nan"))))


def save_checkpoint(path: str | Path, params: dict[str, torch.Tensor], active_sh_degree: int, iteration: int,
                    test_psnr: float) -> None:
    """Writes `params` (raw, unactivated) in the reference's model.pt layout (main.py:86-94)."""
    torch.save({"params": {name: p.detach().cpu() for name, p in params.items()},
                "active_sh_degree": int(active_sh_degree), "iteration": int(iteration), "test_psnr": float(test_psnr)},
               Path(path))


@dataclass
class CameraView:
    """One camera as the reference's dataset holds it (utils/dataset.py:11-22), without the image."""
    world_to_camera: torch.Tensor  # [4, 4] float32
    fx: float
    fy: float
    cx: float
    cy: float
    width: int
    height: int
    name: str = ""

    @property
    def center(self) -> torch.Tensor:
        """Camera position in world space: -R^T t of the world-to-camera transform."""
        rot, t = self.world_to_camera[:3, :3], self.world_to_camera[:3, 3]
        return -(rot.T @ t)


def load_camera(path: str | Path) -> CameraView:
    """Reads a camera from JSON: {"world_to_camera": 4x4 nested list, "fx", "fy", "cx", "cy", "width",
    "height", optional "name"}. The reference reads its cameras from a COLMAP scene (utils/dataset.py),
    which has no loader here; this file carries the one view the bench harness renders
    (bench/harness.py:224).

    Raises:
        ValueError: a missing field, a matrix that is not 4x4 with a last row of (0, 0, 0, 1), or a
        non-positive size or focal length.
    """
    import json

    spec = json.loads(Path(path).read_text())
    missing = [k for k in ("world_to_camera", "fx", "fy", "cx", "cy", "width", "height") if k not in spec]
    if missing:
        raise ValueError(f"{path}: camera is missing {', '.join(missing)}")
    w2c = torch.tensor(spec["world_to_camera"], dtype=torch.float32)
    if w2c.shape != (4, 4) or not torch.equal(w2c[3], torch.tensor([0.0, 0.0, 0.0, 1.0])):
        raise ValueError(f"{path}: world_to_camera must be a 4x4 rigid transform with last row (0, 0, 0, 1)")
    view = CameraView(w2c, float(spec["fx"]), float(spec["fy"]), float(spec["cx"]), float(spec["cy"]),
                      int(spec["width"]), int(spec["height"]), str(spec.get("name", "")))
    if view.width <= 0 or view.height <= 0 or view.fx <= 0 or view.fy <= 0:
        raise ValueError(f"{path}: width, height, fx and fy must be positive")
    return view


def save_camera(path: str | Path, view: CameraView) -> None:
    """Writes `view` in the JSON form load_camera reads."""
    import json

    Path(path).write_text(json.dumps({"name": view.name, "world_to_camera": view.world_to_camera.tolist(),
                                      "fx": view.fx, "fy": view.fy, "cx": view.cx, "cy": view.cy,
                                      "width": view.width, "height": view.height}, indent=1))
