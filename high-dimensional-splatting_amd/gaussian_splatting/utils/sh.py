"""Spherical-harmonic colours with a backward fused into the Adam step (reference utils/sh.py)."""
from __future__ import annotations

import torch

from gaussian_splatting.rasterizer import _get_rasterizer

C0 = 0.28209479177387814
C1 = 0.4886025119029199
C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792, 0.5462742152960396)
C3 = (
    -0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154,
    -0.4570457994644658, 1.445305721320277, -0.5900435899266435,
)


def num_sh_coeffs(degree: int) -> int:
    """Coefficients up to and including a degree: (degree + 1) ** 2."""
    return (degree + 1) ** 2


class EvalSH(torch.autograd.Function):
    """RGB per gaussian from SH weights in one HIP kernel; the backward steps Adam instead of returning
    SH gradients (utils/sh.py:26-86).

    Call it through eval_sh(sh_dc [N,1,3], sh_rest [N,15,3], dirs [N,3], degree, radii [N], optimizer).
    """

    @staticmethod
    def forward(ctx, sh_dc, sh_rest, dirs, degree, radii, optimizer):
        sh_dc, sh_rest, dirs, radii = sh_dc.contiguous(), sh_rest.contiguous(), dirs.contiguous(), radii.contiguous()
        ctx.save_for_backward(dirs, radii)
        ctx.degree = degree
        ctx.optimizer = optimizer
        return _get_rasterizer().eval_sh(sh_dc, sh_rest, dirs, degree, radii)

    @staticmethod
    def backward(ctx, grad_rgb):
        """Steps sh_dc / sh_rest in place with Adam and returns only the gradient for dirs."""
        if ctx.optimizer is None:
            raise RuntimeError("eval_sh backward needs the Adam that holds sh_dc and sh_rest, set model.sh_optimizer")
        dirs, radii = ctx.saved_tensors
        dc, dc_group, dc_state = _adam_slot(ctx.optimizer, "sh_dc")
        rest, rest_group, rest_state = _adam_slot(ctx.optimizer, "sh_rest")
        beta1, beta2 = dc_group["betas"]
        with torch.cuda.nvtx.range("sh_backward"):  # a roctx range on ROCm (utils/sh.py:76)
            grad_dirs = _get_rasterizer().eval_sh_backward_adam(
                grad_rgb.contiguous(), dc.data, rest.data, dirs, ctx.degree, radii,
                dc_state["exp_avg"], dc_state["exp_avg_sq"], rest_state["exp_avg"], rest_state["exp_avg_sq"],
                dc_state["step"], rest_state["step"], dc_group["lr"], rest_group["lr"], beta1, beta2, dc_group["eps"])
        return None, None, grad_dirs, None, None, None


def _adam_slot(optimizer: torch.optim.Adam, name: str) -> tuple[torch.Tensor, dict, dict]:
    """A named parameter's Adam group and state, creating the state like torch.optim.Adam(fused=True) does
    and counting this step (utils/sh.py:89-109)."""
    group = next(g for g in optimizer.param_groups if g["name"] == name)
    param = group["params"][0]
    state = optimizer.state[param]
    if not state:
        state["step"] = torch.zeros((), dtype=torch.float32, device=param.device)
        state["exp_avg"] = torch.zeros_like(param, memory_format=torch.preserve_format)
        state["exp_avg_sq"] = torch.zeros_like(param, memory_format=torch.preserve_format)
    state["step"] += 1
    return param, group, state


eval_sh = EvalSH.apply


def rgb_to_sh(rgb: torch.Tensor) -> torch.Tensor:
    """Degree-0 weights that make eval_sh return rgb from every direction (utils/sh.py:115-124)."""
    return (rgb - 0.5) / C0
