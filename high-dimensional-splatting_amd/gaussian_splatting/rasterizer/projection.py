"""EWA projection of 3D gaussians to screen-space 2D gaussians (reference rasterizer/projection.py)."""
from __future__ import annotations

import torch

NEAR_PLANE = 0.2
LOW_PASS = 0.3
JACOBIAN_FOV_SCALE = 1.3


def quat_to_rotmat(quats: torch.Tensor) -> torch.Tensor:
    """Converts (w, x, y, z) unit quaternions [N, 4] into rotation matrices [N, 3, 3] (projection.py:8-22)."""
    w, x, y, z = quats.unbind(-1)
    return torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y),
    ], dim=-1).reshape(-1, 3, 3)


class ProjectGaussians(torch.autograd.Function):
    """Projects 3D gaussians into the image plane in one HIP kernel (projection.py:25-93).

    Call it through project_gaussians with means [N, 3], activated scales [N, 3], unit quats [N, 4],
    activated opacities [N, 1], the [4, 4] world to camera transform, the intrinsics and the image size.
    Returns means2D [N, 2], depths [N] (sort key only), radii [N] (0 for every gaussian that will not
    render; no gradient) and conics [N, 3] as the inverse 2D covariance (xx, xy, yy).
    """

    @staticmethod
    def forward(ctx, means, scales, quats, opacities, world_to_camera, fx, fy, cx, cy, width, height):
        from gaussian_splatting.rasterizer import _get_rasterizer

        means, scales, quats = means.contiguous(), scales.contiguous(), quats.contiguous()
        world_to_camera = world_to_camera.to(device=means.device, dtype=torch.float32).contiguous()
        outputs = _get_rasterizer().project_gaussians(
            means, scales, quats, opacities.detach(), world_to_camera, fx, fy, cx, cy, width, height,
            NEAR_PLANE, LOW_PASS, JACOBIAN_FOV_SCALE)
        ctx.save_for_backward(means, scales, quats, world_to_camera)
        ctx.camera = (fx, fy, cx, cy, width, height)
        ctx.mark_non_differentiable(outputs[1], outputs[2])
        # Gradients of outputs the loss does not reach arrive as None instead of zero tensors
        # (depths and radii never have one; filling them would cost two N-sized writes per step).
        ctx.set_materialize_grads(False)
        return outputs

    @staticmethod
    def backward(ctx, grad_means2D, grad_depths, grad_radii, grad_conics):
        """Recomputes the projection and walks the gradients back to means, scales and quats."""
        from gaussian_splatting.rasterizer import _get_rasterizer

        means, scales, quats, world_to_camera = ctx.saved_tensors
        if grad_means2D is None:
            grad_means2D = torch.zeros(means.shape[0], 2, device=means.device)
        if grad_conics is None:
            grad_conics = torch.zeros(means.shape[0], 3, device=means.device)
        with torch.cuda.nvtx.range("project_backward"):  # a roctx range on ROCm (projection.py:88)
            grads = _get_rasterizer().project_gaussians_backward(
                grad_means2D.contiguous(), grad_conics.contiguous(), means, scales, quats, world_to_camera,
                *ctx.camera, NEAR_PLANE, LOW_PASS, JACOBIAN_FOV_SCALE)
        return (*grads, None, None, None, None, None, None, None, None)


project_gaussians = ProjectGaussians.apply
