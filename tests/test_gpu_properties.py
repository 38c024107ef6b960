"""Invariants of the HIP blend that hold whatever the scene (the properties the reference's
tests/test_properties.py:44-320 checks on its CUDA path), run through the public Python API on
hypothesis-drawn scene sizes.

Tolerances: images rendered twice with the same geometry order are compared bit for bit; anything
that changes the floating-point order (mirroring, moving the camera, other weights) uses the parity
bars (RGB max 2e-3 / p99 1e-4, features max 1e-3 / p99 5e-4) scaled by the number of renders that
feed the comparison, or the reference's 1e-2 where one gaussian may flip across the 1/255 cut.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from hypothesis import example, given, settings, strategies as st

from gaussian_splatting.rasterizer import project_gaussians, rasterize
from gaussian_splatting.rasterizer.projection import quat_to_rotmat
from tests.scenes import camera, gaussians

pytestmark = pytest.mark.gpu

DEV = "cuda"
CHANNELS = [32, 64, 128]
FEATURE_MAX, FEATURE_P99 = 1e-3, 5e-4
FLIP_MAX = 1e-2  # one gaussian crossing the 1/255 cut between two float orders


def sizes():
    """(seed, n, width, height): small scenes with ragged image sizes (not multiples of 16)."""
    return st.tuples(st.integers(0, 10_000), st.integers(1, 1500), st.integers(17, 150), st.integers(17, 110))


def examples(fn):
    """Always include a one-gaussian scene, a crowded ragged image and a one-tile-high strip."""
    for ex in [(0, 1, 17, 17), (1, 1500, 16 * 9 + 3, 16 * 5 + 7), (2, 400, 150, 17)]:
        fn = example(sizes=ex)(fn)
    return fn


def project(g, width, height, world_to_camera=None):
    """Projection of gaussians() output with the reference tests' camera: the rasterize inputs."""
    cam = camera(width, height)
    w2c = torch.eye(4, device=DEV) if world_to_camera is None else world_to_camera
    means2D, depths, radii, conics = project_gaussians(g["means"], g["scales"], g["quats"], g["opacities"], w2c,
                                                       cam["fx"], cam["fy"], cam["cx"], cam["cy"], width, height)
    return means2D, depths, radii, conics, g["colors"], g["opacities"]


def scene(seed, n, width, height):
    return project(gaussians(seed, n, device=DEV), width, height)


def rand(g, *shape):
    return torch.rand(*shape, generator=g).to(DEV)


def assert_close_image(got, want, max_error, p99):
    diff = (got.double() - want.double()).abs().flatten()
    if diff.numel() == 0:
        return
    q = diff.sort().values[max(0, math.ceil(0.99 * diff.numel()) - 1)].item()
    assert diff.max().item() < max_error and q < p99, f"max {diff.max().item():.2e}, 99th {q:.2e}"


def assert_grads_close(got, want, names=("means2D", "conics", "colors", "opacities", "features")):
    for name, a, b in zip(names, got, want):
        a, b = a.double().cpu().numpy(), b.double().cpu().numpy()
        scale = max(np.abs(b).max(), 1e-30)
        bad = ~np.isclose(a, b, rtol=1e-3, atol=1e-4 * scale)
        assert bad.mean() < 1e-3, f"{name}: {bad.sum()} of {bad.size} outside tolerance"


def render_with_grads(inputs, features, width, height, grad_image, grad_features):
    means2D, depths, radii, conics, colors, opacities = inputs
    leaves = [t.detach().clone().requires_grad_(True) for t in (means2D, conics, colors, opacities, features)]
    image, fimg = rasterize(leaves[0], depths, radii, leaves[1], leaves[2], leaves[3], width, height,
                            features=leaves[4])
    torch.autograd.backward((image, fimg), (grad_image, grad_features))
    return image.detach(), fimg.detach(), [t.grad for t in leaves]


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
def test_forward_is_bitwise_deterministic_and_backward_reproducible(channels, sizes):
    seed, n, width, height = sizes
    inputs = scene(seed, n, width, height)
    g = torch.Generator().manual_seed(seed)
    features = rand(g, n, channels)
    gi, gf = rand(g, height, width, 3), rand(g, height, width, channels)
    image, fimg, grads = render_with_grads(inputs, features, width, height, gi, gf)
    image2, fimg2, grads2 = render_with_grads(inputs, features, width, height, gi, gf)
    assert torch.equal(image, image2) and torch.equal(fimg, fimg2)
    # Atomic accumulation order differs between runs: equal up to rounding.
    assert_grads_close(grads2, grads)


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
def test_input_order_of_gaussians_does_not_matter(channels, sizes):
    seed, n, width, height = sizes
    means2D, depths, radii, conics, colors, opacities = scene(seed, n, width, height)
    # Depth ranks keep the same front-to-back order with every tie broken.
    depths = depths.argsort().argsort().float()
    inputs = (means2D, depths, radii, conics, colors, opacities)
    g = torch.Generator().manual_seed(seed)
    features = rand(g, n, channels)
    gi, gf = rand(g, height, width, 3), rand(g, height, width, channels)
    perm = torch.randperm(n, generator=g).to(DEV)
    image, fimg, grads = render_with_grads(inputs, features, width, height, gi, gf)
    p_image, p_fimg, p_grads = render_with_grads(tuple(t[perm] for t in inputs), features[perm], width, height, gi, gf)
    assert torch.equal(image, p_image) and torch.equal(fimg, p_fimg)
    inv = perm.argsort()
    assert_grads_close([t[inv] for t in p_grads], grads)


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
@torch.no_grad()
def test_invisible_gaussians_change_nothing(channels, sizes):
    seed, n, width, height = sizes
    visible = gaussians(seed, n, device=DEV)
    g = torch.Generator().manual_seed(seed)
    features = rand(g, n, channels)
    transparent = gaussians(seed + 1, 200, device=DEV)
    transparent["opacities"].zero_()
    behind = gaussians(seed + 2, 200, device=DEV)
    behind["means"][:, 2] *= -1
    off_screen = gaussians(seed + 3, 200, device=DEV)
    off_screen["means"][:, 0] += 25
    everything = {k: torch.cat([visible[k], transparent[k], behind[k], off_screen[k]]) for k in visible}
    image, fimg = rasterize(*project(visible, width, height), width, height, features=features)
    image_all, fimg_all = rasterize(*project(everything, width, height), width, height,
                                    features=torch.cat([features, rand(g, 600, channels)]))
    # Culled gaussians never reach a tile list, so every list, and every result, is unchanged.
    assert torch.equal(image, image_all) and torch.equal(fimg, fimg_all)


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
@torch.no_grad()
def test_blend_weights_are_convex(channels, sizes):
    seed, n, width, height = sizes
    means2D, depths, radii, conics, _, opacities = scene(seed, n, width, height)
    geometry = (means2D, depths, radii, conics, torch.ones(n, 3, device=DEV), opacities)
    rgb_cover, cover = rasterize(*geometry, width, height, features=torch.ones(n, channels, device=DEV))
    # Every channel sees the same weights, bit for bit.
    assert torch.equal(cover, cover[..., :1].expand_as(cover))
    assert (cover >= 0).all() and (cover <= 1 + FEATURE_MAX).all()
    assert_close_image(cover[..., :3], rgb_cover, FEATURE_MAX, FEATURE_P99)
    constant = rasterize(*geometry, width, height, features=torch.full((n, channels), 0.3, device=DEV))[1]
    assert_close_image(constant, 0.3 * cover, 2 * FEATURE_MAX, 2 * FEATURE_P99)
    g = torch.Generator().manual_seed(seed)
    lo, hi = 0.25, 0.75
    fimg = rasterize(*geometry, width, height, features=lo + (hi - lo) * rand(g, n, channels))[1]
    assert (fimg >= lo * cover - 1e-5).all() and (fimg <= hi * cover + 1e-5).all()


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
def test_feature_channels_are_independent(channels, sizes):
    seed, n, width, height = sizes
    inputs = scene(seed, n, width, height)
    g = torch.Generator().manual_seed(seed)
    features = rand(g, n, channels)
    channel = seed % channels
    others = torch.arange(channels, device=DEV) != channel
    with torch.no_grad():
        bumped = features.clone()
        bumped[:, channel] += rand(g, n)
        fimg = rasterize(*inputs, width, height, features=features)[1]
        fimg_bumped = rasterize(*inputs, width, height, features=bumped)[1]
    assert torch.equal(fimg[..., others], fimg_bumped[..., others])
    leaf = features.clone().requires_grad_(True)
    grad = torch.zeros(height, width, channels, device=DEV)
    grad[..., channel] = rand(g, height, width)
    rasterize(*inputs, width, height, features=leaf)[1].backward(grad)
    assert (leaf.grad[:, others] == 0).all()


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
@torch.no_grad()
def test_features_blend_linearly(channels, sizes):
    seed, n, width, height = sizes
    inputs = scene(seed, n, width, height)
    g = torch.Generator().manual_seed(seed)
    first, second = rand(g, n, channels), rand(g, n, channels)
    a, b = 2.0, -0.5
    mixed = rasterize(*inputs, width, height, features=a * first + b * second)[1]
    want = a * rasterize(*inputs, width, height, features=first)[1] + b * rasterize(*inputs, width, height,
                                                                                     features=second)[1]
    k = 1 + abs(a) + abs(b)
    assert_close_image(mixed, want, k * FEATURE_MAX, k * FEATURE_P99)


@pytest.mark.parametrize("half", [32, 64])
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
def test_concatenated_features_render_like_their_halves(half, sizes):
    seed, n, width, height = sizes
    inputs = scene(seed, n, width, height)
    g = torch.Generator().manual_seed(seed)
    left, right = rand(g, n, half), rand(g, n, half)
    grad = rand(g, height, width, 2 * half)

    def run(features, grad_image):
        leaf = features.clone().requires_grad_(True)
        img = rasterize(*inputs, width, height, features=leaf)[1]
        img.backward(grad_image)
        return img.detach(), leaf.grad

    whole, whole_grad = run(torch.cat([left, right], dim=1), grad)
    l_img, l_grad = run(left, grad[..., :half].contiguous())
    r_img, r_grad = run(right, grad[..., half:].contiguous())
    # Each channel runs the same operations whatever the width and slicing: bitwise.
    assert torch.equal(whole, torch.cat([l_img, r_img], dim=-1))
    assert_grads_close([whole_grad], [torch.cat([l_grad, r_grad], dim=1)], names=("features",))


def quat_multiply(q1, q2):
    """Hamilton product (w, x, y, z); rotmat(q1 * q2) = rotmat(q1) @ rotmat(q2)."""
    w1, x1, y1, z1 = q1.unbind(-1)
    w2, x2, y2, z2 = q2.unbind(-1)
    return torch.stack([w1 * w2 - x1 * x2 - y1 * y2 - z1 * z2,
                        w1 * x2 + x1 * w2 + y1 * z2 - z1 * y2,
                        w1 * y2 - x1 * z2 + y1 * w2 + z1 * x2,
                        w1 * z2 + x1 * y2 - y1 * x2 + z1 * w2], dim=-1)


def test_quat_multiply_composes_rotations():
    g = torch.Generator().manual_seed(0)
    q1, q2 = F.normalize(torch.randn(2, 64, 4, generator=g, dtype=torch.float64), dim=-1)
    torch.testing.assert_close(quat_to_rotmat(quat_multiply(q1, q2)), quat_to_rotmat(q1) @ quat_to_rotmat(q2))


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
@torch.no_grad()
def test_mirrored_scene_renders_the_mirrored_image(channels, sizes):
    seed, n, width, height = sizes
    scene_g = gaussians(seed, n, device=DEV)
    g = torch.Generator().manual_seed(seed)
    features = rand(g, n, channels)
    image, fimg = rasterize(*project(scene_g, width, height), width, height, features=features)
    # x -> -x in camera space; the mirrored ellipsoid is the original turned half way about x.
    mirrored = dict(scene_g)
    mirrored["means"] = scene_g["means"] * torch.tensor([-1.0, 1.0, 1.0], device=DEV)
    mirrored["quats"] = quat_multiply(torch.tensor([0.0, 1.0, 0.0, 0.0], device=DEV), scene_g["quats"])
    m_image, m_fimg = rasterize(*project(mirrored, width, height), width, height, features=features)
    # cx = W / 2, so pixel x and pixel W - 1 - x see mirrored offsets; only the float order differs.
    assert_close_image(m_image, image.flip(1), FLIP_MAX, 1e-4)
    assert_close_image(m_fimg, fimg.flip(1), FLIP_MAX, 2 * FEATURE_P99)


@pytest.mark.parametrize("channels", CHANNELS)
@settings(max_examples=6, deadline=None)
@given(sizes=sizes())
@examples
@torch.no_grad()
def test_moving_scene_and_camera_together_changes_nothing(channels, sizes):
    seed, n, width, height = sizes
    scene_g = gaussians(seed, n, device=DEV)
    g = torch.Generator().manual_seed(seed)
    features = rand(g, n, channels)
    rotation = F.normalize(torch.randn(4, generator=g), dim=0).to(DEV)
    translation = torch.randn(3, generator=g).to(DEV)
    image, fimg = rasterize(*project(scene_g, width, height), width, height, features=features)
    rot = quat_to_rotmat(rotation[None])[0]
    moved = dict(scene_g)
    moved["means"] = scene_g["means"] @ rot.T + translation
    moved["quats"] = quat_multiply(rotation, scene_g["quats"])
    w2c = torch.eye(4, device=DEV)
    w2c[:3, :3] = rot.T
    w2c[:3, 3] = -rot.T @ translation
    m_image, m_fimg = rasterize(*project(moved, width, height, w2c), width, height, features=features)
    assert_close_image(m_image, image, FLIP_MAX, 1e-4)
    assert_close_image(m_fimg, fimg, FLIP_MAX, 2 * FEATURE_P99)
