"""Pins the CPU oracle (oracle/hds_oracle.c) against checks that do not restate its own formulas.

CPU only. Each stage is checked against something a plausible mistake (a dropped term, a wrong sign
or index, a transposed operand) would fail:
  - hand-solved pixels and edge cases of the reference tests (golden fixture tests/golden/);
  - the dense float64 cumprod blend and torch autograd through it (tests/dense_reference.py);
  - brute-force enumeration of tile pairs and a float64 footprint test for the binning;
  - closed forms and invariances for the projection, autograd of a matrix formulation for its backward;
  - the Legendre definition and orthonormality of the SH basis, torch.optim.Adam for the SH step;
  - torch conv2d SSIM and ssim(x, x) = 1.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests import dense_reference as ref
from tests.scenes import camera, flat_scene, gaussians, synthetic_config

GOLDEN = Path(__file__).resolve().parent / "golden"


def np_(t):
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)


def assert_image_close(got, want, max_error=2e-3, max_perc_99=1e-4):
    diff = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).ravel()
    if diff.size == 0:
        return
    p99 = np.sort(diff)[max(0, math.ceil(0.99 * diff.size) - 1)]
    assert diff.max() < max_error and p99 < max_perc_99, f"max {diff.max():.2e}, 99th {p99:.2e}"


def assert_grads_close(names, grads, wants):
    """test_render.py:45-58 criteria."""
    for name, got, want in zip(names, grads, wants):
        got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
        assert got.shape == want.shape, f"{name}: {got.shape} vs {want.shape}"
        if want.size == 0:
            continue
        scale = np.abs(want).max()
        bad = ~np.isclose(got, want, rtol=1e-3, atol=1e-4 * scale)
        assert bad.mean() < 1e-3, f"{name}: {bad.sum()} of {bad.size} outside tolerance"
        assert np.abs(got - want).max() <= 2e-3 * scale, f"{name}: max error {np.abs(got - want).max():.2e}"


def project_scene(seed, n, width, height):
    """Reference-style scene projected by the oracle: (means2D, depths, radii, conics, colors, opacities)."""
    g = gaussians(seed, n)
    cam = camera(width, height)
    m2, d, r, c = oracle.project_forward(np_(g["means"]), np_(g["scales"]), np_(g["quats"]), np_(g["opacities"]),
                                         np.eye(4), cam["fx"], cam["fy"], cam["cx"], cam["cy"], width, height)
    return m2, d, r, c, np_(g["colors"]), np_(g["opacities"])


# ---- shared arithmetic ------------------------------------------------------------------------

def test_logf_is_within_two_ulp_of_float64_log():
    rng = np.random.default_rng(0)
    xs = np.concatenate([np.exp(rng.uniform(-80, 80, 20000)), rng.uniform(0.5, 2.0, 20000),
                         [1.0, 2.0, 0.5, 255.0, 1e-38, 1e-44, 3e38]]).astype(np.float32)
    got = np.array([oracle.logf(x) for x in xs], np.float32)
    want = np.log(xs.astype(np.float64))
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - want) / ulp
    assert err.max() <= 2.0, f"max error {err.max():.2f} ulp at {xs[err.argmax()]}"
    assert oracle.logf(1.0) == 0.0
    assert oracle.logf(0.0) == -np.inf and np.isnan(oracle.logf(-1.0)) and oracle.logf(np.inf) == np.inf


def test_exp2f_is_within_one_ulp_of_float64_exp2():
    """hds_exp2f, behind every blend alpha on both CPU and GPU: at most one ulp from 2^x in double over
    the range where alpha can reach 1/255 and far beyond, exact at the integers, 0 below 2^-150."""
    rng = np.random.default_rng(4)
    xs = np.concatenate([np.linspace(-30.0, 0.5, 300001), rng.uniform(-126, 10, 100000),
                         -np.arange(0, 126), [-0.5, 0.5, -1e-7, 1e-7]]).astype(np.float32)
    got = oracle.exp2f(xs).astype(np.float64)
    want = np.exp2(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    err = np.abs(got - want) / ulp
    assert err.max() <= 1.0, f"max error {err.max():.2f} ulp at {xs[err.argmax()]}"
    ints = -np.arange(0, 126, dtype=np.float32)
    assert np.array_equal(oracle.exp2f(ints), np.exp2(ints.astype(np.float64)).astype(np.float32))
    assert oracle.exp2f(np.array([-151.0, -1e30, np.nan], np.float32)).tolist() == [0.0, 0.0, 0.0]


def test_tile_rect_covers_every_pixel_the_gaussian_can_reach():
    """Brute force in float64: a pixel with alpha >= 1/255 (a little margin) is always inside the rect."""
    rng = np.random.default_rng(1)
    width, height = 200, 150
    tiles_x, tiles_y = 13, 10
    ys, xs = np.meshgrid(np.arange(height) + 0.5, np.arange(width) + 0.5, indexing="ij")
    for _ in range(300):
        u, v = rng.uniform(-20, width + 20), rng.uniform(-20, height + 20)
        sx, sy, rho = rng.uniform(0.5, 30), rng.uniform(0.5, 30), rng.uniform(-0.9, 0.9)
        cov = np.array([[sx * sx, rho * sx * sy], [rho * sx * sy, sy * sy]])
        a, b, c = np.linalg.inv(cov)[[0, 0, 1], [0, 1, 1]]
        op = rng.uniform(0.0, 1.0)
        rect = oracle.tile_rect(u, v, a, b, c, op, tiles_x, tiles_y)
        dx, dy = xs - u, ys - v
        alpha = op * np.exp(-0.5 * (a * dx * dx + 2 * b * dx * dy + c * dy * dy))
        reach = alpha >= (1 / 255) * (1 + 1e-4)
        if rect is None:
            assert not reach.any()
            continue
        x0, y0, w, h = rect
        tx, ty = (xs // 16).astype(int), (ys // 16).astype(int)
        inside = (tx >= x0) & (tx < x0 + w) & (ty >= y0) & (ty < y0 + h)
        assert not (reach & ~inside).any()
        # And it is the ellipse's bounding box, not more: float64 extents give the same tiles
        # unless an edge sits within 1e-3 px of a tile boundary.
        k = math.sqrt(2 * math.log(op * 255))
        det = a * c - b * b
        ex, ey = k * math.sqrt(c / det), k * math.sqrt(a / det)
        edges = np.array([u - ex, u + ex, v - ey, v + ey]) / 16
        if np.abs(edges - np.round(edges)).min() > 1e-3 / 16:
            lo_x, hi_x = max(0, math.floor((u - ex) / 16)), min(tiles_x - 1, math.floor((u + ex) / 16))
            lo_y, hi_y = max(0, math.floor((v - ey) / 16)), min(tiles_y - 1, math.floor((v + ey) / 16))
            assert (x0, y0, w, h) == (lo_x, lo_y, hi_x - lo_x + 1, hi_y - lo_y + 1)


# ---- binning ----------------------------------------------------------------------------------

def test_binning_matches_brute_force_enumeration():
    m2, d, r, c, _, op = project_scene(3, 2000, 100, 70)
    counts, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, 100, 70)
    tiles_x = 7
    keys, gids = [], []
    for i in range(len(d)):
        rect = oracle.tile_rect(*m2[i], *c[i], op[i, 0], tiles_x, 5) if r[i] > 0 else None
        assert counts[i] == (0 if rect is None else rect[2] * rect[3])
        if rect is None:
            continue
        x0, y0, w, h = rect
        for ty in range(y0, y0 + h):
            for tx in range(x0, x0 + w):
                keys.append((ty * tiles_x + tx, int(np.float32(d[i]).view(np.uint32)), i))
                gids.append(i)
    keys.sort()
    assert np.array_equal(values, np.array([k[2] for k in keys], np.int32))
    want_ranges = np.zeros_like(ranges)
    tiles = np.array([k[0] for k in keys])
    for t in np.unique(tiles):
        idx = np.nonzero(tiles == t)[0]
        want_ranges[t] = (idx[0], idx[-1] + 1)
    assert np.array_equal(ranges, want_ranges)
    assert counts.sum() == values.size


def test_binning_keeps_index_order_on_depth_ties_and_drops_culled():
    means2D = np.array([[8.0, 8.0], [8.5, 8.0], [9.0, 8.0], [8.0, 9.0]], np.float32)
    depths = np.array([2.0, 1.0, 2.0, 2.0], np.float32)
    radii = np.array([1.0, 1.0, 0.0, 1.0], np.float32)
    conics = np.tile(np.array([[1.0, 0.0, 1.0]], np.float32), (4, 1))
    op = np.full((4, 1), 0.5, np.float32)
    _, values, ranges = oracle.bin_gaussians(means2D, depths, radii, conics, op, 16, 16)
    assert values.tolist() == [1, 0, 3]
    assert ranges.tolist() == [[0, 3]]


# ---- blend forward ----------------------------------------------------------------------------

def test_hand_solved_pixels_from_golden_fixture():
    fixture = json.loads((GOLDEN / "hand_solved_pixels.json").read_text())
    bg = np.array(fixture["background"], np.float32)
    for case in fixture["cases"]:
        ops = case["opacities"]
        n = len(ops)
        m2 = np.full((n, 2), 0.5, np.float32)
        depths = np.arange(n, dtype=np.float32)
        conics = np.tile(np.array([[1.0, 0.0, 1.0]], np.float32), (n, 1))
        colors = np.eye(3, dtype=np.float32)[:n]
        opac = np.array(ops, np.float32).reshape(n, 1)
        image = oracle.rasterize(m2, depths, np.ones(n, np.float32), conics, colors, opac, 1, 1, bg)[0]
        np.testing.assert_allclose(image[0, 0], case["float32_kernel"], atol=1e-6, err_msg=case["name"])
        # The float64 dense formulation reproduces the reference's hand-solved values.
        dense = ref.dense_blend(torch.tensor(m2), torch.tensor(depths), torch.ones(n), torch.tensor(conics),
                                torch.tensor(colors).reshape(n, 3), torch.tensor(opac), 1, 1,
                                torch.tensor(bg, dtype=torch.float64))
        np.testing.assert_allclose(dense[0, 0].numpy(), case["float64_reference"], atol=1e-6, err_msg=case["name"])


@pytest.mark.parametrize("seed,n,width,height,channels", [(0, 400, 48, 40, 3), (1, 1500, 33, 17, 32),
                                                          (2, 3000, 64, 48, 16)])
def test_forward_matches_dense_float64_blend(seed, n, width, height, channels):
    m2, d, r, c, col, op = project_scene(seed, n, width, height)
    feats = np.random.default_rng(seed).uniform(0, 1, (n, channels)).astype(np.float32)
    bg = np.array([0.3, 0.5, 0.7], np.float32)
    image, fimg, T, nc, _, _ = oracle.rasterize(m2, d, r, c, col, op, width, height, bg, feats)
    t = lambda a: torch.tensor(a)  # noqa: E731
    want = ref.dense_blend(t(m2), t(d), t(r), t(c), t(col), t(op), width, height, t(bg).double())
    want_f = ref.dense_blend(t(m2), t(d), t(r), t(c), t(feats), t(op), width, height)
    assert_image_close(image, want.numpy())
    assert_image_close(fimg, want_f.numpy(), max_error=1e-3, max_perc_99=5e-4)
    # Coverage: 1 - T equals the blend of all-ones features.
    ones = ref.dense_blend(t(m2), t(d), t(r), t(c), torch.ones(n, 1), t(op), width, height)
    assert_image_close(1 - T, ones[..., 0].numpy())


def test_max_alpha_clamp_and_min_alpha_cut():
    inputs = [np_(x) for x in flat_scene([[8.5, 8.5]], [1.0], [2.0], [1.0])]
    image = oracle.rasterize(*inputs, 16, 16)[0]
    np.testing.assert_allclose(image[8, 8], 0.99 * inputs[4][0], rtol=1e-6)
    inputs = [np_(x) for x in flat_scene([[4.5, 4.5], [12.5, 4.5]], [1.0, 1.0], [0.5, 0.5], [1.01 / 255, 0.99 / 255])]
    image = oracle.rasterize(*inputs, 16, 8)[0]
    assert image[4, 4].sum() > 0 and (image[4, 12] == 0).all()


def test_dense_tile_walks_past_256():
    g = torch.Generator().manual_seed(11)
    n = 2000
    means = (torch.rand(n, 2, generator=g) * 16).tolist()
    depths = (1 + torch.rand(n, generator=g)).tolist()
    inputs = [np_(x) for x in flat_scene(means, depths, [12.0] * n, [0.02] * n)]
    image, _, T, nc, _, _ = oracle.rasterize(*inputs, 16, 16, np.zeros(3, np.float32))
    assert nc.min() > 256
    t = lambda a: torch.tensor(a)  # noqa: E731
    want = ref.dense_blend(*[t(a) for a in inputs], 16, 16, torch.zeros(3, dtype=torch.float64))
    assert_image_close(image, want.numpy())


# ---- blend backward ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed,n,width,height,channels", [(4, 600, 40, 32, 8), (5, 2500, 48, 33, 32)])
def test_backward_matches_autograd_of_dense_blend(seed, n, width, height, channels):
    m2, d, r, c, col, op = project_scene(seed, n, width, height)
    rng = np.random.default_rng(seed)
    feats = rng.uniform(0, 1, (n, channels)).astype(np.float32)
    gimg = rng.uniform(0, 1, (height, width, 3)).astype(np.float32)
    gfeat = rng.uniform(0, 1, (height, width, channels)).astype(np.float32)
    bg = np.array([0.3, 0.5, 0.7], np.float32)
    _, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, width, height)
    _, T, nc, _ = oracle.render_forward(width, height, ranges, values, m2, c, op, col, bg, feats)
    got = oracle.render_backward(width, height, ranges, values, m2, c, op, col, bg, T, nc, gimg, feats, gfeat)

    leaves = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (m2, c, col, op, feats)]
    image = ref.dense_blend(leaves[0], torch.tensor(d), torch.tensor(r), leaves[1], leaves[2], leaves[3], width,
                            height, torch.tensor(bg, dtype=torch.float64))
    fimg = ref.dense_blend(leaves[0], torch.tensor(d), torch.tensor(r), leaves[1], leaves[4], leaves[3], width, height)
    torch.autograd.backward((image, fimg), (torch.tensor(gimg, dtype=torch.float64),
                                            torch.tensor(gfeat, dtype=torch.float64)))
    assert_grads_close(("means2D", "conics", "colors", "opacities", "features"), got,
                       [t.grad.numpy() for t in leaves])


def test_chunked_dense_backward_equals_the_oracle_backward():
    # dense_blend_grad (the dense float64 formulation bench.py times at config 0) splits the frame
    # into pixel chunks, here 97 pixels, which cut image rows: its gradients must still be the
    # oracle's, and its image the dense forward's.
    width, height, n = 40, 32, 600
    m2, d, r, c, col, op = project_scene(4, n, width, height)
    rng = np.random.default_rng(4)
    gimg = rng.uniform(0, 1, (height, width, 3)).astype(np.float32)
    _, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, width, height)
    bg = np.zeros(3, np.float32)
    _, T, nc, _ = oracle.render_forward(width, height, ranges, values, m2, c, op, col, bg)
    got = oracle.render_backward(width, height, ranges, values, m2, c, op, col, bg, T, nc, gimg)
    t = lambda a: torch.tensor(a)  # noqa: E731
    image, grads, t_fwd, t_bwd = ref.dense_blend_grad(t(m2), t(d), t(r), t(c), t(col), t(op), width, height, t(gimg),
                                                      chunk=97)
    assert t_fwd > 0 and t_bwd > 0
    np.testing.assert_allclose(image.numpy(), ref.dense_blend(t(m2), t(d), t(r), t(c), t(col), t(op), width,
                                                              height).numpy(), rtol=0, atol=1e-12)
    names = ("means2D", "conics", "colors", "opacities")
    assert_grads_close(names, got[:4], [grads[k].numpy() for k in names])


# ---- projection ---------------------------------------------------------------------------------

def test_projection_closed_form_for_isotropic_gaussian_on_axis():
    # Identity camera, identity rotation, isotropic scale s, on the optical axis at depth z:
    # Sigma2D = diag((fx s / z)^2 + 0.3, (fy s / z)^2 + 0.3), mean = principal point.
    s, z, fx, fy = 0.05, 4.0, 300.0, 250.0
    m2, d, r, c = oracle.project_forward(np.array([[0, 0, z]], np.float32), np.full((1, 3), s, np.float32),
                                         np.array([[1, 0, 0, 0]], np.float32), np.array([[0.9]], np.float32),
                                         np.eye(4), fx, fy, 160.0, 120.0, 320, 240)
    sxx = (fx * s / (z + 1e-6)) ** 2 + 0.3
    syy = (fy * s / (z + 1e-6)) ** 2 + 0.3
    np.testing.assert_allclose(m2[0], [160.0, 120.0], rtol=1e-6)
    np.testing.assert_allclose(c[0], [1 / sxx, 0.0, 1 / syy], rtol=1e-5)
    np.testing.assert_allclose(r[0], 3 * math.sqrt(max(sxx, syy)), rtol=1e-5)
    assert d[0] == z


def test_projection_culls_behind_near_plane_and_off_screen():
    means = np.array([[0, 0, 0.1], [0, 0, -2.0], [50.0, 0, 2.0], [0, 0, 3.0]], np.float32)
    m2, d, r, c = oracle.project_forward(means, np.full((4, 3), 0.05, np.float32), np.tile([[1.0, 0, 0, 0]], (4, 1)),
                                         np.full((4, 1), 0.8, np.float32), np.eye(4), 100.0, 100.0, 50.0, 50.0, 100, 100)
    assert r.tolist()[:3] == [0.0, 0.0, 0.0] and r[3] > 0
    m2, d, r, c = oracle.project_forward(means[3:], np.full((1, 3), 0.05, np.float32), np.array([[1.0, 0, 0, 0]]),
                                         np.array([[0.5 / 255]], np.float32), np.eye(4), 100.0, 100.0, 50.0, 50.0, 100,
                                         100)
    assert r[0] == 0.0, "opacity below 1/255 is culled"


def test_projection_matches_matrix_formulation_and_its_autograd():
    g = gaussians(6, 500)
    angle = 0.4
    w2c = torch.eye(4, dtype=torch.float64)
    w2c[0, 0], w2c[0, 2], w2c[2, 0], w2c[2, 2] = math.cos(angle), math.sin(angle), -math.sin(angle), math.cos(angle)
    w2c[:3, 3] = torch.tensor([0.3, -0.2, 0.4])
    cam = camera(120, 90)
    args = (cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
    m2, d, r, c = oracle.project_forward(np_(g["means"]), np_(g["scales"]), np_(g["quats"]), np_(g["opacities"]),
                                         np_(w2c), *args)
    leaves = [g[k].double().requires_grad_(True) for k in ("means", "scales", "quats")]
    tm2, td, tc, _ = ref.project_torch(*leaves, w2c, *args)
    np.testing.assert_allclose(m2, tm2.detach().numpy(), rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(d, td.detach().numpy(), rtol=1e-6)
    vis = r > 0
    np.testing.assert_allclose(c[vis], tc.detach().numpy()[vis], rtol=2e-3, atol=1e-6)
    rng = np.random.default_rng(6)
    gm = rng.normal(size=(500, 2)).astype(np.float32)
    gc = rng.normal(size=(500, 3)).astype(np.float32) * 10
    got = oracle.project_backward(gm, gc, np_(g["means"]), np_(g["scales"]), np_(g["quats"]), np_(w2c), *args)
    torch.autograd.backward((tm2, tc), (torch.tensor(gm, dtype=torch.float64), torch.tensor(gc, dtype=torch.float64)))
    assert_grads_close(("means", "scales", "quats"), got, [t.grad.numpy() for t in leaves])


def test_projection_backward_on_the_clamp_and_near_plane_branches_matches_autograd():
    """Gaussians far outside the field of view (the Jacobian's x / z, y / z clamped) and behind the
    near plane (z clamped to 0.2): the gradient flows only where the forward's clamps let it, as
    torch autograd of the float64 matrix formulation says."""
    g = gaussians(9, 600)
    rng = np.random.default_rng(9)
    means = g["means"].clone()
    means[:200, 0] *= 6.0                                   # x / z far beyond 1.3 x the half field
    means[200:400, 1] *= 6.0
    means[400:500, 2] = torch.from_numpy(rng.uniform(-0.5, 0.2, 100).astype(np.float32))  # behind the near plane
    cam = camera(120, 90)
    args = (cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
    w2c = torch.eye(4, dtype=torch.float64)
    leaves = [means.double().requires_grad_(True), g["scales"].double().requires_grad_(True),
              g["quats"].double().requires_grad_(True)]
    tm2, _, tc, _ = ref.project_torch(*leaves, w2c, *args)
    gm = rng.normal(size=(600, 2)).astype(np.float32)
    gc = rng.normal(size=(600, 3)).astype(np.float32) * 10
    torch.autograd.backward((tm2, tc), (torch.tensor(gm, dtype=torch.float64), torch.tensor(gc, dtype=torch.float64)))
    got = oracle.project_backward(gm, gc, np_(means), np_(g["scales"]), np_(g["quats"]), np_(w2c), *args)
    want = [t.grad.numpy() for t in leaves]
    assert np.all(want[0][400:500, 2] == 0.0), "no depth gradient behind the near plane"
    assert np.all(got[0][400:500, 2] == 0.0)
    assert_grads_close(("means", "scales", "quats"), got, want)


def test_rigid_motion_of_scene_and_camera_changes_nothing():
    g = gaussians(7, 800)
    rot = ref.quat_to_rotmat(F.normalize(torch.tensor([[0.9, 0.2, -0.3, 0.1]]), dim=-1))[0]
    trans = torch.tensor([0.5, -0.4, 1.2])
    moved_means = g["means"] @ rot.T + trans
    # q_moved = r (x) q, so quat_to_rotmat(q_moved) = rot @ quat_to_rotmat(q).
    rq = F.normalize(torch.tensor([0.9, 0.2, -0.3, 0.1]), dim=0)
    w, x, y, z = rq
    a1, b1, c1, d1 = g["quats"].unbind(-1)
    moved_quats = torch.stack([w * a1 - x * b1 - y * c1 - z * d1, w * b1 + x * a1 + y * d1 - z * c1,
                               w * c1 - x * d1 + y * a1 + z * b1, w * d1 + x * c1 - y * b1 + z * a1], -1)
    w2c = torch.eye(4)
    w2c[:3, :3] = rot.T
    w2c[:3, 3] = -rot.T @ trans
    cam = camera(100, 80)
    args = (cam["fx"], cam["fy"], cam["cx"], cam["cy"], 100, 80)
    base = oracle.project_forward(np_(g["means"]), np_(g["scales"]), np_(g["quats"]), np_(g["opacities"]), np.eye(4),
                                  *args)
    moved = oracle.project_forward(np_(moved_means), np_(g["scales"]), np_(moved_quats), np_(g["opacities"]),
                                   np_(w2c), *args)
    np.testing.assert_allclose(moved[0], base[0], rtol=1e-4, atol=2e-3)
    np.testing.assert_allclose(moved[1], base[1], rtol=1e-4, atol=1e-5)
    vis = (base[2] > 0) & (moved[2] > 0)
    np.testing.assert_allclose(moved[3][vis], base[3][vis], rtol=2e-3, atol=1e-5)


# ---- spherical harmonics ------------------------------------------------------------------------

def test_sh_constants_match_legendre_definition_and_are_orthonormal():
    rng = np.random.default_rng(8)
    dirs = rng.normal(size=(4000, 3))
    dirs /= np.linalg.norm(dirs, axis=1, keepdims=True)
    basis = ref.sh_numeric(dirs, 3)
    # The oracle's rgb with one-hot weights recovers each basis function.
    for j in range(16):
        sh = np.zeros((len(dirs), 16, 3), np.float32)
        sh[:, j, 0] = 1.0
        got = oracle.eval_sh(sh[:, :1], sh[:, 1:], dirs.astype(np.float32), 3, np.ones(len(dirs), np.float32))
        # rgb = max(0.5 + b_j, 0): compare where no clamp happens.
        ok = got[:, 0] > 0
        np.testing.assert_allclose(got[ok, 0] - 0.5, basis[ok, j], atol=2e-6, err_msg=f"basis {j}")
    # Orthonormality on a Fibonacci sphere.
    m = 20000
    i = np.arange(m) + 0.5
    phi = np.arccos(1 - 2 * i / m)
    theta = np.pi * (1 + 5 ** 0.5) * i
    pts = np.stack([np.cos(theta) * np.sin(phi), np.sin(theta) * np.sin(phi), np.cos(phi)], 1)
    B = ref.sh_numeric(pts, 3)
    gram = 4 * np.pi * B.T @ B / m
    np.testing.assert_allclose(gram, np.eye(16), atol=2e-3)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_eval_sh_matches_closed_form(degree):
    g = torch.Generator().manual_seed(degree)
    n = 3000
    sh = torch.randn(n, 16, 3, generator=g) * 0.5
    dirs = F.normalize(torch.randn(n, 3, generator=g), dim=-1)
    radii = (torch.rand(n, generator=g) > 0.1).float()
    got = oracle.eval_sh(np_(sh[:, :1]), np_(sh[:, 1:]), np_(dirs), degree, np_(radii))
    want = ref.sh_closed_form(sh.double(), dirs.double(), degree, radii).numpy()
    assert (want == 0).any()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_rgb_to_sh_inverts_degree_zero():
    rng = np.random.default_rng(9)
    rgb = rng.uniform(0, 1, (1000, 3)).astype(np.float32)
    dirs = rng.normal(size=(1000, 3)).astype(np.float32)
    sh_dc = ((rgb - 0.5) / 0.28209479177387814).reshape(1000, 1, 3).astype(np.float32)
    got = oracle.eval_sh(sh_dc, np.zeros((1000, 15, 3), np.float32), dirs, 0, np.ones(1000, np.float32))
    np.testing.assert_allclose(got, rgb, atol=1e-6)


@pytest.mark.parametrize("degree", [1, 3])
def test_sh_backward_adam_matches_autograd_and_torch_adam(degree):
    g = torch.Generator().manual_seed(20 + degree)
    n = 2000
    sh = torch.randn(n, 16, 3, generator=g) * 0.5
    dirs = F.normalize(torch.randn(n, 3, generator=g), dim=-1)
    radii = (torch.rand(n, generator=g) > 0.1).float()
    dc, rest = np_(sh[:, :1]).copy(), np_(sh[:, 1:]).copy()
    m_dc, v_dc, m_rest, v_rest = (np.zeros_like(dc), np.zeros_like(dc), np.zeros_like(rest), np.zeros_like(rest))
    ref_dc = torch.nn.Parameter(sh[:, :1].clone())
    ref_rest = torch.nn.Parameter(sh[:, 1:].clone())
    adam = torch.optim.Adam([{"params": [ref_dc], "lr": 0.0025}, {"params": [ref_rest], "lr": 0.0025 / 20}],
                            eps=1e-15)
    for step in range(1, 4):
        grad_rgb = torch.randn(n, 3, generator=g)
        gd = oracle.eval_sh_backward_adam(np_(grad_rgb), dc, rest, np_(dirs), degree, np_(radii), m_dc, v_dc, m_rest,
                                          v_rest, step, step, 0.0025, 0.0025 / 20, 0.9, 0.999, 1e-15)
        d = dirs.clone().requires_grad_(True)
        ref.sh_closed_form(torch.cat([ref_dc, ref_rest], 1), d, degree, radii).backward(grad_rgb)
        adam.step()
        adam.zero_grad(set_to_none=True)
        np.testing.assert_allclose(gd, d.grad.numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dc, ref_dc.detach().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rest, ref_rest.detach().numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(m_rest, adam.state[ref_rest]["exp_avg"].numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(v_rest, adam.state[ref_rest]["exp_avg_sq"].numpy(), rtol=1e-5, atol=1e-9)


# ---- SSIM ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("height,width", [(64, 64), (37, 53), (11, 11), (5, 9)])
def test_ssim_matches_conv2d_float64(height, width):
    g = torch.Generator().manual_seed(height * width)
    gt = torch.rand(height, width, 3, generator=g)
    rendered = (gt + 0.1 * torch.randn(height, width, 3, generator=g)).clamp(0, 1)
    smap, d_mu, d_aa, d_ab = oracle.ssim_forward(np_(rendered), np_(gt))
    a = rendered.double().requires_grad_(True)
    want = ref.ssim_torch(a, gt.double())
    want.backward()
    np.testing.assert_allclose(smap.astype(np.float64).mean(), want.item(), rtol=1e-5, atol=1e-6)
    grad = oracle.ssim_backward(1.0, np_(rendered), np_(gt), d_mu, d_aa, d_ab)
    np.testing.assert_allclose(grad, a.grad.numpy(), rtol=1e-3, atol=1e-8)


def test_ssim_of_image_with_itself_is_one():
    img = np.random.default_rng(0).uniform(0, 1, (32, 40, 3)).astype(np.float32)
    smap = oracle.ssim_forward(img, img)[0]
    np.testing.assert_allclose(smap.mean(), 1.0, rtol=1e-6)


def test_config0_golden_vectors_are_reproduced():
    """Regression fixture: oracle outputs on a reduced config-0 scene (tests/golden/make_golden.py)."""
    data = np.load(GOLDEN / "oracle_config0_small.npz")
    cam = synthetic_config(0, n=16).cam
    m2, d, r, c = oracle.project_forward(data["means"], data["scales"], data["quats"], data["opacities"], np.eye(4),
                                         cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
    for name, got in (("means2D", m2), ("depths", d), ("radii", r), ("conics", c)):
        np.testing.assert_array_equal(got, data[name], err_msg=name)
    counts, values, ranges = oracle.bin_gaussians(m2, d, r, c, data["opacities"], cam["width"], cam["height"])
    np.testing.assert_array_equal(values, data["values_sorted"])
    np.testing.assert_array_equal(ranges, data["tile_ranges"])
    image, fimg, T, nc, _, _ = oracle.rasterize(m2, d, r, c, data["colors"], data["opacities"], cam["width"],
                                               cam["height"], np.zeros(3, np.float32), data["features"])
    np.testing.assert_allclose(image, data["image"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(fimg, data["feature_image"], rtol=1e-5, atol=1e-6)


def _config1_frame(channels):
    """Config 1 (200k gaussians, 979x546) projected, binned and blended by the oracle, with U[0, 1]
    colours and upstream gradients (seeds as bench.py)."""
    from tests.scenes import upstream

    wl = synthetic_config(1, channels=channels)
    cam = wl.cam
    quats = np_(wl.quats / wl.quats.norm(dim=-1, keepdim=True))
    m2, d, r, c = oracle.project_forward(np_(wl.means), np_(wl.scales), quats, np_(wl.opacities),
                                         np.eye(4, dtype=np.float32), cam["fx"], cam["fy"], cam["cx"], cam["cy"],
                                         cam["width"], cam["height"])
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).numpy()
    gi, gf = upstream(2, cam["height"], cam["width"], channels)
    return wl, cam, quats, (m2, d, r, c), colors, np_(gi), np_(gf)


def test_tile_mask_binning_blend_and_backward_equal_the_full_frame_on_the_selected_tiles():
    """oracle.bin_gaussians(tile_mask=) (used for the stress scene's GPU parity on selected tiles)
    against the unmasked oracle at config 1: the selected tiles' lists are the full binning's, the
    others are empty; the blend of the selected tiles' pixels is bit for bit the full frame's; and
    with the upstream gradients zeroed outside the selected tiles every gradient equals the full
    binning's bit for bit (the other tiles then add exact zeros)."""
    wl, cam, quats, (m2, d, r, c), colors, gi, gf = _config1_frame(8)
    W, H = cam["width"], cam["height"]
    op, feats = np_(wl.opacities).reshape(-1), np_(wl.features)
    tx, ty = (W + 15) // 16, (H + 15) // 16
    counts, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, W, H)
    rng = np.random.default_rng(7)
    mask = rng.random(tx * ty) < 0.2
    mask[np.argsort(ranges[:, 1] - ranges[:, 0])[-4:]] = True  # the longest lists too
    mcounts, mvalues, mranges = oracle.bin_gaussians(m2, d, r, c, op, W, H, tile_mask=mask)
    np.testing.assert_array_equal(mcounts, counts)
    assert mvalues.size == int((ranges[mask, 1] - ranges[mask, 0]).sum())
    for t in range(tx * ty):
        got = mvalues[mranges[t, 0]:mranges[t, 1]]
        want = values[ranges[t, 0]:ranges[t, 1]] if mask[t] else values[:0]
        np.testing.assert_array_equal(got, want)
    bg = np.zeros(3, np.float32)
    full = oracle.render_forward(W, H, ranges, values, m2, c, op, colors, bg, feats)
    part = oracle.render_forward(W, H, mranges, mvalues, m2, c, op, colors, bg, feats)
    pix = np.repeat(np.repeat(mask.reshape(ty, tx), 16, 0), 16, 1)[:H, :W]
    for got, want in zip(part, full):
        np.testing.assert_array_equal(got[pix], want[pix])
    assert (part[1][~pix] == 1.0).all() and (part[2][~pix] == 0).all()
    gi_m, gf_m = gi * pix[..., None], gf * pix[..., None]
    want = oracle.render_backward(W, H, ranges, values, m2, c, op, colors, bg, full[1], full[2], gi_m, feats, gf_m)
    got = oracle.render_backward(W, H, mranges, mvalues, m2, c, op, colors, bg, part[1], part[2], gi_m, feats, gf_m)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert np.abs(want[0]).max() > 0


def test_end_to_end_quats_gradient_amplifies_rasterizer_differences_far_below_the_bar():
    """Why bench.py gates the projection backward on identical inputs instead of end to end: the
    quaternion gradient (projection backward, then the normalize of the quats leaf) of the
    elongated gaussians of a scene amplifies differences in the rasterizer's means2D / conic
    gradients by orders of magnitude. At config 1, changing those gradients by 1e-6 of their max
    (500x below the 2e-3 bar that both stages pass) moves the quats gradient by more than that bar,
    and changing each value by about one float32 ulp (1e-7 relative) moves it by more than 1e-5 of
    its max, while the means gradient stays within 1e-4."""
    from tests.tolerances import grad_error

    wl, cam, quats, (m2, d, r, c), colors, gi, _ = _config1_frame(1)
    W, H = cam["width"], cam["height"]
    op = np_(wl.opacities).reshape(-1)
    _, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, W, H)
    bg = np.zeros(3, np.float32)
    _, T, nc, _ = oracle.render_forward(W, H, ranges, values, m2, c, op, colors, bg)
    dm, dc, _, _, _ = oracle.render_backward(W, H, ranges, values, m2, c, op, colors, bg, T, nc, gi)

    def leaves(gm, gc):
        pm, _, pq = oracle.project_backward(gm, gc, np_(wl.means), np_(wl.scales), quats, np.eye(4, dtype=np.float32),
                                            cam["fx"], cam["fy"], cam["cx"], cam["cy"], W, H)
        q = wl.quats.detach().clone().requires_grad_(True)
        F.normalize(q, dim=-1).backward(torch.from_numpy(pq))
        return pm, q.grad.numpy()

    ref_m, ref_q = leaves(dm, dc)
    rng = np.random.default_rng(0)
    eps = 1e-6
    gm = (dm + eps * np.abs(dm).max() * rng.uniform(-1, 1, dm.shape)).astype(np.float32)
    gc = (dc + eps * np.abs(dc).max() * rng.uniform(-1, 1, dc.shape)).astype(np.float32)
    assert grad_error(gm, dm)[1] <= 1.01 * eps and grad_error(gc, dc)[1] <= 1.01 * eps
    got_m, got_q = leaves(gm, gc)
    assert grad_error(got_m, ref_m)[1] < 1e-3
    assert grad_error(got_q, ref_q)[1] > 2e-3
    gm = (dm * (1 + 1e-7 * rng.uniform(-1, 1, dm.shape))).astype(np.float32)
    gc = (dc * (1 + 1e-7 * rng.uniform(-1, 1, dc.shape))).astype(np.float32)
    got_m, got_q = leaves(gm, gc)
    assert grad_error(got_m, ref_m)[1] < 1e-4
    assert grad_error(got_q, ref_q)[1] > 1e-5
