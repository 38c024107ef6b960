"""HIP path vs the CPU oracle on identical seeded inputs, through the C ABI.

Bars: integer work (visibility, tile counts, sorted pairs, tile ranges) bit-exact; projection
outputs bit-exact (both sides round every operation identically); images within the reference's
tolerances (test_render.py:29-58: RGB max 2e-3 / p99 1e-4, features max 1e-3 / p99 5e-4); gradients
within assert_grads_close (rtol 1e-3, atol 1e-4 * max|want|, < 0.1% outside, max error 2e-3 * max).
"""
import math
import sys

import numpy as np
import pytest
import torch

import oracle
from gaussian_splatting.rasterizer import _get_rasterizer, rasterize
from gaussian_splatting.rasterizer.projection import JACOBIAN_FOV_SCALE, LOW_PASS, NEAR_PLANE
from tests.scenes import camera, flat_scene, gaussians, synthetic_config
from tests.tolerances import assert_grads_close, assert_image_close

pytestmark = pytest.mark.gpu

DEV = "cuda"


def np_(t):
    return t.detach().cpu().numpy()


def project_both(wl_means, wl_scales, wl_quats, wl_opac, cam, w2c=None):
    """Projects on the GPU and in the oracle; returns (gpu tuple, oracle tuple)."""
    w2c = torch.eye(4) if w2c is None else w2c
    ext = _get_rasterizer()
    gpu = ext.project_gaussians(wl_means.to(DEV), wl_scales.to(DEV), wl_quats.to(DEV), wl_opac.to(DEV),
                                w2c.to(DEV), cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"],
                                cam["height"], NEAR_PLANE, LOW_PASS, JACOBIAN_FOV_SCALE)
    cpu = oracle.project_forward(np_(wl_means), np_(wl_scales), np_(wl_quats), np_(wl_opac), np_(w2c), cam["fx"],
                                 cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
    return gpu, cpu


def scene(seed, n, width, height):
    """Reference-style test scene projected by the HIP kernel: (means2D, depths, radii, conics, colors, opac)."""
    g = gaussians(seed, n)
    cam = camera(width, height)
    (m2, d, r, c), _ = project_both(g["means"], g["scales"], g["quats"], g["opacities"], cam)
    return m2, d, r, c, g["colors"].to(DEV), g["opacities"].to(DEV)


# ---- projection -------------------------------------------------------------------------------

@pytest.mark.parametrize("index", [0, 1])
def test_projection_is_bitwise_equal_to_oracle(index):
    wl = synthetic_config(index, n=50_000)
    gpu, cpu = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    for name, g, c in zip(("means2D", "depths", "radii", "conics"), gpu, cpu):
        np.testing.assert_array_equal(np_(g), c, err_msg=name)
    assert (cpu[2] > 0).mean() > 0.5, "the scene should be mostly visible"


def test_projection_with_rotated_camera_is_bitwise_equal():
    g = gaussians(5, 4000)
    angle = 0.3
    w2c = torch.eye(4)
    w2c[0, 0], w2c[0, 2], w2c[2, 0], w2c[2, 2] = math.cos(angle), math.sin(angle), -math.sin(angle), math.cos(angle)
    w2c[:3, 3] = torch.tensor([0.2, -0.1, 0.5])
    gpu, cpu = project_both(g["means"], g["scales"], g["quats"], g["opacities"], camera(160, 120), w2c)
    for name, a, b in zip(("means2D", "depths", "radii", "conics"), gpu, cpu):
        np.testing.assert_array_equal(np_(a), b, err_msg=name)


def test_projection_backward_matches_oracle():
    wl = synthetic_config(0, n=20_000)
    cam = wl.cam
    gen = torch.Generator().manual_seed(2)
    gm = torch.randn(wl.n, 2, generator=gen)
    gc = torch.randn(wl.n, 3, generator=gen)
    ext = _get_rasterizer()
    got = ext.project_gaussians_backward(gm.to(DEV), gc.to(DEV), wl.means.to(DEV), wl.scales.to(DEV),
                                         wl.quats.to(DEV), torch.eye(4, device=DEV), cam["fx"], cam["fy"], cam["cx"],
                                         cam["cy"], cam["width"], cam["height"], NEAR_PLANE, LOW_PASS,
                                         JACOBIAN_FOV_SCALE)
    want = oracle.project_backward(np_(gm), np_(gc), np_(wl.means), np_(wl.scales), np_(wl.quats), np.eye(4),
                                   cam["fx"], cam["fy"], cam["cx"], cam["cy"], cam["width"], cam["height"])
    assert_grads_close(("means", "scales", "quats"), [np_(t) for t in got], want)


# ---- binning ----------------------------------------------------------------------------------

@pytest.mark.parametrize("order", ["depth", "tile"])
@pytest.mark.parametrize("index,n", [(0, 10_000), (1, 200_000), (2, None)])
def test_binning_is_bitwise_equal_to_oracle(index, n, order):
    """Both binnings at full size: the global depth sort (bin, the reference's two-phase sequence) and
    tile order (bin_async with the depth order built per tile, the autograd path). (2, None) is the
    headline scene: 1.18M gaussians, 1.92M pairs, 470 sort partitions, tile lists of up to 1,736 pairs."""
    from gaussian_splatting.rasterizer._native import HipRasterizer

    wl = synthetic_config(index, n=n, channels=1)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).to(DEV)
    opac = wl.opacities.to(DEV)
    print(f"[test] binning config {index}, {order} order", file=sys.stderr, flush=True)
    if order == "depth":
        values, ranges, conic4, color4 = _get_rasterizer().bin(m2, d, r, c, colors, opac, wl.width, wl.height)
    else:
        ext = HipRasterizer()
        ext._pair_capacity[m2.device.index] = 1 << 22
        ext.tile_order = True
        bins = ext.bin_async(m2, d, r, c, colors, opac, wl.width, wl.height)
        assert not ext.resolve(bins) and bins.tile_order
        values, ranges, conic4, color4 = bins.values, bins.tile_ranges, bins.conic4, bins.color_opacity4
    counts, want_values, want_ranges = oracle.bin_gaussians(np_(m2), np_(d), np_(r), np_(c), np_(wl.opacities),
                                                            wl.width, wl.height)
    assert values.numel() == counts.sum() == want_values.size
    np.testing.assert_array_equal(np_(values), want_values)
    np.testing.assert_array_equal(np_(ranges), want_ranges)
    np.testing.assert_array_equal(np_(conic4[:, :3]), np_(c))
    np.testing.assert_array_equal(np_(color4), np.concatenate([np_(colors), np_(wl.opacities)], 1))


def test_binning_of_the_stress_scene_restricted_to_a_subset_equals_the_oracle():
    """Config 4 at full size (4M gaussians, 1920x1080, ~94M pairs; too many for the oracle's sort):
    - every gaussian appears exactly as often as the oracle's tile count says;
    - tile_ranges cut [0, P) into consecutive runs in tile order, empty tiles (0, 0);
    - inside a tile, depth bits increase and equal depths keep index order;
    - the (tile, gaussian) sequence restricted to 20k random gaussians equals the oracle's binning of
      those gaussians alone: the sort order is a total order on (tile, depth bits, index), so
      restricting the sorted list and sorting the restricted scene give the same sequence."""
    wl = synthetic_config(4, channels=1)
    cam = wl.cam
    ext = _get_rasterizer()
    m2, d, r, c = ext.project_gaussians(wl.means.to(DEV), wl.scales.to(DEV), wl.quats.to(DEV),
                                        wl.opacities.to(DEV), torch.eye(4, device=DEV), cam["fx"], cam["fy"],
                                        cam["cx"], cam["cy"], wl.width, wl.height, NEAR_PLANE, LOW_PASS,
                                        JACOBIAN_FOV_SCALE)
    opac = wl.opacities.to(DEV)
    values, ranges, _, _ = ext.bin(m2, d, r, c, None, opac, wl.width, wl.height)
    n, p, t = wl.n, values.numel(), ranges.shape[0]
    assert p > 50_000_000, p
    counts, _ = oracle.tile_counts(np_(m2), np_(r), np_(c), np_(opac), wl.width, wl.height)
    vals = values.long()
    np.testing.assert_array_equal(np_(torch.bincount(vals, minlength=n)), counts)

    lens = (ranges[:, 1] - ranges[:, 0]).long()
    full = lens > 0
    assert (ranges[~full] == 0).all()
    starts, ends = ranges[full, 0].long(), ranges[full, 1].long()
    assert int(starts[0]) == 0 and int(ends[-1]) == p and torch.equal(starts[1:], ends[:-1])
    tile_of = torch.repeat_interleave(torch.arange(t, device=DEV)[full], lens[full])
    depth_bits = d.view(torch.int32).long()[vals] & 0xFFFFFFFF
    key = tile_of * (1 << 32) + depth_bits
    step = key[1:] - key[:-1]
    assert bool((step >= 0).all())
    tie = step == 0
    assert bool((vals[1:][tie] > vals[:-1][tie]).all())
    del key, step, tie, depth_bits

    subset = np.sort(np.random.default_rng(7).choice(n, 20_000, replace=False))
    mask = torch.zeros(n, dtype=torch.bool, device=DEV)
    mask[torch.from_numpy(subset).to(DEV)] = True
    keep = mask[vals]
    got_tiles, got_ids = np_(tile_of[keep]), np_(vals[keep])
    sub = torch.from_numpy(subset).to(DEV)
    _, want_local, want_ranges = oracle.bin_gaussians(np_(m2[sub]), np_(d[sub]), np_(r[sub]), np_(c[sub]),
                                                      np_(opac[sub]), wl.width, wl.height)
    want_tiles = np.repeat(np.arange(t), want_ranges[:, 1] - want_ranges[:, 0])
    np.testing.assert_array_equal(got_ids, subset[want_local])
    np.testing.assert_array_equal(got_tiles, want_tiles)


def test_binning_of_more_than_16M_gaussians_is_complete_and_ordered():
    """17M small gaussians on a 256x192 image, depths on a 0.01 grid (many ties): the depth sort and
    the pair sort run on 8192-item partitions above 16M items. Every gaussian appears exactly as often
    as the oracle's tile count says, tile_ranges cut [0, P) in tile order, and inside each tile the
    depth bits increase with equal depths in index order, which together fix the sequence."""
    n, width, height = 17_000_000, 256, 192
    g = torch.Generator().manual_seed(21)
    means2D = torch.rand(n, 2, generator=g) * torch.tensor([float(width), float(height)])
    depths = torch.round(1.0 + torch.rand(n, generator=g) * 999.0) / 100.0
    sigma = 0.5 + torch.rand(n, generator=g) * 1.5
    conics = torch.stack([sigma ** -2, torch.zeros(n), sigma ** -2], -1)
    radii = 3.0 * sigma
    opac = (0.1 + 0.9 * torch.rand(n, generator=g))[:, None]
    m2, d, r, c, op = (t.contiguous().to(DEV) for t in (means2D, depths, radii, conics, opac))
    values, ranges, _, _ = _get_rasterizer().bin(m2, d, r, c, None, op, width, height)
    p, t = values.numel(), ranges.shape[0]
    assert p > (1 << 24), p
    counts, _ = oracle.tile_counts(np_(m2), np_(r), np_(c), np_(op), width, height)
    vals = values.long()
    np.testing.assert_array_equal(np_(torch.bincount(vals, minlength=n)), counts)
    lens = (ranges[:, 1] - ranges[:, 0]).long()
    full = lens > 0
    assert (ranges[~full] == 0).all()
    starts, ends = ranges[full, 0].long(), ranges[full, 1].long()
    assert int(starts[0]) == 0 and int(ends[-1]) == p and torch.equal(starts[1:], ends[:-1])
    tile_of = torch.repeat_interleave(torch.arange(t, device=DEV)[full], lens[full])
    key = tile_of * (1 << 32) + (d.view(torch.int32).long()[vals] & 0xFFFFFFFF)
    step = key[1:] - key[:-1]
    assert bool((step >= 0).all())
    tie = step == 0
    assert int(tie.sum()) > 1_000_000, "the scene should have many depth ties"
    assert bool((vals[1:][tie] > vals[:-1][tie]).all())


def test_binning_keeps_index_order_on_depth_ties():
    # 300 gaussians in 5 depth values over a 3x2 tile image: ties must stay in index order.
    g = torch.Generator().manual_seed(4)
    n = 300
    means2D = torch.rand(n, 2, generator=g) * torch.tensor([40.0, 30.0])
    depths = torch.randint(0, 5, (n,), generator=g).float() + 1.0
    conics = torch.tensor([[0.05, 0.0, 0.05]]).repeat(n, 1)
    opac = torch.full((n, 1), 0.5)
    radii = torch.ones(n)
    values, ranges, _, _ = _get_rasterizer().bin(means2D.to(DEV), depths.to(DEV), radii.to(DEV), conics.to(DEV),
                                                 None, opac.to(DEV), 40, 30)
    _, want_values, want_ranges = oracle.bin_gaussians(np_(means2D), np_(depths), np_(radii), np_(conics),
                                                       np_(opac), 40, 30)
    np.testing.assert_array_equal(np_(values), want_values)
    np.testing.assert_array_equal(np_(ranges), want_ranges)


def test_empty_scene_renders_background():
    ext = _get_rasterizer()
    bg = torch.tensor([0.3, 0.5, 0.7], device=DEV)
    z = torch.zeros(0, device=DEV)
    out = ext.rasterize(torch.zeros(0, 2, device=DEV), z, z, torch.zeros(0, 3, device=DEV),
                        torch.zeros(0, 3, device=DEV), torch.zeros(0, 1, device=DEV), bg, 37, 21)
    image, final_T, n_contrib, values, ranges = out[:5]
    assert torch.equal(image, bg.expand(21, 37, 3))
    assert torch.equal(final_T, torch.ones(21, 37, device=DEV))
    assert int(n_contrib.abs().sum()) == 0 and values.numel() == 0 and int(ranges.abs().sum()) == 0


@pytest.mark.parametrize("order", ["depth", "tile"])
@pytest.mark.parametrize("capacity", ["exact", "short", "tiny", "roomy"])
def test_async_binning_equals_the_oracle_whatever_the_capacity(capacity, order):
    """bin_async + resolve (the autograd path: render enqueued before the host reads P) gives the
    oracle's binning bit for bit when the pair buffers are exactly P, a partition short of P (the
    capped sort runs, then resolve rebins exactly), far too small, or larger than P, with the
    global depth sort and in tile order (depth order per tile); the render of a capped binning
    stays inside its buffers."""
    from gaussian_splatting.rasterizer._native import HipRasterizer

    wl = synthetic_config(1, n=60_000, channels=1)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    opac = wl.opacities.to(DEV)
    counts, want_values, want_ranges = oracle.bin_gaussians(np_(m2), np_(d), np_(r), np_(c), np_(opac), wl.width,
                                                            wl.height)
    p = int(counts.sum())
    cap = {"exact": p, "short": p - 4096, "tiny": 1, "roomy": p + 10_000}[capacity]
    ext = HipRasterizer()
    ext._pair_capacity[m2.device.index] = cap
    ext.tile_order = order == "tile"
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).to(DEV)
    print(f"[test] async binning, capacity {capacity}, {order} order", file=sys.stderr, flush=True)
    bins = ext.bin_async(m2, d, r, c, colors, opac, wl.width, wl.height)
    assert bins.values.numel() == cap and bins.tile_order == (order == "tile")
    _, _, T, _ = ext.render(m2, bins.conic4, bins.color_opacity4, bins.values, bins.tile_ranges, wl.width,
                            wl.height, torch.zeros(3, device=DEV))
    torch.cuda.synchronize()
    rebinned = ext.resolve(bins)
    assert rebinned == (cap < p)
    np.testing.assert_array_equal(np_(bins.values), want_values)
    np.testing.assert_array_equal(np_(bins.tile_ranges), want_ranges)
    assert ext._pair_capacity[m2.device.index] >= p
    assert bool(torch.isfinite(T).all())


@pytest.mark.parametrize("path", ["scatter", "emit"])
@pytest.mark.parametrize("frame", ["mid", "wide", "giants"])
def test_tile_order_binning_paths_equal_the_oracle(path, frame):
    """Both tile-order paths bin like the oracle bit for bit: the counting scatter (per-chunk LDS tile
    histograms, one scan over the (tile, chunk) count matrix, pairs scattered into their runs, then
    the per-tile depth sort) and the emit + pair sort by tile that frames with a count matrix above
    the limit take (forced here with hds_set_tile_scatter_limit). "wide" is a 2048x1088 frame of 8704
    tiles, more than one LDS histogram holds (8192), so the counts and the scatter run in two
    windows of tiles. "giants" adds to that frame 12 gaussians of sigma 150-600 px, whose rectangles
    cover thousands of tiles in both windows (runs of thousands of pairs per wave), and culls every
    seventh gaussian (radius 0)."""
    from gaussian_splatting.rasterizer._native import HipRasterizer, load_library

    if frame == "mid":
        wl = synthetic_config(1, n=120_000, channels=1)
        (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
        opac, width, height = wl.opacities.to(DEV), wl.width, wl.height
    else:
        g = torch.Generator().manual_seed(31)
        n, width, height = 150_000, 2048, 1088
        m2 = torch.rand(n, 2, generator=g) * torch.tensor([float(width), float(height)])
        d = 1.0 + torch.rand(n, generator=g) * 9.0
        sigma = 0.5 + torch.rand(n, generator=g) * 6.0
        if frame == "giants":
            sigma[::12_500] = 150.0 + torch.rand(12, generator=g) * 450.0
        c = torch.stack([sigma ** -2, torch.zeros(n), sigma ** -2], -1)
        r = 3.0 * sigma
        if frame == "giants":
            r[3::7] = 0.0
        opac = (0.05 + 0.9 * torch.rand(n, generator=g))[:, None]
        m2, d, r, c, opac = (t.contiguous().to(DEV) for t in (m2, d, r, c, opac))
    counts, want_values, want_ranges = oracle.bin_gaussians(np_(m2), np_(d), np_(r), np_(c), np_(opac), width,
                                                            height)
    lib = load_library()
    ext = HipRasterizer()
    ext._pair_capacity[m2.device.index] = int(counts.sum()) + 4096
    ext.tile_order = True
    print(f"[test] tile-order binning by {path}, {frame} frame {width}x{height}", file=sys.stderr, flush=True)
    assert lib.hds_set_tile_scatter_limit(1 if path == "emit" else 0) == 0
    try:
        bins = ext.bin_async(m2, d, r, c, None, opac, width, height)
        assert not ext.resolve(bins)
    finally:
        assert lib.hds_set_tile_scatter_limit(0) == 0
    np.testing.assert_array_equal(np_(bins.values), want_values)
    np.testing.assert_array_equal(np_(bins.tile_ranges), want_ranges)


def _one_tile_scene(n, seed, levels=50):
    """n small gaussians whose footprints all lie inside tile 0 of a 64x64 image (one list of n
    pairs), with depths drawn from `levels` values so that ties occur (0: continuous depths)."""
    g = torch.Generator().manual_seed(seed)
    means2D = 5.0 + torch.rand(n, 2, generator=g) * 6.0
    if levels:
        depths = torch.randint(0, levels, (n,), generator=g).float() * (12.5 / levels) + 1.0
    else:
        depths = 1.0 + torch.rand(n, generator=g) * 12.5
    conics = torch.tensor([[0.5, 0.0, 0.5]]).repeat(n, 1)
    return means2D, depths, torch.ones(n), conics, torch.full((n, 1), 0.5)


@pytest.mark.parametrize("n,strided,levels", [(1500, False, 50), (1500, False, 1500), (2000, False, 0),
                                              (3000, False, 50), (5000, False, 50), (5000, True, 50)])
def test_tile_order_binning_sorts_long_lists_in_lds_and_hands_longer_ones_back(n, strided, levels):
    """Tiles of 1500-2000 pairs take the register networks: a first pass on 32-bit (coarse depth,
    list index) keys, then odd-even rounds on the full (depth bits, index) keys where coarse depths
    tie (depths from 1500 levels) or, with too many ties for a few rounds (50 levels), the 64-bit
    network; with continuous depths the first pass alone. A tile of 3000 pairs (beyond the register
    networks, sorted in LDS) bins bit for bit like the oracle in tile order; one of 5000 pairs (beyond
    the per-tile sort) is flagged, resolve bins the frame again with the global depth sort (same
    result) and the device leaves tile order. With `strided`, means2D is a non-contiguous [:, :2]
    view of an [N, 3] tensor: the rebin must read the dense copy the binning made, not the caller's
    view."""
    from gaussian_splatting.rasterizer._native import HipRasterizer

    means2D, depths, radii, conics, opac = _one_tile_scene(n, 9, levels)
    _, want_values, want_ranges = oracle.bin_gaussians(np_(means2D), np_(depths), np_(radii), np_(conics),
                                                       np_(opac), 64, 64)
    assert int(want_ranges[0, 1] - want_ranges[0, 0]) == n
    ext = HipRasterizer()
    dev = torch.device(DEV, torch.cuda.current_device())
    ext._pair_capacity[dev.index] = n + 8192
    ext._tile_order_ok[dev.index] = True
    means2D_dev = means2D.to(DEV)
    if strided:
        wide = torch.full((n, 3), 1e6, device=DEV)
        wide[:, :2] = means2D_dev
        means2D_dev = wide[:, :2]
        assert not means2D_dev.is_contiguous()
    print(f"[test] tile-order binning, one tile of {n} pairs, {levels} depth levels, strided means2D {strided}",
          file=sys.stderr, flush=True)
    bins = ext.bin_async(means2D_dev, depths.to(DEV), radii.to(DEV), conics.to(DEV), None, opac.to(DEV), 64, 64)
    assert bins.tile_order
    rebinned = ext.resolve(bins)
    assert rebinned == (n > ext.TILE_ORDER_MAX)
    assert ext._tile_order_ok[dev.index] == (n <= ext.TILE_ORDER_MAX)
    np.testing.assert_array_equal(np_(bins.values), want_values)
    np.testing.assert_array_equal(np_(bins.tile_ranges), want_ranges)


def test_first_binning_chooses_the_order_from_the_longest_tile_list():
    """bin_async's first (synchronous) call on a device picks tile order for later calls when the
    longest tile list leaves room in the per-tile sort, and the global depth sort when it does not."""
    from gaussian_splatting.rasterizer._native import HipRasterizer

    for n, want in ((1000, True), (4000, False)):
        means2D, depths, radii, conics, opac = _one_tile_scene(n, 10)
        ext = HipRasterizer()
        ext.bin_async(means2D.to(DEV), depths.to(DEV), radii.to(DEV), conics.to(DEV), None, opac.to(DEV), 64, 64)
        assert ext._tile_order_ok[torch.cuda.current_device()] == want


@pytest.mark.parametrize("tile_order", [False, True])
def test_async_binning_of_a_scene_with_no_pairs(tile_order):
    from gaussian_splatting.rasterizer._native import HipRasterizer

    ext = HipRasterizer()
    ext._pair_capacity[0] = 8192
    ext.tile_order = tile_order
    n = 500
    means2D = torch.rand(n, 2, device=DEV) * 40
    bins = ext.bin_async(means2D, torch.ones(n, device=DEV), torch.zeros(n, device=DEV),
                         torch.full((n, 3), 0.1, device=DEV), None, torch.full((n, 1), 0.5, device=DEV), 40, 30)
    assert not ext.resolve(bins)
    assert bins.values.numel() == 0 and int(bins.tile_ranges.abs().sum()) == 0


def test_gradient_buffers_are_zeroed_ahead_only_when_a_graph_is_recorded(monkeypatch):
    """The forward's render zeroes the backward's gradient buffers only when the caller records a graph
    (not under torch.no_grad(), where no backward can follow), and the backward then gives the same
    gradients as one that zeroes its own buffers."""
    wl = synthetic_config(0, n=6000)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).to(DEV)
    feats = wl.features.to(DEV).requires_grad_(True)
    opac = wl.opacities.to(DEV)
    ext = _get_rasterizer()
    calls = []
    original = ext.gradient_buffers
    monkeypatch.setattr(ext, "gradient_buffers", lambda *args: calls.append(args) or original(*args))
    with torch.no_grad():
        rasterize(m2, d, r, c, colors, opac, wl.width, wl.height, features=feats)
    assert not calls
    image, fimg = rasterize(m2, d, r, c, colors, opac, wl.width, wl.height, features=feats)
    assert len(calls) == 1
    g = torch.Generator().manual_seed(6)
    gi = torch.rand(image.shape, generator=g).to(DEV)
    gf = torch.rand(fimg.shape, generator=g).to(DEV)
    torch.autograd.backward((image, fimg), (gi, gf))
    ahead = feats.grad.clone()
    feats.grad = None
    values, ranges, conic4, color4 = ext.bin(m2, d, r, c, colors, opac, wl.width, wl.height)
    _, _, T, nc = ext.render(m2, conic4, color4, values, ranges, wl.width, wl.height, torch.zeros(3, device=DEV),
                             feats.detach())
    own = ext.render_backward(m2, conic4, color4, values, ranges, T, nc, wl.width, wl.height, grad_image=gi,
                              background=torch.zeros(3, device=DEV), features=feats.detach(), grad_feature_image=gf,
                              slice_width=32)[4]
    scale = own.abs().max().item()
    assert (ahead - own).abs().max().item() <= 1e-5 * scale


@pytest.mark.parametrize("workgroups", [0, 3])
def test_zero_fill_clears_exactly_its_range(workgroups):
    """hds_zero_async (the pre-zeroed gradients' fill) clears count floats from p, with as many
    work-groups as fill the device or only three (each then strides over the range), and nothing past
    it."""
    from gaussian_splatting.rasterizer._native import _ptr, _stream, load_library

    lib = load_library()
    buf = torch.full((1_000_064,), 7.0, device=DEV)
    print(f"[test] zero fill, {workgroups} work-groups", file=sys.stderr, flush=True)
    assert lib.hds_zero_async(_ptr(buf), 1_000_000, workgroups, _stream(buf.device)) == 0
    torch.cuda.synchronize()
    assert int((buf[:1_000_000] != 0).sum()) == 0
    assert bool((buf[1_000_000:] == 7.0).all())


@pytest.mark.parametrize("channels,count", [(0, 1_000_004), (256, 2_000_000), (64, 4)])
def test_render_clear_renders_the_same_and_clears_exactly_its_range(channels, count):
    """hds_render_clear gives hds_render's outputs bit for bit and zeroes exactly `count` floats: a range
    that does not divide evenly over the (tile, slice) work-groups, one spread over two 128-channel
    slices, and one smaller than the work-group count (most shares empty)."""
    wl = synthetic_config(0, n=6000)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).to(DEV)
    opac = wl.opacities.to(DEV)
    feats = (torch.randn(wl.n, channels, generator=torch.Generator().manual_seed(4)).to(DEV)
             if channels else None)
    ext = _get_rasterizer()
    values, ranges, conic4, color4 = ext.bin(m2, d, r, c, colors, opac, wl.width, wl.height)
    bg = torch.zeros(3, device=DEV)
    print(f"[test] render_clear, C {channels}, count {count}", file=sys.stderr, flush=True)
    want = ext.render(m2, conic4, color4, values, ranges, wl.width, wl.height, bg, feats)
    buf = torch.full((count + 64,), 7.0, device=DEV)
    got = ext.render(m2, conic4, color4, values, ranges, wl.width, wl.height, bg, feats, clear=buf[:count])
    torch.cuda.synchronize()
    assert int((buf[:count] != 0).sum()) == 0
    assert bool((buf[count:] == 7.0).all())
    for a, b in zip(got, want):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)


def test_rasterize_is_identical_with_and_without_the_pair_count_read():
    # The first call on a fresh binding bins synchronously, later ones bin ahead of the count.
    import gaussian_splatting.rasterizer as rasterizer_module
    from gaussian_splatting.rasterizer._native import HipRasterizer

    wl = synthetic_config(0, n=8000)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).to(DEV)
    feats, opac = wl.features.to(DEV), wl.opacities.to(DEV)
    saved = rasterizer_module._rasterizer_module
    rasterizer_module._rasterizer_module = HipRasterizer()
    try:
        outs = [rasterize(m2, d, r, c, colors, opac, wl.width, wl.height, features=feats) for _ in range(3)]
    finally:
        rasterizer_module._rasterizer_module = saved
    for image, fimg in outs[1:]:
        assert torch.equal(image, outs[0][0]) and torch.equal(fimg, outs[0][1])


# ---- blend forward ----------------------------------------------------------------------------

def oracle_render(inputs, width, height, background=None, features=None, near_cut=False):
    m2, d, r, c, col, op = [np_(t) for t in inputs]
    _, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, width, height)
    out = oracle.render_forward(width, height, ranges, values, m2, c, op, col,
                                None if background is None else np_(background),
                                None if features is None else np_(features), near_cut=near_cut)
    image, final_T, n_contrib, fimg = out[:4]
    if near_cut:
        return image, fimg, final_T, n_contrib, values, ranges, out[4]
    return image, fimg, final_T, n_contrib, values, ranges


def assert_forward_exact(got, want):
    """(image, final_T, n_contrib) equal to the oracle's bit for bit: both sides take every alpha from
    hds_gauss_alpha and blend RGB with the same fused multiply-adds in list order."""
    for name, g, w in zip(("image", "final_T", "n_contrib"), got, want):
        g = np_(g)
        assert g.shape == w.shape and np.array_equal(g, w), f"{name}: {int(np.sum(g != w))} values differ"


def test_rgb_forward_matches_oracle():
    width, height = 128, 96
    inputs = scene(0, 3000, width, height)
    bg = torch.tensor([0.3, 0.5, 0.7], device=DEV)
    image, final_T, n_contrib, values, ranges, _, _ = _get_rasterizer().rasterize(*inputs, bg, width, height)
    want_image, _, want_T, want_nc, want_values, want_ranges = oracle_render(inputs, width, height, bg)
    np.testing.assert_array_equal(np_(values), want_values)
    assert_forward_exact((image, final_T, n_contrib), (want_image, want_T, want_nc))


@pytest.mark.parametrize("channels", [32, 64, 128, 256, 512])
def test_features_forward_matches_oracle(channels):
    width, height = 128, 96
    inputs = scene(0, 3000, width, height)
    features = torch.rand(3000, channels, generator=torch.Generator().manual_seed(2)).to(DEV)
    image, feature_image = rasterize(*inputs, width, height, features=features)
    assert torch.equal(image, rasterize(*inputs, width, height)), "RGB must not depend on the features"
    _, want, _, _, _, _ = oracle_render(inputs, width, height, features=features)
    assert_image_close(np_(feature_image), want, max_error=1e-3, max_perc_99=5e-4)


def test_feature_forward_of_config0_matches_oracle():
    wl = synthetic_config(0)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(3)).to(DEV)
    inputs = (m2, d, r, c, colors, wl.opacities.to(DEV))
    image, feature_image = rasterize(*inputs, wl.width, wl.height, features=wl.features.to(DEV))
    want_image, want_f, _, _, _, _ = oracle_render(inputs, wl.width, wl.height, torch.zeros(3), wl.features)
    np.testing.assert_array_equal(np_(image), want_image)
    assert_image_close(np_(feature_image), want_f, max_error=1e-3, max_perc_99=5e-4)


# ---- backward ---------------------------------------------------------------------------------

def grads_gpu(inputs, width, height, features, grad_image, grad_feat, background):
    m2, d, r, c, col, op = inputs
    leaves = [t.detach().clone().requires_grad_(True) for t in (m2, c, col, op, features)]
    image, fimg = rasterize(leaves[0], d, r, leaves[1], leaves[2], leaves[3], width, height, background,
                            features=leaves[4])
    torch.autograd.backward((image, fimg), (grad_image, grad_feat))
    return [np_(t.grad) for t in leaves]


def grads_oracle(inputs, width, height, features, grad_image, grad_feat, background):
    m2, d, r, c, col, op = [np_(t) for t in inputs]
    _, values, ranges = oracle.bin_gaussians(m2, d, r, c, op, width, height)
    _, T, nc, _ = oracle.render_forward(width, height, ranges, values, m2, c, op, col, np_(background), np_(features))
    dm, dc, dcol, dop, df = oracle.render_backward(width, height, ranges, values, m2, c, op, col, np_(background), T,
                                                   nc, np_(grad_image), np_(features), np_(grad_feat))
    return [dm, dc, dcol, dop, df]


@pytest.mark.parametrize("channels", [64, 128])
def test_reference_feature_entry_points_match_oracle(channels):
    """The reference extension's rasterize / rasterize_features / rasterize_features_backward sequence
    (rasterizer/__init__.py:130-165 there), through hds_render_backward with its own zeroing: the
    feature-only gradients equal the oracle's with a zero image gradient."""
    width, height = 128, 96
    m2, d, r, c, col, op = scene(1, 3000, width, height)
    g = torch.Generator().manual_seed(4)
    features = torch.rand(3000, channels, generator=g).to(DEV)
    grad_feat = torch.rand(height, width, channels, generator=g).to(DEV)
    ext = _get_rasterizer()
    bg = torch.zeros(3, device=DEV)
    _, _, _, values, ranges, conic4, color4 = ext.rasterize(m2, d, r, c, col, op, bg, width, height)
    fimg, fT, fnc = ext.rasterize_features(features, m2, conic4, color4, values, ranges, width, height)
    got = ext.rasterize_features_backward(grad_feat, features, m2, conic4, color4, values, ranges, fT, fnc, width,
                                          height, min(channels, 128))
    want = grads_oracle((m2, d, r, c, col, op), width, height, features, torch.zeros(height, width, 3, device=DEV),
                        grad_feat, bg)
    _, want_f, _, _, _, _ = oracle_render((m2, d, r, c, col, op), width, height, features=features)
    assert_image_close(np_(fimg), want_f, max_error=1e-3, max_perc_99=5e-4)
    # got = (grad_features, dmeans2D, dconics, dopac); want = (dm, dc, dcol, dop, df)
    assert_grads_close(("features", "means2D", "conics", "opacities"), [np_(t) for t in got],
                       [want[4], want[0], want[1], want[3]])


@pytest.mark.parametrize("channels,slice_width", [(32, 32), (64, 64), (64, 32), (128, 128), (128, 64), (128, 32),
                                                  (256, 128), (256, 64), (512, 128), (512, 64)])
def test_backward_matches_oracle(channels, slice_width, monkeypatch):
    monkeypatch.setattr("gaussian_splatting.rasterizer.FEATURE_SLICE_WIDTH", slice_width)
    width, height = 128, 96
    inputs = scene(0, 3000, width, height)
    g = torch.Generator().manual_seed(3)
    features = torch.rand(3000, channels, generator=g).to(DEV)
    grad_image = torch.rand(height, width, 3, generator=g).to(DEV)
    grad_feat = torch.rand(height, width, channels, generator=g).to(DEV)
    bg = torch.tensor([0.3, 0.5, 0.7], device=DEV)
    got = grads_gpu(inputs, width, height, features, grad_image, grad_feat, bg)
    want = grads_oracle(inputs, width, height, features, grad_image, grad_feat, bg)
    assert_grads_close(("means2D", "conics", "colors", "opacities", "features"), got, want)


def test_rgb_only_backward_matches_oracle():
    width, height = 128, 96
    inputs = scene(1, 3000, width, height)
    g = torch.Generator().manual_seed(1)
    grad_image = torch.rand(height, width, 3, generator=g).to(DEV)
    bg = torch.tensor([0.3, 0.5, 0.7], device=DEV)
    m2, d, r, c, col, op = inputs
    leaves = [t.detach().clone().requires_grad_(True) for t in (m2, c, col, op)]
    rasterize(leaves[0], d, r, leaves[1], leaves[2], leaves[3], width, height, bg).backward(grad_image)
    mn, cn, coln, opn = [np_(t) for t in inputs][0], np_(c), np_(col), np_(op)
    _, values, ranges = oracle.bin_gaussians(mn, np_(d), np_(r), cn, opn, width, height)
    _, T, nc, _ = oracle.render_forward(width, height, ranges, values, mn, cn, opn, coln, np_(bg))
    want = oracle.render_backward(width, height, ranges, values, mn, cn, opn, coln, np_(bg), T, nc, np_(grad_image))
    assert_grads_close(("means2D", "conics", "colors", "opacities"), [np_(t.grad) for t in leaves], want[:4])


EDGE_CASES = {
    "depth_ties": ([[7.5, 8.5], [9.5, 8.5]], [2.0, 2.0], [3.0, 3.0], [0.7, 0.7], 16, 16),
    "min_alpha": ([[4.5, 4.5], [12.5, 4.5]], [1.0, 1.0], [0.5, 0.5], [1.01 / 255, 0.99 / 255], 16, 8),
    "max_alpha": ([[8.5, 8.5]], [1.0], [2.0], [1.0], 16, 16),
    "transmittance_floor": ([[8.5, 8.5]] * 50, [1.0 + i for i in range(50)], [4.0] * 50, [0.9] * 50, 16, 16),
}


@pytest.mark.parametrize("case", list(EDGE_CASES))
def test_edge_case_matches_oracle(case):
    means, depths, sigmas, opac, width, height = EDGE_CASES[case]
    inputs = flat_scene(means, depths, sigmas, opac, device=DEV)
    n = len(depths)
    g = torch.Generator().manual_seed(7)
    bg = torch.tensor([0.3, 0.5, 0.7], device=DEV)
    grad_image = torch.rand(height, width, 3, generator=g).to(DEV)
    features = torch.rand(n, 128, generator=g).to(DEV)
    grad_feat = torch.rand(height, width, 128, generator=g).to(DEV)
    image = rasterize(*inputs, width, height, bg)
    want_image = oracle_render(inputs, width, height, bg)[0]
    np.testing.assert_array_equal(np_(image), want_image)
    got = grads_gpu(inputs, width, height, features, grad_image, grad_feat, bg)
    want = grads_oracle(inputs, width, height, features, grad_image, grad_feat, bg)
    assert_grads_close(("means2D", "conics", "colors", "opacities", "features"), got, want)


def test_max_alpha_clamp_gives_099_colour():
    inputs = flat_scene([[8.5, 8.5]], [1.0], [2.0], [1.0], device=DEV)
    torch.testing.assert_close(rasterize(*inputs, 16, 16)[8, 8], 0.99 * inputs[4][0])


def test_min_alpha_threshold_blends_only_above():
    inputs = flat_scene([[4.5, 4.5], [12.5, 4.5]], [1.0, 1.0], [0.5, 0.5], [1.01 / 255, 0.99 / 255], device=DEV)
    image = rasterize(*inputs, 16, 8)
    assert image[4, 4].abs().sum() > 0
    assert torch.equal(image[4, 12], torch.zeros(3, device=DEV))


def test_dense_tile_walks_past_every_batch():
    g = torch.Generator().manual_seed(11)
    n = 2000
    means = (torch.rand(n, 2, generator=g) * 16).tolist()
    depths = (1 + torch.rand(n, generator=g)).tolist()
    inputs = flat_scene(means, depths, [12.0] * n, [0.02] * n, device=DEV)
    bg = torch.zeros(3, device=DEV)
    out = _get_rasterizer().rasterize(*inputs, bg, 16, 16)
    assert out[2].min() > 256, f"some pixel stopped at {out[2].min().item()}"
    want_image, _, want_T, want_nc, _, _ = oracle_render(inputs, 16, 16, bg)
    assert_forward_exact(out[:3], (want_image, want_T, want_nc))
    gg = torch.Generator().manual_seed(12)
    features = torch.rand(n, 64, generator=gg).to(DEV)
    grad_image = torch.rand(16, 16, 3, generator=gg).to(DEV)
    grad_feat = torch.rand(16, 16, 64, generator=gg).to(DEV)
    got = grads_gpu(inputs, 16, 16, features, grad_image, grad_feat, bg)
    want = grads_oracle(inputs, 16, 16, features, grad_image, grad_feat, bg)
    assert_grads_close(("means2D", "conics", "colors", "opacities", "features"), got, want)


def elongated_scene(seed, n, width, height):
    """Thin, long, rotated gaussians centred near the corners and edges of the 8x8 pixel blocks, with
    opacities down to just above 1/255: the cases where a cull of whole blocks could wrongly drop a
    gaussian that reaches a pixel (the oracle renders every pixel without any block cull)."""
    g = torch.Generator().manual_seed(seed)
    corners = torch.randint(0, width // 8 + 1, (n,), generator=g) * 8.0, torch.randint(0, height // 8 + 1, (n,), generator=g) * 8.0
    means2D = torch.stack(corners, -1) + (torch.rand(n, 2, generator=g) * 2 - 1) * 6.0
    theta = torch.rand(n, generator=g) * math.pi
    thin = 0.3 + torch.rand(n, generator=g) * 0.7            # covariance eigenvalues: 0.3-1 px^2 ...
    long = torch.exp(torch.rand(n, generator=g) * math.log(600.0))  # ... against 1-600 px^2
    cs, sn = torch.cos(theta), torch.sin(theta)
    sxx = long * cs * cs + thin * sn * sn
    syy = long * sn * sn + thin * cs * cs
    sxy = (long - thin) * cs * sn
    det = sxx * syy - sxy * sxy
    conics = torch.stack([syy / det, -sxy / det, sxx / det], -1)
    radii = 3.0 * torch.sqrt(torch.maximum(long, thin))
    depths = 1.0 + torch.rand(n, generator=g) * 9.0
    opac = torch.where(torch.rand(n, generator=g) < 0.3, 1.0 / 255 * (1.0 + torch.rand(n, generator=g) * 0.2),
                       torch.rand(n, generator=g))[:, None]
    colors = torch.rand(n, 3, generator=g)
    return tuple(t.float().contiguous().to(DEV) for t in (means2D, depths, radii, conics, colors, opac))


@pytest.mark.parametrize("seed", [0, 1])
def test_block_cull_keeps_every_contributor(seed):
    """The blend kernels visit a gaussian in an 8x8 block only if the minimum of its quadratic form over
    the block's pixel-centre rectangle is under the 1/255 threshold; on adversarial ellipses the result
    must still equal the oracle's (RGB image, final T and n_contrib bit for bit, features and gradients
    within the usual bars)."""
    width, height = 96, 80
    n = 3000
    inputs = elongated_scene(seed, n, width, height)
    bg = torch.tensor([0.3, 0.5, 0.7], device=DEV)
    image, final_T, n_contrib, values, ranges, _, _ = _get_rasterizer().rasterize(*inputs, bg, width, height)
    want_image, _, want_T, want_nc, want_values, _ = oracle_render(inputs, width, height, bg)
    np.testing.assert_array_equal(np_(values), want_values)
    assert_forward_exact((image, final_T, n_contrib), (want_image, want_T, want_nc))
    g = torch.Generator().manual_seed(100 + seed)
    features = torch.rand(n, 32, generator=g).to(DEV)
    _, fimg = rasterize(*inputs, width, height, bg, features=features)
    assert_image_close(np_(fimg), oracle_render(inputs, width, height, bg, features)[1], max_error=1e-3,
                       max_perc_99=5e-4)
    grad_image = torch.rand(height, width, 3, generator=g).to(DEV)
    grad_feat = torch.rand(height, width, 32, generator=g).to(DEV)
    got = grads_gpu(inputs, width, height, features, grad_image, grad_feat, bg)
    want = grads_oracle(inputs, width, height, features, grad_image, grad_feat, bg)
    assert_grads_close(("means2D", "conics", "colors", "opacities", "features"), got, want)


def test_kernel_profile_records_only_the_named_kernels():
    """hds_profile_begin_only: with kernel names given, only those launches get timing events (what
    bench.py relies on inside its timed region); without, every hot-path launch does."""
    from gaussian_splatting.rasterizer._native import KernelProfile

    width, height = 64, 48
    inputs = scene(0, 800, width, height)
    features = torch.rand(800, 32, generator=torch.Generator().manual_seed(2)).to(DEV).requires_grad_(True)

    def step():
        image, fimg = rasterize(*inputs, width, height, features=features)
        torch.autograd.backward((image, fimg), (torch.ones_like(image), torch.ones_like(fimg)))
        torch.cuda.synchronize()

    step()
    with KernelProfile(only=("backward_geometry_kernel", "backward_features_kernel")) as only:
        step()
    with KernelProfile() as every:
        step()
    assert set(only.summary()) == {"backward_geometry_kernel", "backward_features_kernel"}
    assert {"render_forward_kernel", "backward_geometry_kernel", "backward_features_kernel"} <= set(every.summary())
    assert all(v["mean_ms"] > 0 for v in only.summary().values())


def test_unsupported_feature_width_is_rejected():
    inputs = scene(0, 100, 32, 32)
    with pytest.raises(RuntimeError, match="32, 64, 128, 256 or 512"):
        rasterize(*inputs, 32, 32, features=torch.rand(100, 24, device=DEV))


# ---- SSIM and SH ------------------------------------------------------------------------------

@pytest.mark.parametrize("height,width", [(64, 64), (37, 53), (11, 11), (546, 979)])
def test_ssim_matches_oracle(height, width):
    g = torch.Generator().manual_seed(height * width)
    gt = torch.rand(height, width, 3, generator=g)
    rendered = (gt + 0.1 * torch.randn(height, width, 3, generator=g)).clamp(0, 1)
    ext = _get_rasterizer()
    got = ext.ssim_forward(rendered.to(DEV), gt.to(DEV))
    want = oracle.ssim_forward(np_(rendered), np_(gt))
    for name, a, b in zip(("map", "d_mu", "d_aa", "d_ab"), got, want):
        np.testing.assert_allclose(np_(a), b, rtol=1e-4, atol=1e-6, err_msg=name)
    grad = ext.ssim_backward(torch.tensor([0.7], device=DEV), rendered.to(DEV), gt.to(DEV), *got[1:])
    want_grad = oracle.ssim_backward(0.7, np_(rendered), np_(gt), *want[1:])
    np.testing.assert_allclose(np_(grad), want_grad, rtol=1e-4, atol=1e-9)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_eval_sh_matches_oracle(degree):
    g = torch.Generator().manual_seed(degree)
    n = 5000
    sh = torch.randn(n, 16, 3, generator=g) * 0.5
    dirs = torch.nn.functional.normalize(torch.randn(n, 3, generator=g), dim=-1)
    radii = (torch.rand(n, generator=g) > 0.1).float()
    got = _get_rasterizer().eval_sh(sh[:, :1].contiguous().to(DEV), sh[:, 1:].contiguous().to(DEV), dirs.to(DEV),
                                    degree, radii.to(DEV))
    want = oracle.eval_sh(np_(sh[:, :1]), np_(sh[:, 1:]), np_(dirs), degree, np_(radii))
    np.testing.assert_allclose(np_(got), want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("degree", [1, 3])
def test_sh_backward_adam_matches_oracle(degree):
    g = torch.Generator().manual_seed(10 + degree)
    n = 5000
    sh = torch.randn(n, 16, 3, generator=g) * 0.5
    dirs = torch.nn.functional.normalize(torch.randn(n, 3, generator=g), dim=-1)
    radii = (torch.rand(n, generator=g) > 0.1).float()
    grad_rgb = torch.randn(n, 3, generator=g)
    dc, rest = sh[:, :1].contiguous(), sh[:, 1:].contiguous()
    state = [torch.rand(n, 1, 3, generator=g) * 0.01, torch.rand(n, 1, 3, generator=g) * 1e-4,
             torch.rand(n, 15, 3, generator=g) * 0.01, torch.rand(n, 15, 3, generator=g) * 1e-4]
    dev = [t.to(DEV) for t in (dc, rest, *state)]
    step = torch.tensor(3.0, device=DEV)
    gd = _get_rasterizer().eval_sh_backward_adam(grad_rgb.to(DEV), dev[0], dev[1], dirs.to(DEV), degree, radii.to(DEV),
                                                 dev[2], dev[3], dev[4], dev[5], step, step, 0.0025, 0.0025 / 20,
                                                 0.9, 0.999, 1e-15)
    host = [np_(t).copy() for t in (dc, rest, *state)]
    want_gd = oracle.eval_sh_backward_adam(np_(grad_rgb), host[0], host[1], np_(dirs), degree, np_(radii), host[2],
                                           host[3], host[4], host[5], 3.0, 3.0, 0.0025, 0.0025 / 20, 0.9, 0.999, 1e-15)
    np.testing.assert_allclose(np_(gd), want_gd, rtol=1e-4, atol=1e-5)
    for a, b in zip(dev, host):
        np.testing.assert_allclose(np_(a), b, rtol=1e-5, atol=1e-7)


def _offset_copy(t, offset):
    """A contiguous device copy of t whose data starts `offset` floats into a larger buffer (offset 1:
    4-byte aligned only)."""
    buf = torch.zeros(t.numel() + offset, device=DEV)
    view = buf[offset:].view(t.shape)
    view.copy_(t.to(DEV))
    return view


@pytest.mark.parametrize("offset", [0, 1])
def test_sh_kernels_take_partial_blocks_and_unaligned_runs(offset):
    """eval_sh and the SH backward + Adam step through the C ABI with 5001 gaussians (the last
    256-gaussian block holds 137, so its 45-float coefficient run ends in a 1-float tail after the
    16-byte copies) and, with offset 1, sh_rest and the sh_rest moments 4 bytes off a 16-byte
    boundary (the 4-byte copy path); both against the oracle."""
    from gaussian_splatting.rasterizer._native import _ptr, _stream, load_library

    lib = load_library()
    g = torch.Generator().manual_seed(77)
    n, degree = 5001, 3
    sh = torch.randn(n, 16, 3, generator=g) * 0.5
    dirs = torch.nn.functional.normalize(torch.randn(n, 3, generator=g), dim=-1)
    radii = (torch.rand(n, generator=g) > 0.1).float()
    grad_rgb = torch.randn(n, 3, generator=g)
    dc, rest = sh[:, :1].contiguous(), sh[:, 1:].contiguous()
    state = [torch.rand(n, 1, 3, generator=g) * 0.01, torch.rand(n, 1, 3, generator=g) * 1e-4,
             torch.rand(n, 15, 3, generator=g) * 0.01, torch.rand(n, 15, 3, generator=g) * 1e-4]
    print(f"[test] SH kernels, n {n}, offset {offset}", file=sys.stderr, flush=True)
    d_dc, d_rest = dc.to(DEV), _offset_copy(rest, offset)
    d_dirs, d_radii, d_grad = dirs.to(DEV), radii.to(DEV), grad_rgb.to(DEV)
    assert (d_rest.data_ptr() % 16 == 0) == (offset == 0)
    rgb = torch.empty(n, 3, device=DEV)
    assert lib.hds_eval_sh(n, degree, _ptr(d_dc), _ptr(d_rest), _ptr(d_dirs), _ptr(d_radii), _ptr(rgb),
                           _stream(rgb.device)) == 0
    torch.cuda.synchronize()
    np.testing.assert_allclose(np_(rgb), oracle.eval_sh(np_(dc), np_(rest), np_(dirs), degree, np_(radii)),
                               rtol=1e-6, atol=1e-6)

    m_dc, v_dc = state[0].to(DEV), state[1].to(DEV)
    m_rest, v_rest = _offset_copy(state[2], offset), _offset_copy(state[3], offset)
    step = torch.tensor(3.0, device=DEV)
    grad_dirs = torch.empty(n, 3, device=DEV)
    assert lib.hds_eval_sh_backward_adam(n, degree, _ptr(d_grad), _ptr(d_dc), _ptr(d_rest), _ptr(d_dirs),
                                         _ptr(d_radii), _ptr(m_dc), _ptr(v_dc), _ptr(m_rest), _ptr(v_rest), _ptr(step),
                                         _ptr(step), 0.0025, 0.0025 / 20, 0.9, 0.999, 1e-15, _ptr(grad_dirs),
                                         _stream(step.device)) == 0
    torch.cuda.synchronize()
    host = [np_(t).copy() for t in (dc, rest, *state)]
    want_gd = oracle.eval_sh_backward_adam(np_(grad_rgb), host[0], host[1], np_(dirs), degree, np_(radii), host[2],
                                           host[3], host[4], host[5], 3.0, 3.0, 0.0025, 0.0025 / 20, 0.9, 0.999, 1e-15)
    np.testing.assert_allclose(np_(grad_dirs), want_gd, rtol=1e-4, atol=1e-5)
    for a, b in zip((d_dc, d_rest, m_dc, v_dc, m_rest, v_rest), host):
        np.testing.assert_allclose(np_(a), b, rtol=1e-5, atol=1e-7)
