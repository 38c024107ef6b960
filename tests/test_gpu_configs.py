"""Blend forward + backward against the CPU oracle at the BASELINE.json scales, through the C ABI.

Each test renders a BASELINE config on the GPU (HIP projection, SH colours, binning, fused RGB +
feature blend, autograd backward of U[0, 1] upstream gradients), then runs the same frame through
the oracle and compares, at the rasterizer's own inputs (means2D, conics, colours, opacities,
features):
  - the tile lists, bit for bit;
  - the RGB image, final T and n_contrib bit for bit (both sides take alpha from hds_gauss_alpha and
    accumulate with the same fused multiply-adds in list order), the feature image within max 1e-3 /
    p99 5e-4 (split-bf16 MFMA sums);
  - every gradient within assert_grads_close (rtol 1e-3 with an atol of 1e-4 max|want|, < 0.1% of
    values outside, largest error 2e-3 max|want|; the reference's bar, tests/test_render.py:45-58
    there).

Configs 1, 2 and 3 (200k and 1.18M gaussians at 979x546, C = 32 ... 512) run the whole frame.
Config 4 (4M gaussians at 1920x1080, C = 256, ~94M pairs) is too large for the oracle's sort, so the
comparison is restricted to 64 tiles: the 16 with the longest lists and 48 drawn at random. The
oracle bins only those tiles (their lists equal the full binning's) and the upstream gradients are
zero outside them; tiles are independent in the forward and add up in the backward, so the GPU's
full-frame gradients must then equal the oracle's. Its loss gradient (0.8 L1 + 0.2 (1 - SSIM) against
a U[0, 1] target, main.py:179-182 there) is checked against the oracle's SSIM on the same image.
"""
from __future__ import annotations

import sys
import time

import numpy as np
import pytest
import torch

import oracle
from gaussian_splatting.rasterizer import _get_rasterizer, rasterize
from gaussian_splatting.rasterizer.projection import JACOBIAN_FOV_SCALE, LOW_PASS, NEAR_PLANE
from gaussian_splatting.utils.loss import l1_loss, ssim
from tests.scenes import pixel_mask, synthetic_config, tile_selection, upstream, view_dirs
from tests.tolerances import assert_grads_close, assert_image_close, grad_error

pytestmark = pytest.mark.gpu

DEV = "cuda"
GRAD_NAMES = ("means2D", "conics", "colors", "opacities", "features")


def np_(t):
    return t.detach().cpu().numpy()


def log(msg: str) -> None:
    print(f"[configs] {msg}", file=sys.stderr, flush=True)


def project_and_shade(wl):
    """HIP projection and degree-3 SH colours of a workload: the rasterizer's inputs on the device."""
    ext = _get_rasterizer()
    cam = wl.cam
    means, scales, quats, opac = (t.to(DEV) for t in (wl.means, wl.scales, wl.quats, wl.opacities))
    m2, d, r, c = ext.project_gaussians(means, scales, quats, opac, torch.eye(4, device=DEV), cam["fx"], cam["fy"],
                                        cam["cx"], cam["cy"], wl.width, wl.height, NEAR_PLANE, LOW_PASS,
                                        JACOBIAN_FOV_SCALE)
    colors = ext.eval_sh(wl.sh_dc.to(DEV), wl.sh_rest.to(DEV), view_dirs(means), 3, r)
    return m2, d, r, c, colors, opac


def report_worst(name, got, want, extra: dict[str, np.ndarray], k: int = 5) -> str:
    """The k largest errors of one gradient with the gaussians' records, for a failure message."""
    got, want = np.asarray(got).reshape(want.shape[0], -1), np.asarray(want).reshape(want.shape[0], -1)
    err = np.abs(got.astype(np.float64) - want).max(axis=1)
    lines = [f"{name}: max|want| {np.abs(want).max():.4e}"]
    for g in np.argsort(-err)[:k]:
        rec = ", ".join(f"{key} {np.round(v[g], 4).tolist()}" for key, v in extra.items())
        lines.append(f"  gaussian {g}: got {got[g].tolist()} want {want[g].tolist()} ({rec})")
    return "\n".join(lines)


def frame_parity(wl, tile_mask: np.ndarray | None = None, loss: bool = False, frozen: bool = False):
    """Renders `wl` on the GPU and in the oracle (restricted to tile_mask when given) and compares."""
    W, H, C, N = wl.width, wl.height, wl.channels, wl.n
    t0 = time.perf_counter()
    m2, d, r, c, colors, opac = project_and_shade(wl)
    features = wl.features.to(DEV)
    ext = _get_rasterizer()
    values, ranges, _, _ = ext.bin(m2, d, r, c, None, opac, W, H)
    ranges_np = np_(ranges)
    if isinstance(tile_mask, str):  # "select"
        tile_mask = tile_selection(ranges_np, (W + 15) // 16)
    pix = None if tile_mask is None else pixel_mask(tile_mask, W, H)

    grad_image, grad_feat = upstream(2, H, W, C, device=DEV)
    target = grad_image.clone() if loss else None
    leaves = [t.detach().clone().requires_grad_(True) for t in (m2, c, colors, opac)]
    leaves.append(features.clone().requires_grad_(not frozen))
    image, fimg = rasterize(leaves[0], d, r, leaves[1], leaves[2], leaves[3], W, H, features=leaves[4])
    if loss:
        # dL/dimage of 0.8 L1 + 0.2 (1 - SSIM) on the HIP SSIM kernels, checked below against the
        # oracle's SSIM on the same image.
        img = image.detach().clone().requires_grad_(True)
        (0.8 * l1_loss(img, target) + 0.2 * (1.0 - ssim(img, target))).backward()
        grad_image = img.grad.detach()
    if pix is not None:
        keep = torch.from_numpy(pix).to(DEV)
        grad_image = grad_image * keep[..., None]
        grad_feat = grad_feat * keep[..., None]
    torch.autograd.backward((image, fimg), (grad_image, grad_feat))
    torch.cuda.synchronize()
    got = {"image": np_(image), "feature_image": np_(fimg)}
    got.update({name: np_(leaf.grad) for name, leaf in zip(GRAD_NAMES, leaves) if leaf.grad is not None})
    _, T, nc, _, _, _, _ = ext.rasterize(m2, d, r, c, colors, opac, torch.zeros(3, device=DEV), W, H)
    got["final_T"], got["n_contrib"] = np_(T), np_(nc)
    gi_np, gf_np = np_(grad_image), np_(grad_feat)
    values_np = np_(values)
    del grad_feat, fimg, leaves
    log(f"{wl.name}: GPU done in {time.perf_counter() - t0:.1f} s, P = {values_np.size}")

    t1 = time.perf_counter()
    m2n, dn, rn, cn, coln, opn, fn = (np_(t) for t in (m2, d, r, c, colors, opac, features))
    _, want_values, want_ranges = oracle.bin_gaussians(m2n, dn, rn, cn, opn, W, H, tile_mask=tile_mask)
    bg = np.zeros(3, np.float32)
    w_image, w_T, w_nc, w_fimg = oracle.render_forward(W, H, want_ranges, want_values, m2n, cn, opn, coln, bg, fn)
    if loss:
        _, d_mu, d_aa, d_ab = oracle.ssim_forward(got["image"], np_(target))
        want_gi = (0.8 * np.sign(got["image"] - np_(target)) / got["image"].size).astype(np.float32)
        want_gi += oracle.ssim_backward(-0.2, got["image"], np_(target), d_mu, d_aa, d_ab)
        outside, rel = grad_error(np.where(pix[..., None], np_(grad_image), 0) if pix is not None else np_(grad_image),
                                  np.where(pix[..., None], want_gi, 0) if pix is not None else want_gi)
        assert outside < 1e-3 and rel <= 2e-3, f"loss gradient: {outside:.2e} outside, max error {rel:.2e}"
    want = oracle.render_backward(W, H, want_ranges, want_values, m2n, cn, opn, coln, bg, w_T, w_nc, gi_np, fn, gf_np)
    log(f"{wl.name}: oracle done in {time.perf_counter() - t1:.1f} s, compared pairs = {want_values.size}")

    # Tile lists: equal to the oracle's, tile for tile.
    if tile_mask is None:
        np.testing.assert_array_equal(values_np, want_values)
        np.testing.assert_array_equal(ranges_np, want_ranges)
    else:
        for t in np.flatnonzero(tile_mask):
            np.testing.assert_array_equal(values_np[ranges_np[t, 0]:ranges_np[t, 1]],
                                          want_values[want_ranges[t, 0]:want_ranges[t, 1]], err_msg=f"tile {t}")
    # Every decision is the oracle's: n_contrib, final T and the RGB image bit for bit.
    compared = np.ones((H, W), bool) if pix is None else pix
    sel = lambda a: a[compared]  # noqa: E731
    for name, want_arr in (("n_contrib", w_nc), ("final_T", w_T), ("image", w_image)):
        differ = int(np.sum(sel(got[name]) != sel(want_arr)))
        assert differ == 0, f"{name}: {differ} values differ from the oracle"
    assert_image_close(sel(got["feature_image"]), sel(w_fimg), max_error=1e-3, max_perc_99=5e-4)
    log(f"{wl.name}: images compared on {compared.sum()} pixels")

    wants = dict(zip(GRAD_NAMES, want))
    names = [n for n in GRAD_NAMES if n in got]
    if frozen:
        assert "features" not in got
    extra = {"means2D": m2n, "conic": cn, "opacity": opn.reshape(-1, 1)}
    for name in names:
        outside, rel = grad_error(got[name].reshape(wants[name].shape), wants[name])
        log(f"{wl.name}: {name} {outside:.2e} outside, max error {rel:.2e} of max|want|")
        if not (outside < 1e-3 and rel <= 2e-3):
            log(report_worst(name, got[name], wants[name], extra))
    assert_grads_close(names, [got[n].reshape(wants[n].shape) for n in names], [wants[n] for n in names])


def test_config1_mid_scene_full_frame():
    frame_parity(synthetic_config(1))


def test_config2_headline_full_frame():
    frame_parity(synthetic_config(2))


@pytest.mark.parametrize("channels", [32, 64, 256, 512])
def test_config3_channel_sweep_full_frame(channels):
    frame_parity(synthetic_config(3, channels=channels))


def test_config4_stress_scene_on_selected_tiles_with_the_loss():
    frame_parity(synthetic_config(4), tile_mask="select", loss=True)


def test_config0_with_the_loss_full_frame():
    frame_parity(synthetic_config(0), loss=True)


@pytest.mark.parametrize("channels", [32, 64, 128])
def test_frozen_features_still_shape_the_geometry_gradients(channels):
    """Features without requires_grad (reference tests/test_render.py:118-134): no feature gradient is
    written, but the geometry gradients keep the features' term."""
    wl = synthetic_config(1, n=50_000, channels=channels)
    frame_parity(wl, frozen=True)


def test_hip_path_reproduces_the_golden_config0_vectors():
    """tests/golden/oracle_config0_small.npz (the oracle on the first 2000 gaussians of config 0 with 8
    feature channels): projection, binning and the RGB image bit for bit, the feature image within its
    bar. The 8 channels ride in a 32-channel feature block whose other 24 channels are zero."""
    from pathlib import Path

    z = np.load(Path(__file__).resolve().parent / "golden" / "oracle_config0_small.npz")
    n = int(z["n"])
    cam = synthetic_config(0, n=16).cam
    W, H = cam["width"], cam["height"]
    ext = _get_rasterizer()
    dev = lambda name: torch.from_numpy(z[name]).to(DEV)  # noqa: E731
    opac = dev("opacities")
    m2, d, r, c = ext.project_gaussians(dev("means"), dev("scales"), dev("quats"), opac, torch.eye(4, device=DEV),
                                        cam["fx"], cam["fy"], cam["cx"], cam["cy"], W, H, NEAR_PLANE, LOW_PASS,
                                        JACOBIAN_FOV_SCALE)
    for name, got in (("means2D", m2), ("depths", d), ("radii", r), ("conics", c)):
        np.testing.assert_array_equal(np_(got), z[name], err_msg=name)
    colors = dev("colors")
    feats = torch.zeros(n, 32)
    feats[:, :8] = torch.from_numpy(z["features"])
    image, fimg = rasterize(m2, d, r, c, colors, opac, W, H, torch.zeros(3, device=DEV), features=feats.to(DEV))
    values, ranges, _, _ = ext.bin(m2, d, r, c, None, opac, W, H)
    np.testing.assert_array_equal(np_(values), z["values_sorted"])
    np.testing.assert_array_equal(np_(ranges), z["tile_ranges"])
    np.testing.assert_array_equal(np_(image), z["image"])
    assert_image_close(np_(fimg)[..., :8], z["feature_image"], max_error=1e-3, max_perc_99=5e-4)
    assert not np_(fimg)[..., 8:].any()
