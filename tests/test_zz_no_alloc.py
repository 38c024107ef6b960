"""hds_bin_static, the binning entry point that allocates nothing, against the binning with workspaces.

hds_bin_static runs hds_bin_count_async + hds_bin_emit_capped with both workspaces in the library's
static device scratch. Through the C ABI it must give, bit for bit, what hds_bin_count + hds_bin_emit
give with caller-allocated workspaces (values_sorted, tile_ranges, conic4, color_opacity4 and the
pair count), on two calls in a row, the second with a smaller scene; and reject, before touching
the device, a scene whose workspaces exceed the scratch.
"""
import ctypes

import pytest
import torch

from gaussian_splatting.rasterizer import _get_rasterizer
from gaussian_splatting.rasterizer._native import _ptr, _stream, load_library
from gaussian_splatting.rasterizer.projection import JACOBIAN_FOV_SCALE, LOW_PASS, NEAR_PLANE
from tests.scenes import synthetic_config

pytestmark = pytest.mark.gpu

DEV = "cuda"


def projected(index: int, n: int | None = None):
    wl = synthetic_config(index, n=n, channels=1)
    cam = wl.cam
    opac = wl.opacities.to(DEV)
    m2, d, r, c = _get_rasterizer().project_gaussians(
        wl.means.to(DEV), wl.scales.to(DEV), wl.quats.to(DEV), opac, torch.eye(4, device=DEV), cam["fx"], cam["fy"],
        cam["cx"], cam["cy"], wl.width, wl.height, NEAR_PLANE, LOW_PASS, JACOBIAN_FOV_SCALE)
    colors = torch.rand(wl.n, 3, generator=torch.Generator().manual_seed(index)).to(DEV)
    return m2, d, r, c, colors, opac, wl.width, wl.height


def bin_static(m2, d, r, c, colors, opac, width, height, capacity):
    lib = load_library()
    n = m2.shape[0]
    tiles = ((width + 15) // 16) * ((height + 15) // 16)
    conic4 = torch.empty((n, 4), device=DEV)
    color4 = torch.empty((n, 4), device=DEV)
    values = torch.full((capacity,), -1, device=DEV, dtype=torch.int32)
    ranges = torch.full((tiles, 2), -1, device=DEV, dtype=torch.int32)
    status = torch.full((2,), -1, dtype=torch.int64, pin_memory=True)
    st = lib.hds_bin_static(n, _ptr(m2), _ptr(d), _ptr(r), _ptr(c), _ptr(colors), _ptr(opac), width, height,
                            _ptr(conic4), _ptr(color4), capacity, _ptr(values), _ptr(ranges), _ptr(status),
                            _stream(m2.device))
    assert st == 0, lib.hds_last_error().decode()
    torch.cuda.synchronize()
    return values, ranges, conic4, color4, int(status[0]), int(status[1])


def test_static_binning_equals_the_workspace_binning_on_two_calls_in_a_row():
    for index, n in ((1, None), (0, 6000)):  # 200k gaussians at 979x546, then 6000 at 128x128
        scene = projected(index, n)
        want_values, want_ranges, want_conic4, want_color4 = _get_rasterizer().bin(*scene)
        p = want_values.numel()
        assert p > 0
        values, ranges, conic4, color4, total, flags = bin_static(*scene, capacity=p + 1000)
        assert total == p and flags == 0
        assert torch.equal(values[:p], want_values)
        assert torch.equal(ranges, want_ranges)
        assert torch.equal(conic4, want_conic4) and torch.equal(color4, want_color4)


def test_static_binning_reports_a_short_capacity():
    scene = projected(0, 6000)
    p = _get_rasterizer().bin(*scene)[0].numel()
    values, ranges, _, _, total, flags = bin_static(*scene, capacity=p // 2)
    assert total == p and flags == 0  # the caller sees P > capacity and bins again
    assert int(ranges.max()) <= p // 2


def test_static_binning_rejects_scenes_beyond_its_scratch():
    lib = load_library()
    dummy = ctypes.c_void_p(16)
    st = lib.hds_bin_static(20_000_000, dummy, dummy, dummy, dummy, None, dummy, 1920, 1080, dummy, None, 1 << 26,
                            dummy, dummy, dummy, None)
    assert st == 1
    assert "more than its" in lib.hds_last_error().decode()
