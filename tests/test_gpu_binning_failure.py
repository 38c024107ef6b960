"""The binning's failure path: a look-back that gives up is reported and leaves no tile list to read.

The sorts and the count scan wait for their predecessors' published counts with a bounded poll
(decoupled look-back). If a wait ever ran out, the sorted list would be wrong and some of its
slots unwritten, so nothing may index it. The host forces the condition with
hds_set_lookback_limit(0), which makes every look-back give up before its first poll (no kernel
waits at all, every kernel runs to its end), and checks that:
  - a failed tile sort leaves every tile range (0, 0) and raises the tile-sort flag that
    hds_bin_status copies out;
  - a failed depth sort or count scan makes hds_bin_count fail, and the asynchronous path's resolve()
    raise;
  - with the default limit restored, the next binning equals the one before.
"""
import ctypes

import numpy as np
import pytest
import torch

from gaussian_splatting.rasterizer import _get_rasterizer
from gaussian_splatting.rasterizer._native import HipRasterizer, _ptr, _stream, load_library
from tests.test_gpu_parity import np_, project_both
from tests.scenes import synthetic_config

pytestmark = pytest.mark.gpu

DEV = "cuda"
DEFAULT_LIMIT = 4194304


@pytest.fixture
def lib():
    lib = load_library()
    yield lib
    lib.hds_set_lookback_limit(DEFAULT_LIMIT)


def scene():
    wl = synthetic_config(1, n=200_000, channels=1)
    (m2, d, r, c), _ = project_both(wl.means, wl.scales, wl.quats, wl.opacities, wl.cam)
    return m2, d, r, c, wl.opacities.to(DEV), wl.width, wl.height


def test_failed_tile_sort_leaves_every_range_empty_and_is_reported(lib):
    m2, d, r, c, op, width, height = scene()
    want_values, want_ranges, _, _ = _get_rasterizer().bin(m2, d, r, c, None, op, width, height)
    n = m2.shape[0]
    tiles = want_ranges.shape[0]
    conic4 = torch.empty((n, 4), device=DEV)
    ws = torch.empty(lib.hds_bin_workspace_bytes(n, width, height), device=DEV, dtype=torch.uint8)
    pairs = ctypes.c_int64(0)
    stream = _stream(m2.device)
    assert lib.hds_bin_count(n, _ptr(m2), _ptr(d), _ptr(r), _ptr(c), None, _ptr(op), width, height, _ptr(conic4),
                             None, _ptr(ws), ws.numel(), ctypes.byref(pairs), stream) == 0
    p = int(pairs.value)
    assert p == want_values.numel() and p > 100_000
    values = torch.full((p,), -7, device=DEV, dtype=torch.int32)
    ranges = torch.full((tiles, 2), -7, device=DEV, dtype=torch.int32)
    pws = torch.empty(lib.hds_pairs_workspace_bytes(p, width, height), device=DEV, dtype=torch.uint8)
    lib.hds_set_lookback_limit(0)  # the tile sort's look-backs give up
    assert lib.hds_bin_emit(n, p, width, height, _ptr(ws), _ptr(pws), pws.numel(), _ptr(values), _ptr(ranges),
                            stream) == 0
    status = torch.zeros(2, dtype=torch.int64, pin_memory=True)
    assert lib.hds_bin_status(n, _ptr(ws), _ptr(status), stream) == 0
    torch.cuda.synchronize()
    lib.hds_set_lookback_limit(DEFAULT_LIMIT)
    word = int(status[1])
    assert int(status[0]) == p
    assert word & 0xFFFFFFFF == 0, "the depth sort and scan ran with the default limit"
    assert word >> 32 == 1, "the tile sort's failure must be reported"
    assert int(ranges.abs().sum()) == 0, "a failed tile sort must leave every range empty"


def test_failed_depth_sort_fails_the_count_and_the_async_resolve(lib):
    m2, d, r, c, op, width, height = scene()
    ext = HipRasterizer()
    want_values, want_ranges, _, _ = ext.bin(m2, d, r, c, None, op, width, height)
    lib.hds_set_lookback_limit(0)
    with pytest.raises(RuntimeError, match="look-back did not complete"):
        ext.bin(m2, d, r, c, None, op, width, height)
    ext._pair_capacity[m2.device.index] = want_values.numel()
    bins = ext.bin_async(m2, d, r, c, None, op, width, height)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="look-back did not complete"):
        ext.resolve(bins)
    assert int(bins.tile_ranges.abs().sum()) == 0, "a capped emit after a failed count writes no range"
    lib.hds_set_lookback_limit(DEFAULT_LIMIT)
    values, ranges, _, _ = ext.bin(m2, d, r, c, None, op, width, height)
    assert torch.equal(values, want_values) and torch.equal(ranges, want_ranges)


def test_failed_tile_count_scan_fails_the_resolve_and_leaves_every_range_empty(lib):
    """Tile order by counting scatter: when the scan of the (tile, chunk) count matrix gives up, the
    scatter writes nothing, the per-tile sort does not run, every tile range stays (0, 0) and resolve()
    raises; with the default limit restored the next tile-order binning equals the depth-order one."""
    m2, d, r, c, op, width, height = scene()
    ext = HipRasterizer()
    want_values, want_ranges, _, _ = ext.bin(m2, d, r, c, None, op, width, height)
    ext._pair_capacity[m2.device.index] = want_values.numel()
    ext.tile_order = True
    lib.hds_set_lookback_limit(0)
    bins = ext.bin_async(m2, d, r, c, None, op, width, height)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="look-back did not complete"):
        ext.resolve(bins)
    assert int(bins.tile_ranges.abs().sum()) == 0, "a failed count scan writes no range"
    lib.hds_set_lookback_limit(DEFAULT_LIMIT)
    bins = ext.bin_async(m2, d, r, c, None, op, width, height)
    assert not ext.resolve(bins)
    assert torch.equal(bins.values, want_values) and torch.equal(bins.tile_ranges, want_ranges)
