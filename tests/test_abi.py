"""The C-ABI library and the Python mirror of the reference API, checked without a GPU.

The library must load and export every entry point include/hds_rasterizer.h declares, the ctypes
prototypes must match the header, and argument validation (which runs before anything touches the
device) must reject bad input with the reference's messages. No kernel is launched here.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hds_rasterizer.h"


def declared_functions() -> dict[str, int]:
    """name -> parameter count of every HDS_API function in the public header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"HDS_API\s+[\w\s\*]+?\b(hds_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


@pytest.fixture(scope="module")
def lib():
    from gaussian_splatting.rasterizer._native import load_library

    return load_library()


def test_header_declares_the_reference_entry_points():
    names = declared_functions()
    # One C entry per reference extension function (bindings.cpp:4-42), rasterize split around the
    # host read of the pair count.
    for name in ("hds_project_gaussians", "hds_project_gaussians_backward", "hds_eval_sh",
                 "hds_eval_sh_backward_adam", "hds_bin_count", "hds_bin_emit", "hds_render", "hds_render_backward",
                 "hds_ssim_forward", "hds_ssim_backward"):
        assert name in names, name


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"


def test_ctypes_prototypes_match_the_header():
    from gaussian_splatting.rasterizer._native import PROTOTYPES

    declared = declared_functions()
    assert set(PROTOTYPES) == set(declared)
    for name, (_, argtypes) in PROTOTYPES.items():
        assert len(argtypes) == declared[name], f"{name}: {len(argtypes)} ctypes args vs {declared[name]} declared"


def test_abi_version_matches_header(lib):
    version = int(re.search(r"#define HDS_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.hds_abi_version() == version


def test_kernel_profile_records_nothing_without_launches(lib):
    """hds_profile_* brackets kernel launches with events; with no launch in between there is nothing
    to record, and asking for a record that does not exist is an error with a message."""
    from gaussian_splatting.rasterizer._native import KernelProfile

    with KernelProfile() as prof:
        pass
    assert prof.records == [] and prof.timeline == [] and prof.summary() == {}
    name, ms, end = ctypes.c_char_p(), ctypes.c_float(), ctypes.c_float()
    assert lib.hds_profile_record(0, ctypes.byref(name), ctypes.byref(ms)) != 0
    assert b"no record 0" in lib.hds_last_error()
    assert lib.hds_profile_timeline(0, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(end)) != 0
    assert b"no record 0" in lib.hds_last_error()


def test_workspace_queries_grow_with_the_problem(lib):
    small = lib.hds_bin_workspace_bytes(1000, 128, 128)
    big = lib.hds_bin_workspace_bytes(1_000_000, 128, 128)
    assert 0 < small < big and big >= 7 * 4 * 1_000_000
    # The tile-order count matrix: 4 bytes per (tile, 4096-gaussian chunk), 245 x 64 here, which the
    # depth-order size (no tiles) leaves out; above 2^24 words it is not reserved at all.
    assert big - lib.hds_bin_workspace_bytes(1_000_000, 0, 0) >= 4 * 245 * 64
    assert (lib.hds_bin_workspace_bytes(4096 * 4097, 64 * 16, 64 * 16)
            - lib.hds_bin_workspace_bytes(4096 * 4097, 0, 0)) < 1 << 20
    assert lib.hds_pairs_workspace_bytes(10_000, 64, 64) >= 3 * 4 * 10_000


def test_unsupported_feature_width_is_rejected_before_launch(lib):
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    status = lib.hds_render(10, 32, 32, 24, fake, fake, 10, fake, fake, None, None, fake, None, fake, fake, fake, None)
    assert status == 1
    assert b"32, 64, 128, 256 or 512" in lib.hds_last_error()


def test_bad_slice_width_is_rejected_before_launch(lib):
    fake = ctypes.c_void_p(16)
    status = lib.hds_render_backward(10, 32, 32, 128, 48, fake, fake, 10, fake, fake, None, None, fake, fake, None,
                                     fake, fake, fake, fake, None, fake, None, None)
    assert status == 1 and b"slices of 48" in lib.hds_last_error()


def test_zero_fill_rejects_bad_ranges_before_launch(lib):
    assert lib.hds_zero_async(None, -4, 0, None) == 1 and b"negative" in lib.hds_last_error()
    assert lib.hds_zero_async(ctypes.c_void_p(16), 8, -1, None) == 1 and b"negative" in lib.hds_last_error()
    assert lib.hds_zero_async(ctypes.c_void_p(20), 8, 0, None) == 1 and b"16-byte aligned" in lib.hds_last_error()
    assert lib.hds_zero_async(ctypes.c_void_p(16), 6, 0, None) == 1 and b"multiple of 4" in lib.hds_last_error()
    assert lib.hds_zero_async(None, 0, 0, None) == 0  # nothing to clear, nothing enqueued


def test_tile_order_binning_rejects_bad_arguments_before_launch(lib):
    fake = ctypes.c_void_p(16)

    def call(width=32, capacity=8, status=fake, workspace_bytes=1 << 20, pairs_bytes=1 << 20):
        return lib.hds_bin_tile_order_async(10, fake, fake, fake, fake, None, fake, width, 32, fake, None, fake,
                                            workspace_bytes, capacity, fake, pairs_bytes, fake, fake, status, None)

    assert call(status=None) == 1 and b"null status_host" in lib.hds_last_error()
    assert call(capacity=-1) == 1 and b"capacity" in lib.hds_last_error()
    assert call(width=0) == 1 and b"must be positive" in lib.hds_last_error()
    assert call(workspace_bytes=16) == 1 and b"workspace of 16 bytes" in lib.hds_last_error()
    # The counting scatter (a 1 x 4 count matrix here) uses no pairs workspace; the emit + pair sort,
    # which a matrix above the limit takes, checks it.
    assert call(pairs_bytes=16, workspace_bytes=16) == 1 and b"workspace of 16 bytes" in lib.hds_last_error()
    assert lib.hds_set_tile_scatter_limit(1) == 0
    try:
        assert call(pairs_bytes=16) == 1 and b"pairs workspace" in lib.hds_last_error()
    finally:
        assert lib.hds_set_tile_scatter_limit(0) == 0


def test_emits_reject_a_workspace_no_matching_count_filled(lib):
    """Each emit reads what its own count left in the gaussian workspace (depth-ordered offsets and
    rectangles, or index-ordered ones); an emit handed a workspace the other count filled, or that
    no count filled, is rejected before any launch."""
    fake = ctypes.c_void_p(1 << 20)
    args = (10, 8, 32, 32, fake, fake, 1 << 20, fake, fake, None)
    assert lib.hds_bin_emit(*args) == 1 and b"not filled by a count" in lib.hds_last_error()
    assert lib.hds_bin_emit_capped(*args) == 1 and b"not filled by a count" in lib.hds_last_error()
    assert lib.hds_bin_emit_tile_order(*args) == 1 and b"hds_bin_tile_order_async" in lib.hds_last_error()
    # With nothing to emit the workspace is not read: the tile ranges are only cleared (a launch, so
    # not called here).


def test_static_binning_rejects_a_null_values_sorted_before_launch(lib):
    fake = ctypes.c_void_p(16)
    st = lib.hds_bin_static(10, fake, fake, fake, fake, None, fake, 32, 32, fake, None, 8, None, fake, fake, None)
    assert st == 1 and b"null values_sorted" in lib.hds_last_error()


def test_render_clear_rejects_bad_ranges_before_launch(lib):
    fake = ctypes.c_void_p(16)

    def call(clear, count):
        # A valid-looking RGB render of 10 pairs; the range checks come first.
        return lib.hds_render_clear(10, 32, 32, 0, fake, fake, 10, fake, fake, fake, fake, None, fake, fake, fake,
                                    None, clear, count, None)

    assert call(fake, -4) == 1 and b"negative" in lib.hds_last_error()
    assert call(None, 8) == 1 and b"16-byte aligned" in lib.hds_last_error()
    assert call(ctypes.c_void_p(20), 8) == 1 and b"16-byte aligned" in lib.hds_last_error()
    assert call(fake, 6) == 1 and b"multiple of 4" in lib.hds_last_error()
    # Past the range checks, the render's own checks still apply.
    status = lib.hds_render_clear(10, 0, 32, 0, fake, fake, 10, fake, fake, fake, fake, None, fake, fake, fake, None,
                                  fake, 8, None)
    assert status == 1 and b"must be positive" in lib.hds_last_error()


def test_bad_image_size_and_sh_degree_are_rejected(lib):
    status = lib.hds_eval_sh(10, 4, None, None, None, None, None, None)
    assert status == 1 and b"degree 4" in lib.hds_last_error()
    pairs = ctypes.c_int64(-1)
    status = lib.hds_bin_count(10, None, None, None, None, None, None, 0, 10, None, None, None, 0,
                               ctypes.byref(pairs), None)
    assert status == 1 and b"image size" in lib.hds_last_error() and pairs.value == 0


def test_python_api_mirrors_the_reference_module():
    import gaussian_splatting.rasterizer as rasterizer
    from gaussian_splatting.rasterizer.projection import JACOBIAN_FOV_SCALE, LOW_PASS, NEAR_PLANE
    from gaussian_splatting.utils import loss, sh

    assert rasterizer.FEATURE_SLICE_WIDTH is None
    assert (NEAR_PLANE, LOW_PASS, JACOBIAN_FOV_SCALE) == (0.2, 0.3, 1.3)
    ext = rasterizer._get_rasterizer()
    for name in ("rasterize", "rasterize_backward", "rasterize_features", "rasterize_features_backward", "eval_sh",
                 "eval_sh_backward_adam", "ssim_forward", "ssim_backward", "project_gaussians",
                 "project_gaussians_backward"):
        assert callable(getattr(ext, name)), name
    for name in ("rasterize", "project_gaussians", "RasterizeGaussians", "_get_rasterizer"):
        assert hasattr(rasterizer, name)
    for name in ("eval_sh", "rgb_to_sh", "num_sh_coeffs", "EvalSH", "_adam_slot"):
        assert hasattr(sh, name)
    for name in ("ssim", "l1_loss", "psnr", "FusedSSIM"):
        assert hasattr(loss, name)
    assert sh.num_sh_coeffs(3) == 16


def test_host_tensors_are_refused_not_computed_on_the_cpu():
    from gaussian_splatting.rasterizer import rasterize

    n = 4
    with pytest.raises(RuntimeError, match="CUDA"):
        rasterize(torch.zeros(n, 2), torch.ones(n), torch.ones(n), torch.ones(n, 3), torch.ones(n, 3),
                  torch.full((n, 1), 0.5), 16, 16)


def test_rasterize_asserts_shapes_like_the_reference():
    from gaussian_splatting.rasterizer import rasterize

    with pytest.raises(AssertionError):
        rasterize(torch.zeros(4, 3), torch.ones(4), torch.ones(4), torch.ones(4, 3), torch.ones(4, 3),
                  torch.full((4, 1), 0.5), 16, 16)


def test_sh_backward_requires_the_named_adam():
    from gaussian_splatting.utils.sh import EvalSH

    class Ctx:
        optimizer = None

    with pytest.raises(RuntimeError, match="needs the Adam"):
        EvalSH.backward(Ctx(), torch.zeros(1, 3))


def test_static_binning_scratch_holds_the_documented_scene(lib):
    """hds_bin_static's scratch (HDS_BIN_STATIC_SCRATCH_MIB) fits the workspaces of 1.5M gaussians
    with 4M pairs, as its declaration states, and the headline scene with 25% pair headroom."""
    mib = int(re.search(r"#define HDS_BIN_STATIC_SCRATCH_MIB (\d+)", HEADER.read_text()).group(1))
    for n, pairs in ((1_500_000, 4_000_000), (1_180_000, int(1.25 * 1_921_191))):
        assert lib.hds_bin_workspace_bytes(n, 979, 546) + lib.hds_pairs_workspace_bytes(pairs, 979, 546) <= mib << 20


def test_debug_mode_prints_the_reference_binning_line(monkeypatch, capsys):
    """GS_DEBUG (or HDS_DEBUG) prints the reference's one-line binning statistics (common.cuh:93-101)
    once the pair count is known; without it nothing is printed."""
    from gaussian_splatting.rasterizer._native import _debug_pairs

    monkeypatch.delenv("HDS_DEBUG", raising=False)
    monkeypatch.delenv("GS_DEBUG", raising=False)
    _debug_pairs(1000, 979, 546, 2500)
    assert capsys.readouterr().err == ""
    monkeypatch.setenv("GS_DEBUG", "1")
    _debug_pairs(1000, 979, 546, 2500)
    assert capsys.readouterr().err == (
        "[gs] gaussians=1000  tiles=62x35(2170)  duplicates=2500  dup/gaussian=2.5  dup/tile=1.2\n")
