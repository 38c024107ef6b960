"""ctypes binding of libhds_rasterizer.so (include/hds_rasterizer.h) behind the reference's extension API.

`HipRasterizer` exposes the ten functions of the reference's torch extension "gaussian_rasterizer"
(gaussian_splatting/rasterizer/bindings.cpp:4-42) with the same names, argument order and return
tuples, taking and returning torch tensors. Outputs are allocated here with the torch caching
allocator and raw pointers go to the C ABI together with torch's current HIP stream; the library
itself never allocates. On top of those ten it offers the fused calls the autograd functions use:
`bin` (binning only), `render` (RGB + features in one tile walk) and `render_backward`.

There is no CPU path: a missing library or a tensor off the GPU raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import math
import os
import sys
from pathlib import Path

import torch

_PACKAGE_ROOT = Path(__file__).resolve().parents[2]
LIBRARY_PATH = Path(os.environ.get("HDS_LIBRARY", _PACKAGE_ROOT / "lib" / "libhds_rasterizer.so"))

SUPPORTED_CHANNELS = (32, 64, 128, 256, 512)
TILE = 16

_i64, _i32, _f32, _f64, _vp, _sz = (ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double,
                                    ctypes.c_void_p, ctypes.c_size_t)

# name -> (restype, argtypes), exactly the prototypes of include/hds_rasterizer.h.
_CAMERA = [_f32, _f32, _f32, _f32, _i32, _i32, _f32, _f32, _f32]
PROTOTYPES = {
    "hds_last_error": (ctypes.c_char_p, []),
    "hds_abi_version": (_i32, []),
    "hds_zero_async": (_i32, [_vp, _i64, _i32, _vp]),
    "hds_project_gaussians": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp] + _CAMERA + [_vp, _vp, _vp, _vp, _vp]),
    "hds_project_gaussians_backward": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp] + _CAMERA + [_vp, _vp, _vp, _vp]),
    "hds_eval_sh": (_i32, [_i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hds_eval_sh_backward_adam": (_i32, [_i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                         _f64, _f64, _f64, _f64, _f64, _vp, _vp]),
    "hds_bin_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "hds_bin_count": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz,
                             ctypes.POINTER(ctypes.c_int64), _vp]),
    "hds_bin_count_async": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp, _vp]),
    "hds_pairs_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "hds_bin_emit": (_i32, [_i64, _i64, _i32, _i32, _vp, _vp, _sz, _vp, _vp, _vp]),
    "hds_bin_emit_capped": (_i32, [_i64, _i64, _i32, _i32, _vp, _vp, _sz, _vp, _vp, _vp]),
    "hds_bin_tile_order_async": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _i64,
                                        _vp, _sz, _vp, _vp, _vp, _vp]),
    "hds_bin_emit_tile_order": (_i32, [_i64, _i64, _i32, _i32, _vp, _vp, _sz, _vp, _vp, _vp]),
    "hds_bin_status": (_i32, [_i64, _vp, _vp, _vp]),
    "hds_set_lookback_limit": (_i32, [ctypes.c_uint32]),
    "hds_set_tile_scatter_limit": (_i32, [ctypes.c_uint64]),
    "hds_bin_static": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "hds_render": (_i32, [_i64, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                          _vp]),
    "hds_render_clear": (_i32, [_i64, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _vp, _vp, _i64, _vp]),
    "hds_render_backward": (_i32, [_i64, _i32, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hds_render_backward_accumulate": (_i32, [_i64, _i32, _i32, _i32, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
                                              _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hds_ssim_forward": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hds_ssim_backward": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hds_densification_stats": (_i32, [_i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp]),
    "hds_profile_begin": (_i32, []),
    "hds_profile_begin_only": (_i32, [ctypes.c_char_p]),
    "hds_profile_end": (_i64, []),
    "hds_profile_record": (_i32, [_i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_float)]),
    "hds_profile_timeline": (_i32, [_i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_float),
                                    ctypes.POINTER(ctypes.c_float)]),
}

_lib: ctypes.CDLL | None = None


def load_library() -> ctypes.CDLL:
    """Loads the HIP library once; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"HIP rasterizer library not found at {LIBRARY_PATH}; build it with "
            "`python -c 'import __graft_entry__; __graft_entry__.build()'` (or make -C high-dimensional-splatting_amd)")
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (restype, argtypes) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        raise RuntimeError(load_library().hds_last_error().decode(errors="replace"))


class KernelProfile:
    """Per-kernel HIP-event durations recorded inside the library (hds_profile_begin / _end).

    Used as a context manager around a timed region; afterwards `summary()` gives
    {kernel: {"launches": n, "total_ms": t, "mean_ms": t / n}}. Every hot-path launch is bracketed
    with events on its own stream, so the durations are those of the kernels themselves; with `only`
    (kernel names) just those launches are, which keeps the events' own cost out of the rest."""

    def __init__(self, only=None):
        self.only = None if only is None else ",".join(only)
        self.records: list[tuple[str, float]] = []
        self.timeline: list[tuple[str, float, float]] = []  # (kernel, start ms, end ms) from the first start

    def __enter__(self):
        lib = load_library()
        _check(lib.hds_profile_begin() if self.only is None else lib.hds_profile_begin_only(self.only.encode()))
        return self

    def __exit__(self, *exc):
        lib = load_library()
        count = lib.hds_profile_end()
        if count < 0:
            _check(-count)
        name, ms, t0, t1 = ctypes.c_char_p(), ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        for i in range(count):
            _check(lib.hds_profile_record(i, ctypes.byref(name), ctypes.byref(ms)))
            self.records.append((name.value.decode(), float(ms.value)))
            _check(lib.hds_profile_timeline(i, ctypes.byref(name), ctypes.byref(t0), ctypes.byref(t1)))
            self.timeline.append((name.value.decode(), float(t0.value), float(t1.value)))
        return False

    def summary(self) -> dict[str, dict[str, float]]:
        out: dict[str, dict[str, float]] = {}
        for name, ms in self.records:
            row = out.setdefault(name, {"launches": 0, "total_ms": 0.0})
            row["launches"] += 1
            row["total_ms"] += ms
        for row in out.values():
            row["mean_ms"] = row["total_ms"] / row["launches"]
        return out


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_BLACK: dict[int, torch.Tensor] = {}


def black_background(device: torch.device) -> torch.Tensor:
    """The default background (0, 0, 0) on `device`, made once per device: a fresh torch.zeros(3) in
    every call was one more fill kernel in every step. Read-only: nothing writes it."""
    index = torch.device(device).index
    index = torch.cuda.current_device() if index is None else index
    black = _BLACK.get(index)
    if black is None:
        black = _BLACK[index] = torch.zeros(3, device=torch.device("cuda", index), dtype=torch.float32)
    return black


def _dev(t: torch.Tensor, name: str) -> torch.Tensor:
    """The reference's TORCH_CHECK(is_cuda / is_contiguous), plus float32 and 16-byte alignment."""
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA (HIP) tensor")
    if t.dtype not in (torch.float32, torch.int32):
        raise RuntimeError(f"{name} must be float32 or int32, got {t.dtype}")
    if not t.is_contiguous() or t.data_ptr() % 16:
        t = t.contiguous() if not t.is_contiguous() else t.clone()
    return t


class StageTimer:
    """Brackets library calls with HIP events on the stream they run on (the current torch stream).

    The profiling counterpart of the reference's NVTX ranges (rasterizer/__init__.py:135, 153): while
    enabled, every timed call appends (stage, start, end) events; `summary()` synchronises and
    returns per-stage launch counts and mean milliseconds.
    """

    def __init__(self) -> None:
        self.events: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []

    def record(self, stage: str, fn):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        out = fn()
        end.record()
        self.events.append((stage, start, end))
        return out

    def summary(self) -> dict[str, dict[str, float]]:
        torch.cuda.synchronize()
        out: dict[str, dict[str, float]] = {}
        for stage, start, end in self.events:
            row = out.setdefault(stage, {"launches": 0, "total_ms": 0.0})
            row["launches"] += 1
            row["total_ms"] += start.elapsed_time(end)
        for row in out.values():
            row["mean_ms"] = row["total_ms"] / row["launches"]
        return out


def _raise_on_sort_error(status: torch.Tensor) -> bool:
    """Raises if the (pair count, depth/scan flag | tile-sort word << 32) words of hds_bin_status
    report a look-back that gave up; returns whether a tile-order binning met a tile list longer
    than its per-tile sort takes (bit 1 of the tile-sort word)."""
    word = int(status[1])
    if word & 0xFFFFFFFF:
        raise RuntimeError("bin_count: a sort or scan look-back did not complete")
    pair_word = (word >> 32) & 0xFFFFFFFF
    if pair_word & 1:
        raise RuntimeError("bin_emit: a look-back of the tile sort did not complete (every tile range left empty)")
    return bool(pair_word & 2)


def _debug_pairs(n: int, width: int, height: int, pairs: int) -> None:
    """With HDS_DEBUG or GS_DEBUG set, one line of binning statistics on stderr once the pair count
    is known, in the reference's debug format (common.cuh:93-101)."""
    if not (os.environ.get("HDS_DEBUG") or os.environ.get("GS_DEBUG")):
        return
    tx, ty = (width + TILE - 1) // TILE, (height + TILE - 1) // TILE
    print(f"[gs] gaussians={n}  tiles={tx}x{ty}({tx * ty})  duplicates={pairs}  "
          f"dup/gaussian={pairs / max(n, 1):.1f}  dup/tile={pairs / (tx * ty):.1f}", file=sys.stderr, flush=True)


class PendingBins:
    """A binning enqueued by HipRasterizer.bin_async whose pair count the host has not read yet.

    `values` is the capacity-sized pair buffer (exact once resolved), `tile_ranges`, `conic4` and
    `color_opacity4` are final as soon as the stream has run the binning."""

    def __init__(self, values, tile_ranges, conic4, color_opacity4, *, capacity=None, event=None, count=None,
                 workspace=None, emit_args=None, status=None, status_event=None):
        self.values = values
        self.tile_ranges = tile_ranges
        self.conic4 = conic4
        self.color_opacity4 = color_opacity4
        self.capacity = capacity        # None: already exact
        self.event = event              # recorded after the count's copy to `count`
        self.count = count              # pinned int64 [2]: pair count, look-back error flag
        self.workspace = workspace      # per-gaussian workspace the exact re-emit reads
        self.emit_args = emit_args      # (n, width, height, device)
        self.tile_order = False         # binned by hds_bin_tile_order_async
        self.inputs = None              # the binning inputs, for a rebin with the global depth sort
        self.status = status            # pinned int64 [2] of hds_bin_status after the capped emit
        self.status_event = status_event  # recorded after that copy


class HipRasterizer:
    """The reference extension's ten functions (bindings.cpp:4-42) on the HIP library, plus fused calls."""

    # Pair buffers of bin_async are sized this much above the last pair count seen on the device.
    PAIR_HEADROOM = 1.25
    # Longest tile list the tile-order binning sorts (hds_bin_tile_order_async), and the share
    # of it the last frame's longest list may reach for bin_async to choose that binning.
    TILE_ORDER_MAX = 4096
    TILE_ORDER_MARGIN = 0.9

    def __init__(self) -> None:
        self.lib = load_library()
        self.timer: StageTimer | None = None
        self._pair_capacity: dict[int, int] = {}
        # Per device: whether bin_async bins in tile order (set from the first frame's longest tile
        # list, cleared for good when a frame's list overflows). `tile_order` forces the choice.
        self._tile_order_ok: dict[int, bool] = {}
        self.tile_order: bool | None = None

    def gradient_buffers(self, n: int, channels: int, device: torch.device):
        """Output buffers for a later render_backward (grad_means2D [N,2], grad_conics [N,3],
        grad_colors [N,3], grad_opacities [N,1], grad_features [N,C]) as views of one allocation, each
        starting on a 256-byte boundary. Returns (storage, buffers): pass storage to render(clear=...),
        which zeroes it, and the buffers to render_backward(prezeroed=...)."""
        shapes = ((n, 2), (n, 3), (n, 3), (n, 1), (n, channels))
        offsets, total = [], 0
        for shape in shapes:
            offsets.append(total)
            total += (math.prod(shape) + 63) // 64 * 64
        storage = torch.empty((total,), device=device, dtype=torch.float32)
        return storage, tuple(storage[o:o + math.prod(shape)].view(shape) for o, shape in zip(offsets, shapes))

    def _run(self, stage: str, fn) -> None:
        """Runs one C call (raising on error), inside the stage timer when one is installed."""
        if self.timer is None:
            _check(fn())
        else:
            _check(self.timer.record(stage, fn))

    # -- projection ---------------------------------------------------------------------------

    def project_gaussians(self, means, scales, quats, opacities, world_to_camera, fx, fy, cx, cy, width, height,
                          near_plane, low_pass, fov_scale):
        """projection.cu:210-231: returns (means2D [N,2], depths [N], radii [N], conics [N,3])."""
        means, scales, quats = _dev(means, "means"), _dev(scales, "scales"), _dev(quats, "quats")
        opacities, pose = _dev(opacities, "opacities"), _dev(world_to_camera, "world_to_camera")
        n = means.shape[0]
        means2D = torch.empty((n, 2), device=means.device, dtype=torch.float32)
        depths = torch.empty((n,), device=means.device, dtype=torch.float32)
        radii = torch.empty((n,), device=means.device, dtype=torch.float32)
        conics = torch.empty((n, 3), device=means.device, dtype=torch.float32)
        with torch.cuda.device(means.device):
            self._run("project_forward", lambda: self.lib.hds_project_gaussians(
                n, _ptr(means), _ptr(scales), _ptr(quats), _ptr(opacities), _ptr(pose), float(fx), float(fy),
                float(cx), float(cy), int(width), int(height), float(near_plane), float(low_pass), float(fov_scale),
                _ptr(means2D), _ptr(depths), _ptr(radii), _ptr(conics), _stream(means.device)))
        return means2D, depths, radii, conics

    def project_gaussians_backward(self, grad_means2D, grad_conics, means, scales, quats, world_to_camera, fx, fy,
                                   cx, cy, width, height, near_plane, low_pass, fov_scale):
        """projection.cu:234-253: returns (grad_means, grad_scales, grad_quats)."""
        gm, gc = _dev(grad_means2D, "grad_means2D"), _dev(grad_conics, "grad_conics")
        means, scales, quats = _dev(means, "means"), _dev(scales, "scales"), _dev(quats, "quats")
        pose = _dev(world_to_camera, "world_to_camera")
        dm, ds, dq = torch.empty_like(means), torch.empty_like(scales), torch.empty_like(quats)
        with torch.cuda.device(means.device):
            self._run("project_backward", lambda: self.lib.hds_project_gaussians_backward(
                means.shape[0], _ptr(gm), _ptr(gc), _ptr(means), _ptr(scales), _ptr(quats), _ptr(pose), float(fx),
                float(fy), float(cx), float(cy), int(width), int(height), float(near_plane), float(low_pass),
                float(fov_scale), _ptr(dm), _ptr(ds), _ptr(dq), _stream(means.device)))
        return dm, ds, dq

    # -- spherical harmonics --------------------------------------------------------------------

    def eval_sh(self, sh_dc, sh_rest, dirs, degree, radii):
        """sh.cu:157-168: returns rgb [N,3]."""
        sh_dc, sh_rest = _dev(sh_dc, "sh_dc"), _dev(sh_rest, "sh_rest")
        dirs, radii = _dev(dirs, "dirs"), _dev(radii, "radii")
        n = sh_dc.shape[0]
        rgb = torch.empty((n, 3), device=sh_dc.device, dtype=torch.float32)
        with torch.cuda.device(sh_dc.device):
            self._run("eval_sh", lambda: self.lib.hds_eval_sh(n, int(degree), _ptr(sh_dc), _ptr(sh_rest), _ptr(dirs), _ptr(radii),
                                        _ptr(rgb), _stream(sh_dc.device)))
        return rgb

    def eval_sh_backward_adam(self, grad_rgb, sh_dc, sh_rest, dirs, degree, radii, m_dc, v_dc, m_rest, v_rest,
                              step_dc, step_rest, lr_dc, lr_rest, beta1, beta2, eps):
        """sh.cu:171-190: steps sh_dc / sh_rest and their moments in place, returns grad_dirs [N,3]."""
        for t, name in ((sh_dc, "sh_dc"), (sh_rest, "sh_rest"), (m_dc, "exp_avg"), (v_dc, "exp_avg_sq"),
                        (m_rest, "exp_avg"), (v_rest, "exp_avg_sq"), (step_dc, "step"), (step_rest, "step")):
            if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
                raise RuntimeError(f"{name} must be a contiguous float32 CUDA tensor (updated in place)")
        grad_rgb, dirs, radii = _dev(grad_rgb, "grad_rgb"), _dev(dirs, "dirs"), _dev(radii, "radii")
        grad_dirs = torch.empty_like(dirs)
        with torch.cuda.device(sh_dc.device):
            self._run("eval_sh_backward_adam", lambda: self.lib.hds_eval_sh_backward_adam(
                sh_dc.shape[0], int(degree), _ptr(grad_rgb), _ptr(sh_dc), _ptr(sh_rest), _ptr(dirs), _ptr(radii),
                _ptr(m_dc), _ptr(v_dc), _ptr(m_rest), _ptr(v_rest), _ptr(step_dc), _ptr(step_rest), float(lr_dc),
                float(lr_rest), float(beta1), float(beta2), float(eps), _ptr(grad_dirs), _stream(sh_dc.device)))
        return grad_dirs

    # -- binning + blend --------------------------------------------------------------------------

    def bin(self, means2D, depths, radii, conics, colors, opacities, width, height):
        """Binning of rasterize (forward.cu:284-404).

        Returns (values_sorted [P] int32, tile_ranges [T,2] int32, conic4 [N,4], color_opacity4 [N,4]).
        """
        means2D, depths, radii = _dev(means2D, "means2D"), _dev(depths, "depths"), _dev(radii, "radii")
        conics, opacities = _dev(conics, "conics"), _dev(opacities, "opacities")
        colors = None if colors is None else _dev(colors, "colors")
        dev = means2D.device
        n = means2D.shape[0]
        width, height = int(width), int(height)
        tiles = ((width + TILE - 1) // TILE) * ((height + TILE - 1) // TILE)
        conic4 = torch.empty((n, 4), device=dev, dtype=torch.float32)
        color_opacity4 = torch.empty((n, 4), device=dev, dtype=torch.float32)
        tile_ranges = torch.empty((tiles, 2), device=dev, dtype=torch.int32)
        with torch.cuda.device(dev):
            stream = _stream(dev)
            ws = torch.empty(self.lib.hds_bin_workspace_bytes(n, width, height), device=dev, dtype=torch.uint8)
            pairs = ctypes.c_int64(0)
            self._run("bin_count", lambda: self.lib.hds_bin_count(n, _ptr(means2D), _ptr(depths), _ptr(radii), _ptr(conics), _ptr(colors),
                                          _ptr(opacities), width, height, _ptr(conic4), _ptr(color_opacity4),
                                          _ptr(ws), ws.numel(), ctypes.byref(pairs), stream))
            p = int(pairs.value)
            _debug_pairs(n, width, height, p)
            values_sorted = torch.empty((p,), device=dev, dtype=torch.int32)
            pws = torch.empty(self.lib.hds_pairs_workspace_bytes(p, width, height) if p else 0, device=dev,
                              dtype=torch.uint8)
            self._run("bin_emit", lambda: self.lib.hds_bin_emit(n, p, width, height, _ptr(ws), _ptr(pws), pws.numel(), _ptr(values_sorted),
                                         _ptr(tile_ranges), stream))
            if p:
                # The pair sort's look-back flag (a failed sort leaves every tile range empty).
                status = torch.zeros(2, dtype=torch.int64, pin_memory=True)
                _check(self.lib.hds_bin_status(n, _ptr(ws), _ptr(status), stream))
                torch.cuda.current_stream(dev).synchronize()
                _raise_on_sort_error(status)
        return values_sorted, tile_ranges, conic4, color_opacity4

    def bin_async(self, means2D, depths, radii, conics, colors, opacities, width, height) -> PendingBins:
        """`bin` without the blocking read of P (forward.cu:311-326 deferred): the pair buffers are
        sized from the last pair count seen on this device and the count reaches the host by an
        asynchronous copy, so the render can be enqueued before the host knows P. `resolve` then
        reads P, and rebins exactly when the capacity was too small. The first call on a device
        has no history and bins synchronously. Later calls bin in tile order (no global depth sort,
        each tile's list ordered by depth in LDS; the same values_sorted and tile_ranges) while the
        device's longest tile list stays within TILE_ORDER_MARGIN of what that takes, else with
        the global depth sort."""
        dev = means2D.device
        if dev.index not in self._pair_capacity:
            values, ranges, conic4, color_opacity4 = self.bin(means2D, depths, radii, conics, colors, opacities,
                                                              width, height)
            self._remember_pairs(dev, values.numel())
            longest = int((ranges[:, 1] - ranges[:, 0]).max()) if ranges.numel() else 0
            self._tile_order_ok[dev.index] = longest <= self.TILE_ORDER_MARGIN * self.TILE_ORDER_MAX
            return PendingBins(values, ranges, conic4, color_opacity4)
        tile_order = self.tile_order if self.tile_order is not None else self._tile_order_ok.get(dev.index, False)
        means2D, depths, radii = _dev(means2D, "means2D"), _dev(depths, "depths"), _dev(radii, "radii")
        conics, opacities = _dev(conics, "conics"), _dev(opacities, "opacities")
        colors = None if colors is None else _dev(colors, "colors")
        # Kept for a rebin with the global depth sort, which passes their pointers to the library as
        # dense aligned float32: the converted tensors, not the caller's.
        inputs = (means2D, depths, radii, conics, colors, opacities)
        n = means2D.shape[0]
        width, height = int(width), int(height)
        tiles = ((width + TILE - 1) // TILE) * ((height + TILE - 1) // TILE)
        cap = self._pair_capacity[dev.index]
        conic4 = torch.empty((n, 4), device=dev, dtype=torch.float32)
        color_opacity4 = torch.empty((n, 4), device=dev, dtype=torch.float32)
        tile_ranges = torch.empty((tiles, 2), device=dev, dtype=torch.int32)
        with torch.cuda.device(dev):
            stream = _stream(dev)
            ws = torch.empty(self.lib.hds_bin_workspace_bytes(n, width, height), device=dev, dtype=torch.uint8)
            values = torch.empty((cap,), device=dev, dtype=torch.int32)
            pws = torch.empty(self.lib.hds_pairs_workspace_bytes(cap, width, height), device=dev, dtype=torch.uint8)
            status = torch.zeros(2, dtype=torch.int64, pin_memory=True)
            if tile_order:
                # One call: the whole binning, then its status words (P and the flags) to `status`.
                self._run("bin", lambda: self.lib.hds_bin_tile_order_async(
                    n, _ptr(means2D), _ptr(depths), _ptr(radii), _ptr(conics), _ptr(colors), _ptr(opacities), width,
                    height, _ptr(conic4), _ptr(color_opacity4), _ptr(ws), ws.numel(), cap, _ptr(pws), pws.numel(),
                    _ptr(values), _ptr(tile_ranges), _ptr(status), stream))
                count, event = status, torch.cuda.Event()
                event.record()
                status_event = event
            else:
                count = torch.zeros(2, dtype=torch.int64, pin_memory=True)
                self._run("bin_count", lambda: self.lib.hds_bin_count_async(
                    n, _ptr(means2D), _ptr(depths), _ptr(radii), _ptr(conics), _ptr(colors), _ptr(opacities), width,
                    height, _ptr(conic4), _ptr(color_opacity4), _ptr(ws), ws.numel(), _ptr(count), stream))
                event = torch.cuda.Event()
                event.record()
                self._run("bin_emit", lambda: self.lib.hds_bin_emit_capped(
                    n, cap, width, height, _ptr(ws), _ptr(pws), pws.numel(), _ptr(values), _ptr(tile_ranges), stream))
                _check(self.lib.hds_bin_status(n, _ptr(ws), _ptr(status), stream))
                status_event = torch.cuda.Event()
                status_event.record()
        pending = PendingBins(values, tile_ranges, conic4, color_opacity4, capacity=cap, event=event, count=count,
                              workspace=ws, emit_args=(n, width, height, dev), status=status,
                              status_event=status_event)
        pending.tile_order, pending.inputs = tile_order, inputs
        return pending

    def resolve(self, pending: PendingBins) -> bool:
        """Reads the pair count of a bin_async binning (waiting for its copy only, not for later
        work on the stream) and trims `pending.values` to it. If the count exceeded the capacity,
        bins again with exact buffers and returns True: whatever was rendered from the capped
        binning must be rendered again. So does a tile-order binning that met a tile list too long
        for its per-tile sort: the frame is binned again with the global depth sort (into the same
        tile_ranges, conic4 and color_opacity4), and the device stays on that binning."""
        if pending.capacity is None:
            return False
        pending.event.synchronize()
        total, error = int(pending.count[0]), int(pending.count[1]) & 0xFFFFFFFF
        n, width, height, dev = pending.emit_args
        cap = pending.capacity
        pending.capacity = None
        if error:
            raise RuntimeError("bin_count: a sort or scan look-back did not complete")
        # The capped emit's pair sort (its copy of the flags follows the sort, ahead of the render).
        pending.status_event.synchronize()
        overflow = _raise_on_sort_error(pending.status)
        if total >= 2**31 - 1:
            raise RuntimeError(f"bin_count: {total} tile-gaussian pairs overflow int32 indices")
        _debug_pairs(n, width, height, total)
        self._remember_pairs(dev, total)
        if total <= cap and not overflow:
            pending.values = pending.values[:total]
            return False
        values = torch.empty((total,), device=dev, dtype=torch.int32)
        with torch.cuda.device(dev):
            pws = torch.empty(self.lib.hds_pairs_workspace_bytes(total, width, height), device=dev,
                              dtype=torch.uint8)
            if not overflow:
                emit = self.lib.hds_bin_emit_tile_order if pending.tile_order else self.lib.hds_bin_emit
                self._run("bin_emit", lambda: emit(
                    n, total, width, height, _ptr(pending.workspace), _ptr(pws), pws.numel(), _ptr(values),
                    _ptr(pending.tile_ranges), _stream(dev)))
                status = torch.zeros(2, dtype=torch.int64, pin_memory=True)
                _check(self.lib.hds_bin_status(n, _ptr(pending.workspace), _ptr(status), _stream(dev)))
                torch.cuda.current_stream(dev).synchronize()
                overflow = _raise_on_sort_error(status)
            if overflow:
                self._tile_order_ok[dev.index] = False
                self._rebin_depth_order(pending, values, pws)
        pending.values = values
        return True

    def _rebin_depth_order(self, pending: PendingBins, values: torch.Tensor, pws: torch.Tensor) -> None:
        """Bins pending's frame again with the global depth sort, into `values` (exact P) and the
        pending tile_ranges, conic4 and color_opacity4."""
        n, width, height, dev = pending.emit_args
        means2D, depths, radii, conics, colors, opacities = pending.inputs
        ws = torch.empty(self.lib.hds_bin_workspace_bytes(n, width, height), device=dev, dtype=torch.uint8)
        total = ctypes.c_int64(0)
        self._run("bin_count", lambda: self.lib.hds_bin_count(
            n, _ptr(means2D), _ptr(depths), _ptr(radii), _ptr(conics), _ptr(colors), _ptr(opacities), width, height,
            _ptr(pending.conic4), _ptr(pending.color_opacity4), _ptr(ws), ws.numel(), ctypes.byref(total),
            _stream(dev)))
        if total.value != values.numel():
            raise RuntimeError(f"bin_count: {total.value} pairs on the rebin against {values.numel()} counted")
        self._run("bin_emit", lambda: self.lib.hds_bin_emit(
            n, total.value, width, height, _ptr(ws), _ptr(pws), pws.numel(), _ptr(values), _ptr(pending.tile_ranges),
            _stream(dev)))
        status = torch.zeros(2, dtype=torch.int64, pin_memory=True)
        _check(self.lib.hds_bin_status(n, _ptr(ws), _ptr(status), _stream(dev)))
        torch.cuda.current_stream(dev).synchronize()
        _raise_on_sort_error(status)

    def _remember_pairs(self, dev: torch.device, pairs: int) -> None:
        chunk = 4096
        self._pair_capacity[dev.index] = (int(pairs * self.PAIR_HEADROOM) + 2 * chunk) // chunk * chunk

    def render(self, means2D, conic4, color_opacity4, values_sorted, tile_ranges, width, height, background=None,
               features=None, rgb=True, clear=None):
        """One front-to-back tile walk (forward.cu:141-237 + features.cu:116-282). With `clear` (a float32
        tensor from gradient_buffers), the walk's work-groups also zero it (hds_render_clear).

        Returns (image [H,W,3] or None, feature_image [H,W,C] or None, final_T [H,W], n_contrib [H,W]).
        """
        dev = means2D.device
        width, height = int(width), int(height)
        means2D = _dev(means2D, "means2D")
        channels = 0
        if features is not None:
            features = _dev(features, "features")
            if features.dtype != torch.float32:
                raise RuntimeError("features must be a contiguous float32 CUDA tensor")
            channels = int(features.shape[1])
            if channels not in SUPPORTED_CHANNELS:
                raise RuntimeError(f"features must have 32, 64, 128, 256 or 512 channels, got {channels}")
        image = torch.empty((height, width, 3), device=dev, dtype=torch.float32) if rgb else None
        feature_image = (torch.empty((height, width, channels), device=dev, dtype=torch.float32)
                         if features is not None else None)
        final_T = torch.empty((height, width), device=dev, dtype=torch.float32)
        n_contrib = torch.empty((height, width), device=dev, dtype=torch.int32)
        if rgb and background is None:
            background = black_background(dev)
        args = (means2D.shape[0], width, height, channels, _ptr(tile_ranges), _ptr(values_sorted),
                values_sorted.numel(), _ptr(means2D), _ptr(conic4), _ptr(color_opacity4) if rgb else None,
                _ptr(background) if rgb else None, _ptr(features), _ptr(image), _ptr(final_T), _ptr(n_contrib),
                _ptr(feature_image))
        if clear is not None and not (clear.is_cuda and clear.is_contiguous() and clear.dtype == torch.float32
                                      and clear.device == dev):
            raise RuntimeError("clear must be a contiguous float32 tensor on the render's device")
        with torch.cuda.device(dev):
            if clear is None:
                self._run("render", lambda: self.lib.hds_render(*args, _stream(dev)))
            else:
                self._run("render", lambda: self.lib.hds_render_clear(*args, _ptr(clear), clear.numel(),
                                                                      _stream(dev)))
        return image, feature_image, final_T, n_contrib

    def render_backward(self, means2D, conic4, color_opacity4, values_sorted, tile_ranges, final_T, n_contrib,
                        width, height, grad_image=None, background=None, features=None, grad_feature_image=None,
                        slice_width=None, want_feature_grad=True, prezeroed=None):
        """The blend backward (backward.cu:7-164 + features.cu:350-542): geometry gradients from a
        back-to-front replay, feature gradients from a front-to-back replay beside it. `prezeroed` is the
        buffers of gradient_buffers, zeroed by earlier work on the current stream (render(clear=...)):
        the gradients are then added into those buffers instead of into buffers zeroed here.

        Returns (grad_means2D [N,2], grad_conics [N,3], grad_colors [N,3] or None, grad_opacities [N,1],
        grad_features [N,C] or None).
        """
        dev = means2D.device
        n = means2D.shape[0]
        channels = 0 if features is None else int(features.shape[1])
        if features is not None:
            features = _dev(features, "features")
            grad_feature_image = _dev(grad_feature_image, "grad_feature_image")
            slice_width = int(slice_width or default_slice_width(channels))
        if grad_image is not None:
            grad_image = _dev(grad_image, "grad_image")
            if background is None:
                background = black_background(dev)
        want_feat = features is not None and want_feature_grad
        if prezeroed is not None:
            g_means, g_conics, g_colors, g_opac, g_feat = prezeroed
            if grad_image is None:
                g_colors = None
            if not want_feat:
                g_feat = None
            elif g_feat.shape != (n, channels):
                raise RuntimeError(f"prezeroed grad_features {tuple(g_feat.shape)} != ({n}, {channels})")
            entry = self.lib.hds_render_backward_accumulate
        else:
            # hds_render_backward zeroes the outputs itself before its atomics add into them.
            f32 = dict(device=dev, dtype=torch.float32)
            g_means = torch.empty((n, 2), **f32)
            g_conics = torch.empty((n, 3), **f32)
            g_colors = torch.empty((n, 3), **f32) if grad_image is not None else None
            g_opac = torch.empty((n, 1), **f32)
            g_feat = torch.empty((n, channels), **f32) if want_feat else None
            entry = self.lib.hds_render_backward
        with torch.cuda.device(dev):
            self._run("render_backward", lambda: entry(
                n, int(width), int(height), channels, slice_width or 0, _ptr(tile_ranges), _ptr(values_sorted),
                values_sorted.numel(), _ptr(_dev(means2D, "means2D")), _ptr(conic4), _ptr(color_opacity4),
                _ptr(background), _ptr(final_T), _ptr(n_contrib), _ptr(grad_image), _ptr(features),
                _ptr(grad_feature_image), _ptr(g_means), _ptr(g_conics), _ptr(g_colors), _ptr(g_opac), _ptr(g_feat),
                _stream(dev)))
        return g_means, g_conics, g_colors, g_opac, g_feat

    # -- the reference extension's rasterize* entry points --------------------------------------

    def rasterize(self, means2D, depths, radii, conics, colors, opacities, background, image_width, image_height):
        """forward.cu:239-435: (image, final_T, n_contrib, values_sorted, tile_ranges, conic, color_opacity)."""
        values, ranges, conic4, color_opacity4 = self.bin(means2D, depths, radii, conics, colors, opacities,
                                                          image_width, image_height)
        image, _, final_T, n_contrib = self.render(means2D, conic4, color_opacity4, values, ranges, image_width,
                                                   image_height, _dev(background, "background"))
        return image, final_T, n_contrib, values, ranges, conic4, color_opacity4

    def rasterize_backward(self, grad_image, means2D, conic, color_opacity, values_sorted, tile_ranges,
                           final_transmittance, n_contrib, background, image_width, image_height):
        """backward.cu:166-226: (grad_means2D, grad_conics, grad_colors, grad_opacities)."""
        gm, gc, gcol, gop, _ = self.render_backward(means2D, conic, color_opacity, values_sorted, tile_ranges,
                                                    final_transmittance, n_contrib, image_width, image_height,
                                                    grad_image=grad_image, background=background)
        return gm, gc, gcol, gop

    def rasterize_features(self, features, means2D, conic, color_opacity, values_sorted, tile_ranges, image_width,
                           image_height):
        """features.cu:299-346: (feature_image, feature_T, feature_contrib)."""
        _, feature_image, final_T, n_contrib = self.render(means2D, conic, color_opacity, values_sorted,
                                                           tile_ranges, image_width, image_height,
                                                           features=features, rgb=False)
        return feature_image, final_T, n_contrib

    def rasterize_features_backward(self, grad_output, features, means2D, conic, color_opacity, values_sorted,
                                    tile_ranges, final_transmittance, n_contrib, image_width, image_height,
                                    slice_width):
        """features.cu:561-616: (grad_features, grad_means2D, grad_conics, grad_opacities)."""
        gm, gc, _, gop, gf = self.render_backward(means2D, conic, color_opacity, values_sorted, tile_ranges,
                                                  final_transmittance, n_contrib, image_width, image_height,
                                                  features=features, grad_feature_image=grad_output,
                                                  slice_width=slice_width)
        return gf, gm, gc, gop

    # -- densification statistics ----------------------------------------------------------------

    def densification_stats(self, grad_means2D, radii, width, height, max_radii2D, grad_accum, denom):
        """utils/gaussian.py:143-160, in place on max_radii2D [N], grad_accum [N, 1] and denom [N, 1]."""
        for t, name in ((max_radii2D, "max_radii2D"), (grad_accum, "means2D_grad_accum"), (denom, "denom")):
            if not (t.is_cuda and t.is_contiguous() and t.dtype == torch.float32):
                raise RuntimeError(f"{name} must be a contiguous float32 CUDA tensor (updated in place)")
        grad_means2D, radii = _dev(grad_means2D, "means2D_grad"), _dev(radii, "radii")
        n = radii.shape[0]
        if grad_means2D.shape != (n, 2) or max_radii2D.numel() != n or grad_accum.numel() != n or denom.numel() != n:
            raise RuntimeError("densification statistics need means2D_grad [N,2], radii [N] and [N] / [N,1] buffers")
        with torch.cuda.device(radii.device):
            self._run("densification_stats", lambda: self.lib.hds_densification_stats(
                n, _ptr(grad_means2D), _ptr(radii), int(width), int(height), _ptr(max_radii2D), _ptr(grad_accum),
                _ptr(denom), _stream(radii.device)))

    # -- SSIM -------------------------------------------------------------------------------------

    def ssim_forward(self, rendered, gt):
        """ssim.cu:116-148: (ssim_map, d_mu, d_aa, d_ab), each [H,W,3]."""
        rendered, gt = _dev(rendered, "rendered"), _dev(gt, "gt")
        if rendered.dim() != 3 or rendered.shape[2] != 3 or rendered.shape != gt.shape:
            raise RuntimeError("ssim inputs must both be [H, W, 3]")
        h, w = rendered.shape[0], rendered.shape[1]
        outs = [torch.empty_like(rendered) for _ in range(4)]
        with torch.cuda.device(rendered.device):
            self._run("ssim_forward", lambda: self.lib.hds_ssim_forward(h, w, _ptr(rendered), _ptr(gt), *[_ptr(o) for o in outs],
                                             _stream(rendered.device)))
        return tuple(outs)

    def ssim_backward(self, grad_mean, rendered, gt, d_mu, d_aa, d_ab):
        """ssim.cu:151-177: gradient with respect to rendered, [H,W,3]."""
        rendered, gt = _dev(rendered, "rendered"), _dev(gt, "gt")
        grad_mean = _dev(grad_mean.reshape(1).to(torch.float32), "grad_mean")
        grad = torch.empty_like(rendered)
        h, w = rendered.shape[0], rendered.shape[1]
        with torch.cuda.device(rendered.device):
            self._run("ssim_backward", lambda: self.lib.hds_ssim_backward(h, w, _ptr(grad_mean), _ptr(rendered), _ptr(gt), _ptr(_dev(d_mu, "d_mu")),
                                              _ptr(_dev(d_aa, "d_aa")), _ptr(_dev(d_ab, "d_ab")), _ptr(grad),
                                              _stream(rendered.device)))
        return grad


def default_slice_width(channels: int) -> int:
    """Channels per backward work-group when FEATURE_SLICE_WIDTH is None: the widest supported slice.
    Each slice replays the tile walk and issues its own geometry atomics, so fewer, wider slices win
    (measured on MI355X at C=128: 128 beats 64 and 32) while dL/dF still fits the registers of two
    waves per SIMD."""
    return min(channels, 128)


def pairs_upper_bound_bytes(num_pairs: int) -> int:
    """Bytes the pair workspace needs for num_pairs pairs, for capacity planning."""
    return int(load_library().hds_pairs_workspace_bytes(num_pairs, 1, 1)) if num_pairs else 0


def tile_count(width: int, height: int) -> int:
    return math.ceil(width / TILE) * math.ceil(height / TILE)
