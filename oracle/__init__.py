"""numpy front end of the CPU oracle (oracle/hds_oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package, and only
as the checker. The product path (high-dimensional-splatting_amd/) never imports it and has no CPU
fallback.

Every function takes and returns float32 / int32 numpy arrays in the reference's layouts:
means2D [N, 2], conics [N, 3], colors [N, 3], opacities [N] or [N, 1], images [H, W, 3],
feature images [H, W, C], tile_ranges [T, 2]. The C side cites the reference file:line of each
stage it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "_build" / "libhds_oracle.so"
_lib: ctypes.CDLL | None = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build(force: bool = False) -> Path:
    """Compiles the oracle with its Makefile (gcc + OpenMP) and returns the library path."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(lib: ctypes.CDLL) -> None:
    i64, i32, f32, f64, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_void_p
    lib.orc_logf.argtypes = [f32]
    lib.orc_logf.restype = f32
    lib.orc_exp2f.argtypes = [i64, vp, vp]
    lib.orc_exp2f.restype = None
    lib.orc_tile_rect.argtypes = [f32] * 6 + [i32, i32, vp]
    lib.orc_tile_rect.restype = i32
    cam = [f32, f32, f32, f32, i32, i32, f32, f32, f32]
    lib.orc_project_forward.argtypes = [i64, vp, vp, vp, vp, vp] + cam + [vp, vp, vp, vp]
    lib.orc_project_forward.restype = None
    lib.orc_project_backward.argtypes = [i64, vp, vp, vp, vp, vp, vp] + cam + [vp, vp, vp]
    lib.orc_project_backward.restype = None
    lib.orc_eval_sh.argtypes = [i64, i32, vp, vp, vp, vp, vp]
    lib.orc_eval_sh.restype = None
    lib.orc_eval_sh_backward_adam.argtypes = [i64, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                              f64, f64, f64, f64, f64, vp]
    lib.orc_eval_sh_backward_adam.restype = None
    lib.orc_bin_count.argtypes = [i64, vp, vp, vp, vp, i32, i32, vp, vp]
    lib.orc_bin_count.restype = i64
    lib.orc_bin_fill.argtypes = [i64, vp, vp, vp, i32, i32, i64, vp, vp, vp]
    lib.orc_bin_fill.restype = None
    lib.orc_bin_count_masked.argtypes = [i64, vp, vp, i32]
    lib.orc_bin_count_masked.restype = i64
    lib.orc_render_forward.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, i32, vp, vp, vp, vp, vp]
    lib.orc_render_forward.restype = None
    lib.orc_render_backward.argtypes = [i32, i32, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                        vp, i32, vp, vp, vp, vp, vp]
    lib.orc_render_backward.restype = None
    lib.orc_ssim_forward.argtypes = [i32, i32, vp, vp, vp, vp, vp, vp]
    lib.orc_ssim_forward.restype = None
    lib.orc_ssim_backward.argtypes = [i32, i32, f32, vp, vp, vp, vp, vp, vp]
    lib.orc_ssim_backward.restype = None


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def num_threads() -> int:
    """OpenMP threads the oracle runs on (OMP_NUM_THREADS if set, else every host core)."""
    env = os.environ.get("OMP_NUM_THREADS")
    return int(env) if env else os.cpu_count() or 1


def logf(x: float) -> float:
    """hds_logf, the shared float32 natural log used by the tile rectangle on both CPU and GPU."""
    return float(_load().orc_logf(float(x)))


def exp2f(x: np.ndarray) -> np.ndarray:
    """hds_exp2f elementwise: the shared float32 2^x behind every blend alpha on CPU and GPU."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    _load().orc_exp2f(x.size, x.ctypes.data, y.ctypes.data)
    return y


def tile_rect(ux, uy, a, b, c, opacity, tiles_x, tiles_y):
    """(x0, y0, w, h) of the tiles a gaussian can touch, or None when culled (common.cuh:55-65)."""
    out = np.zeros(4, dtype=np.int32)
    ok = _load().orc_tile_rect(ux, uy, a, b, c, opacity, tiles_x, tiles_y, _p(out))
    return tuple(int(v) for v in out) if ok else None


def project_forward(means, scales, quats, opacities, world_to_camera, fx, fy, cx, cy, width, height,
                    near_plane=0.2, low_pass=0.3, fov_scale=1.3):
    """project_gaussians forward (projection.cu:80-111): means2D, depths, radii, conics."""
    means, scales, quats = _f32(means), _f32(scales), _f32(quats)
    opacities, w2c = _f32(opacities).reshape(-1), _f32(world_to_camera).reshape(16)
    n = means.shape[0]
    means2D = np.empty((n, 2), np.float32)
    depths = np.empty(n, np.float32)
    radii = np.empty(n, np.float32)
    conics = np.empty((n, 3), np.float32)
    _load().orc_project_forward(n, _p(means), _p(scales), _p(quats), _p(opacities), _p(w2c), fx, fy, cx, cy,
                                width, height, near_plane, low_pass, fov_scale, _p(means2D), _p(depths),
                                _p(radii), _p(conics))
    return means2D, depths, radii, conics


def project_backward(grad_means2D, grad_conics, means, scales, quats, world_to_camera, fx, fy, cx, cy,
                     width, height, near_plane=0.2, low_pass=0.3, fov_scale=1.3):
    """project_gaussians backward (projection.cu:114-197): grads of means, scales, quats."""
    gm, gc = _f32(grad_means2D), _f32(grad_conics)
    means, scales, quats, w2c = _f32(means), _f32(scales), _f32(quats), _f32(world_to_camera).reshape(16)
    n = means.shape[0]
    dm, ds, dq = np.empty((n, 3), np.float32), np.empty((n, 3), np.float32), np.empty((n, 4), np.float32)
    _load().orc_project_backward(n, _p(gm), _p(gc), _p(means), _p(scales), _p(quats), _p(w2c), fx, fy, cx, cy,
                                 width, height, near_plane, low_pass, fov_scale, _p(dm), _p(ds), _p(dq))
    return dm, ds, dq


def eval_sh(sh_dc, sh_rest, dirs, degree, radii):
    """eval_sh forward (sh.cu:62-83): [N, 3] rgb."""
    sh_dc, sh_rest, dirs, radii = _f32(sh_dc), _f32(sh_rest), _f32(dirs), _f32(radii)
    n = dirs.shape[0]
    rgb = np.empty((n, 3), np.float32)
    _load().orc_eval_sh(n, degree, _p(sh_dc), _p(sh_rest), _p(dirs), _p(radii), _p(rgb))
    return rgb


def eval_sh_backward_adam(grad_rgb, sh_dc, sh_rest, dirs, degree, radii, m_dc, v_dc, m_rest, v_rest,
                          step_dc, step_rest, lr_dc, lr_rest, beta1, beta2, eps):
    """eval_sh_backward_adam (sh.cu:104-154): returns grad_dirs; steps sh/m/v arrays IN PLACE."""
    for a in (sh_dc, sh_rest, m_dc, v_dc, m_rest, v_rest):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    grad_rgb, dirs, radii = _f32(grad_rgb), _f32(dirs), _f32(radii)
    n = dirs.shape[0]
    grad_dirs = np.empty((n, 3), np.float32)
    _load().orc_eval_sh_backward_adam(n, degree, _p(grad_rgb), _p(sh_dc), _p(sh_rest), _p(dirs), _p(radii),
                                      _p(m_dc), _p(v_dc), _p(m_rest), _p(v_rest), float(step_dc),
                                      float(step_rest), lr_dc, lr_rest, beta1, beta2, eps, _p(grad_dirs))
    return grad_dirs


def tile_counts(means2D, radii, conics, opacities, width, height):
    """Per-gaussian tile count and tile rectangle (x0, y0, w, h) of rasterize's binning
    (forward.cu:13-61), without the pair list. Returns (counts [N] int32, rects [N, 4] int32)."""
    means2D, radii, conics = _f32(means2D), _f32(radii), _f32(conics)
    opacities = _f32(opacities).reshape(-1)
    n = means2D.shape[0]
    counts = np.zeros(n, np.int32)
    rects = np.zeros((n, 4), np.int32)
    _load().orc_bin_count(n, _p(means2D), _p(radii), _p(conics), _p(opacities), width, height, _p(counts),
                          _p(rects))
    return counts, rects


def bin_gaussians(means2D, depths, radii, conics, opacities, width, height, tile_mask=None):
    """Binning of rasterize (forward.cu:13-139).

    Returns (counts [N] int32, values_sorted [P] int32, tile_ranges [T, 2] int32).

    tile_mask ([T] bool, optional) keeps only the pairs of the selected tiles: their lists equal
    the full binning's lists for those tiles, every other tile is empty, and values_sorted holds
    only the selected tiles' pairs. counts stay the full per-gaussian tile counts.
    """
    means2D, depths, radii, conics = _f32(means2D), _f32(depths), _f32(radii), _f32(conics)
    opacities = _f32(opacities).reshape(-1)
    n = means2D.shape[0]
    tiles = ((width + 15) // 16) * ((height + 15) // 16)
    counts = np.zeros(n, np.int32)
    rects = np.zeros((n, 4), np.int32)
    lib = _load()
    total = lib.orc_bin_count(n, _p(means2D), _p(radii), _p(conics), _p(opacities), width, height,
                              _p(counts), _p(rects))
    mask = None
    if tile_mask is not None:
        mask = np.ascontiguousarray(np.asarray(tile_mask, dtype=np.uint8).reshape(-1))
        assert mask.size == tiles, (mask.size, tiles)
        total = lib.orc_bin_count_masked(n, _p(rects), _p(mask), width)
    values = np.empty(total, np.int32)
    ranges = np.zeros((tiles, 2), np.int32)
    lib.orc_bin_fill(n, _p(depths), _p(counts), _p(rects), width, height, total, _p(mask), _p(values),
                     _p(ranges))
    return counts, values, ranges


def render_forward(width, height, tile_ranges, values_sorted, means2D, conics, opacities, colors=None,
                   background=None, features=None, near_cut=False):
    """Front-to-back blend (forward.cu:141-237, features.cu:116-282).

    Returns (image [H, W, 3] or None, final_T [H, W], n_contrib [H, W], feature_image [H, W, C] or None),
    and with near_cut=True also a [H, W] bool mask of the pixels whose walk passed an alpha or a
    transmittance within twice its propagated rounding uncertainty of the 1/255 or 1e-4 cut:
    the decisions that an implementation with other rounding (another exp, other fused
    multiply-adds) could flip. The HIP kernels share this oracle's alpha arithmetic
    (hds_gauss_alpha) and take every decision identically on identical inputs.
    """
    ranges, values = _i32(tile_ranges), _i32(values_sorted)
    means2D, conics, opacities = _f32(means2D), _f32(conics), _f32(opacities).reshape(-1)
    colors = None if colors is None else _f32(colors)
    bg = _f32(background if background is not None else np.zeros(3))
    feats = None if features is None else _f32(features)
    channels = 0 if feats is None else feats.shape[1]
    image = np.empty((height, width, 3), np.float32) if colors is not None else None
    final_T = np.empty((height, width), np.float32)
    n_contrib = np.empty((height, width), np.int32)
    fimg = np.empty((height, width, channels), np.float32) if feats is not None else None
    near = np.zeros((height, width), np.uint8) if near_cut else None
    _load().orc_render_forward(width, height, _p(ranges), _p(values), _p(means2D), _p(conics), _p(opacities),
                               _p(colors), _p(bg), _p(feats), channels, _p(image), _p(final_T), _p(n_contrib),
                               _p(fimg), _p(near))
    if near_cut:
        return image, final_T, n_contrib, fimg, near.astype(bool)
    return image, final_T, n_contrib, fimg


def render_backward(width, height, tile_ranges, values_sorted, means2D, conics, opacities, colors, background,
                    final_T, n_contrib, grad_image=None, features=None, grad_feature_image=None):
    """Back-to-front replay (backward.cu:7-164 + features.cu:350-542).

    Returns grads (means2D [N, 2], conics [N, 3], colors [N, 3], opacities [N, 1], features [N, C] or None).
    """
    ranges, values = _i32(tile_ranges), _i32(values_sorted)
    means2D, conics, opacities = _f32(means2D), _f32(conics), _f32(opacities).reshape(-1)
    n = means2D.shape[0]
    colors = _f32(colors if colors is not None else np.zeros((n, 3)))
    bg = _f32(background if background is not None else np.zeros(3))
    final_T, n_contrib = _f32(final_T), _i32(n_contrib)
    gimg = None if grad_image is None else _f32(grad_image)
    feats = None if features is None else _f32(features)
    gfeat = None if feats is None else _f32(grad_feature_image)
    channels = 0 if feats is None else feats.shape[1]
    dm, dc = np.zeros((n, 2), np.float32), np.zeros((n, 3), np.float32)
    dcol, dop = np.zeros((n, 3), np.float32), np.zeros((n, 1), np.float32)
    dfeat = np.zeros((n, channels), np.float32) if feats is not None else None
    _load().orc_render_backward(width, height, n, values.shape[0], _p(ranges), _p(values), _p(means2D),
                                _p(conics), _p(opacities), _p(colors), _p(bg), _p(final_T), _p(n_contrib),
                                _p(gimg), _p(feats), _p(gfeat), channels, _p(dm), _p(dc), _p(dcol), _p(dop),
                                _p(dfeat))
    return dm, dc, dcol, dop, dfeat


def rasterize(means2D, depths, radii, conics, colors, opacities, width, height, background=None, features=None):
    """Binning + blend in one call: (image, feature_image or None, final_T, n_contrib, values, ranges)."""
    counts, values, ranges = bin_gaussians(means2D, depths, radii, conics, opacities, width, height)
    image, final_T, n_contrib, fimg = render_forward(width, height, ranges, values, means2D, conics, opacities,
                                                     colors, background, features)
    return image, fimg, final_T, n_contrib, values, ranges


def ssim_forward(rendered, gt):
    """ssim_forward (ssim.cu:116-148): (ssim_map, d_mu, d_aa, d_ab), each [H, W, 3]."""
    a, b = _f32(rendered), _f32(gt)
    h, w, _ = a.shape
    outs = [np.empty_like(a) for _ in range(4)]
    _load().orc_ssim_forward(h, w, _p(a), _p(b), *[_p(o) for o in outs])
    return tuple(outs)


def ssim_backward(grad_mean, rendered, gt, d_mu, d_aa, d_ab):
    """ssim_backward (ssim.cu:151-177): gradient of the mean SSIM times grad_mean, [H, W, 3]."""
    a, b = _f32(rendered), _f32(gt)
    h, w, _ = a.shape
    grad = np.empty_like(a)
    _load().orc_ssim_backward(h, w, float(grad_mean), _p(a), _p(b), _p(_f32(d_mu)), _p(_f32(d_aa)),
                              _p(_f32(d_ab)), _p(grad))
    return grad
