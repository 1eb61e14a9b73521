"""ctypes wrapper of raster_seq.c (the rasteriser's per-pixel contract).
TEST INFRASTRUCTURE ONLY. See raster_seq.c for what it restates and how it is
pinned. Arrays are numpy; tile lists come from binning_ref or the GPU."""

from __future__ import annotations

import ctypes

import numpy as np

from . import build as _build

_lib = None


def _load():
    global _lib
    if _lib is None:
        if not _build.OUT.exists():
            _build.build()
        _lib = ctypes.CDLL(str(_build.OUT))
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def forward(uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, t_min=1e-4):
    """-> (rgb (H,W,3), alpha (H,W), T (H,W), stop (H,W) int32, ambiguous (H,W) bool)."""
    lib = _load()
    uv, conic, opacity, color = _f32(uv), _f32(conic), _f32(opacity), _f32(color)
    ids, offs = _i32(gauss_ids), _i32(tile_offsets)
    tiles_x = -(-W // tile)
    rgb = np.zeros((H, W, 3), np.float32)
    alpha = np.zeros((H, W), np.float32)
    T = np.zeros((H, W), np.float32)
    stop = np.zeros((H, W), np.int32)
    amb = np.zeros((H, W), np.uint8)
    f = lib.raster_seq_forward
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int64] + [ctypes.c_void_p] * 6 + [ctypes.c_int32] * 4 + \
        [ctypes.c_float] + [ctypes.c_void_p] * 5
    rc = f(uv.shape[0], _p(uv), _p(conic), _p(opacity), _p(color), _p(ids), _p(offs), W, H, tile,
           tiles_x, float(t_min), _p(rgb), _p(alpha), _p(T), _p(stop), _p(amb))
    if rc:
        raise RuntimeError(f"raster_seq_forward failed ({rc})")
    return rgb, alpha, T, stop, amb.astype(bool)


def backward(uv, conic, opacity, color, gauss_ids, tile_offsets, final_T, stop, grad_rgb,
             grad_alpha, W, H, tile):
    """-> (d_uv, d_conic, d_opacity, d_color, d_absuv)."""
    lib = _load()
    uv, conic, opacity, color = _f32(uv), _f32(conic), _f32(opacity), _f32(color)
    ids, offs = _i32(gauss_ids), _i32(tile_offsets)
    final_T, stop = _f32(final_T), _i32(stop)
    grad_rgb, grad_alpha = _f32(grad_rgb), _f32(grad_alpha)
    N = uv.shape[0]
    tiles_x = -(-W // tile)
    d_uv = np.zeros((N, 2), np.float32)
    d_conic = np.zeros((N, 3), np.float32)
    d_op = np.zeros(N, np.float32)
    d_col = np.zeros((N, 3), np.float32)
    d_abs = np.zeros(N, np.float32)
    f = lib.raster_seq_backward
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int64] + [ctypes.c_void_p] * 10 + [ctypes.c_int32] * 4 + \
        [ctypes.c_void_p] * 5
    rc = f(N, _p(uv), _p(conic), _p(opacity), _p(color), _p(ids), _p(offs), _p(final_T),
           _p(stop), _p(grad_rgb), _p(grad_alpha), W, H, tile, tiles_x, _p(d_uv), _p(d_conic),
           _p(d_op), _p(d_col), _p(d_abs))
    if rc:
        raise RuntimeError(f"raster_seq_backward failed ({rc})")
    return d_uv, d_conic, d_op, d_col, d_abs
