"""ctypes binding of libmgauss.so (the C ABI in include/mgauss.h).

The reference binds its native code as a pybind11 torch extension
(metal_gauss/csrc/rasterize.mm:518-533) that takes torch tensors. Here the
native boundary is a plain C ABI over device pointers, and this module is the
only place that turns tensors into pointers: it checks device, dtype and
contiguity, passes ``data_ptr()`` and torch's current HIP stream, and maps a
non-zero status to ``RuntimeError`` carrying the library's own message.

There is no fallback: if the library is missing or does not load, every entry
point raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libmgauss.so"

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_u64 = ctypes.c_uint64
_pp = ctypes.POINTER(ctypes.c_void_p)

_SIGNATURES = {
    "mg_last_error": (ctypes.c_char_p, []),
    "mg_version": (_i32, []),
    "mg_init": (_i32, []),
    "mg_max_tile": (_i32, []),
    "mg_timing_enable": (_i32, [_i32]),
    "mg_timing_reset": (_i32, []),
    "mg_timing_query": (_i32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(_i64)]),
    "mg_stream_copy": (_i32, [_vp, _vp, _i64, _vp]),
    "mg_preprocess_forward": (_i32, [
        _i64, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _f32, _f32, _f32, _i32, _i32,
        _f32, _f32, _f32, _f32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mg_preprocess_backward": (_i32, [
        _i64, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _f32, _f32,
        _f32, _i32, _i32, _f32, _f32, _f32, _f32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mg_preprocess_forward_mip": (_i32, [
        _i64, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _f32, _f32, _f32, _i32, _i32,
        _f32, _f32, _f32, _f32, _vp, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
        _vp, _i32, _vp, _vp]),
    "mg_preprocess_backward_mip": (_i32, [
        _i64, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _f32, _f32, _f32,
        _f32, _i32, _i32, _f32, _f32, _f32, _f32, _vp, _i32, _vp, _vp, _i32, _i32, _f32, _f32,
        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mg_compute_3d_filter": (_i32, [_i64, _vp, _i32, _vp, _f32, _f32, _vp, _vp, _vp]),
    "mg_add_noise": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _f32, _f32, _f32, _u64, _vp]),
    "mg_mcmc_workspace_bytes": (_i64, [_i64, _i64]),
    "mg_mcmc_weights": (_i32, [_i64, _vp, _vp, _f32, _i32, _vp, _i64, _i64,
                               ctypes.POINTER(_f64), _vp]),
    "mg_mcmc_apply": (_i32, [_i64, _vp, _vp, _f32, _i32, _i32, _vp, _i64, _i64, _i64, _i64,
                             _u64, _i32, _pp, ctypes.POINTER(_i32), ctypes.POINTER(_i32), _vp]),
    "mg_ply_decode": (_i32, [_i64, _vp, _i32, ctypes.POINTER(_i32), _i32, _vp, _vp, _vp, _vp,
                             _vp, _vp]),
    "mg_ply_encode": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32,
                             ctypes.POINTER(_i32), _i32, _vp, _vp]),
    "mg_bin_count": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp,
                            _vp]),
    "mg_scan_workspace_bytes": (_i64, [_i64]),
    "mg_exclusive_scan_i32": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp]),
    "mg_bin_write": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32,
                            _i32, _i32, _vp, _vp, _vp]),
    "mg_sort_workspace_bytes": (_i64, [_i64]),
    "mg_sort_pairs_u64": (_i32, [_vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp, _i64, _vp]),
    "mg_tile_ranges": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "mg_sort_pairs_by_tile_workspace_bytes": (_i64, [_i64, _i32]),
    "mg_sort_pairs_by_tile": (_i32, [_i64, _vp, _vp, _i32, _vp, _vp, _vp, _i64, _vp]),
    "mg_bin_lists_workspace_bytes": (_i64, [_i64]),
    "mg_bin_lists_finish_workspace_bytes": (_i64, [_i64]),
    "mg_bin_lists_begin": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                  _i32, _vp, _i64, _vp, _vp]),
    "mg_bin_lists_finish": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                   _i32, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "mg_bin_lists_capped_workspace_bytes": (_i64, [_i64, _i64]),
    "mg_bin_lists_capped": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                   _i32, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _vp,
                                   _vp]),
    "mg_rasterize_chunk_workspace_bytes": (_i64, [_i64, _i32, _i32]),
    "mg_rasterize_sched_ints": (_i64, [_i32, _i32, _i32]),
    "mg_rasterize_forward": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                    _f32, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _vp]),
    "mg_rasterize_backward": (_i32, [_i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _i32,
                                     _i32, _vp, _vp]),
    "mg_adam_step": (_i32, [_vp, _vp, _vp, _vp, _i64, _f64, _f64, _f64, _f64, _i64, _vp]),
    "mg_adam_step_multi": (_i32, [_i32, _pp, _pp, _pp, _pp, ctypes.POINTER(_i64),
                                  ctypes.POINTER(_f64), ctypes.POINTER(_i64), _f64, _f64, _f64,
                                  _i32, _vp]),
    "mg_adam_step_multi_guarded": (_i32, [_i32, _pp, _pp, _pp, _pp, ctypes.POINTER(_i64),
                                          ctypes.POINTER(_f64), ctypes.POINTER(_i64), _f64, _f64,
                                          _f64, _i32, _vp, _vp]),
    "mg_selective_adam_step": (_i32, [_i32, _pp, _pp, _pp, _pp, _pp, ctypes.POINTER(_i64),
                                      ctypes.POINTER(_i32), ctypes.POINTER(_f32), _vp, _i64,
                                      _f64, _f64, _f64, _vp]),
    "mg_selective_adam_step_guarded": (_i32, [_i32, _pp, _pp, _pp, _pp, _pp,
                                              ctypes.POINTER(_i64), ctypes.POINTER(_i32),
                                              ctypes.POINTER(_f32), _vp, _i64, _f64, _f64,
                                              _f64, _vp, _vp]),
    "mg_ssim_stack_blur_h": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "mg_ssim_blur15": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "mg_ssim_tail_forward": (_i32, [_vp, _i32, _i32, _vp, _vp]),
    "mg_ssim_tail_backward": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "mg_ssim_chain_backward": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "mg_ssim_fused_workspace_bytes": (_i64, [_i32, _i32]),
    "mg_ssim_fused_forward": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _vp]),
    "mg_ssim_fused_backward": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "mg_photometric_loss_forward": (_i32, [_vp, _vp, _vp, _i32, _i32, _f32, _vp, _vp, _vp, _i64,
                                           _vp]),
    "mg_photometric_loss_forward_noalloc": (_i32, [_vp, _vp, _vp, _i32, _i32, _f32, _vp, _vp,
                                                   _vp]),
    "mg_photometric_loss_backward": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp,
                                            _vp]),
}

EXPORTS = tuple(_SIGNATURES)

_lib = None
_initialised = False


def open_library():
    """Load libmgauss.so and declare every signature. Needs no GPU."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"hip backend not built: {LIB_PATH} is missing. Build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (or "
            "metal-gauss_amd/build.py). Refusing to silently substitute a different renderer.")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def load():
    """The library, initialised on the current HIP device (mg_init)."""
    global _initialised
    lib = open_library()
    if not _initialised:
        check(lib.mg_init())
        _initialised = True
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = open_library().mg_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"libmgauss call failed with status {rc}")


def stream(t: torch.Tensor | None = None) -> int:
    dev = t.device if t is not None else None
    return torch.cuda.current_stream(dev).cuda_stream


def dev_tensor(t: torch.Tensor, what: str, dtype: torch.dtype | None = torch.float32) -> int:
    """Pointer of a contiguous GPU tensor, with the reference's error wording."""
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} must be a HIP (ROCm) tensor, got device '{t.device}'")
    if not t.is_contiguous():
        raise RuntimeError(f"{what} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{what} must be {dtype}, got {t.dtype}")
    return t.data_ptr()


class AdamEpilogue(ctypes.Structure):
    """mg_adam_epilogue (include/mgauss.h): the preprocess backward's
    optimizer epilogue over means, quats, scales, opacities, sh, sh_rest."""
    _fields_ = [("p", _vp * 6), ("m", _vp * 6), ("v", _vp * 6), ("lr", _f64 * 6),
                ("step", _i64 * 6), ("beta1", _f64), ("beta2", _f64), ("eps", _f64),
                ("skip", _vp)]


def ptr_array(ptrs):
    return (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)


def i64_array(xs):
    return (_i64 * max(1, len(xs)))(*xs)


def i32_array(xs):
    return (_i32 * max(1, len(xs)))(*xs)


def f32_array(xs):
    return (_f32 * max(1, len(xs)))(*xs)


def f64_array(xs):
    return (_f64 * max(1, len(xs)))(*xs)


def host_f32(t: torch.Tensor) -> ctypes.Array:
    """A small host tensor (pose, camera centre) as a C float array."""
    vals = t.detach().to("cpu", torch.float32).contiguous().reshape(-1).tolist()
    return (_f32 * len(vals))(*vals)


class KernelTimer:
    """Per-kernel HIP-event timing inside the library (mg_timing_*)."""

    def __enter__(self):
        lib = load()
        check(lib.mg_timing_reset())
        check(lib.mg_timing_enable(1))
        return self

    def __exit__(self, *exc):
        check(load().mg_timing_enable(0))
        return False

    @staticmethod
    def query(kernel: str) -> tuple[float, int]:
        ms = ctypes.c_double(0.0)
        n = _i64(0)
        check(load().mg_timing_query(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value
