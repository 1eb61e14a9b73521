"""HIP backend: the reference's ``metal_backend`` operator surface on gfx950.

Same functions, argument meaning and error behaviour as
metal_gauss/metal_backend.py, so a caller of the reference's surface can switch
to this module:

* ``render`` (metal_backend.py:396-559) - projection + SH, binning, raster,
  background blend; returns (rgb (H,W,3), alpha (H,W), info);
* ``build_tile_lists`` (metal_backend.py:111-214) and
  ``build_tile_lists_metal`` (metal_backend.py:217-285) - tile lists, here both
  on the GPU: count, scan, pair emission and the stable tile and depth sorts
  are HIP kernels (the reference keeps argsort/cumsum/searchsorted in torch);
* ``_PreprocessMetal`` / ``_RasterizeMetal`` (metal_backend.py:288-364) - the
  autograd bridges, under the same names;
* ``antialias_scale`` (metal_backend.py:367-393), ``_load`` (76-108) and
  ``stale_lock_message`` (37-61).

What changes is underneath: every heavy step is a hand-written HIP kernel in
libmgauss.so (include/mgauss.h) reached through ``_lib``. Torch is used only
for allocation, the stream, autograd plumbing and the small elementwise glue
the reference also leaves in torch (SH zero-padding, a background given as a
device tensor). The antialias compensation and Mip-Splatting's 3D filter,
which the reference computes in torch, run inside the projection kernel
(``_PreprocessMip``); ``antialias_scale`` is kept for callers that use it
directly.
"""

from __future__ import annotations

import ctypes
import math
import time
import warnings
import weakref
from pathlib import Path

import numpy as np
import torch

from . import _lib

_HERE = Path(__file__).resolve().parent

# Longer than any build of the library takes; past it, a lock is a leftover.
_STALE_LOCK_S = 180.0

# The per-pixel stop transmittance of the reference kernel (rasterize.metal:149).
DEFAULT_T_MIN = 1e-4


def stale_lock_message(build_dir, now: float | None = None) -> str | None:
    """What to say about a lock left in the library's build directory.

    The ahead-of-time build (build.py) holds ``<build_dir>/lock`` while it
    compiles. Nothing is deleted here: two processes may build at once. Same
    contract as metal_backend.py:37-61.
    """
    try:
        lock = Path(build_dir) / "lock"
        age = (now if now is not None else time.time()) - lock.stat().st_mtime
    except OSError:
        return None
    where = f"waiting for the kernel build lock at {lock} ({age:.0f}s old)"
    if age < _STALE_LOCK_S:
        return f"{where}; another process is probably compiling."
    return (f"{where}. A build takes under a minute, so this one is stale -- left by an "
            f"interrupted build. Delete it to carry on:\n    rm {lock}")


def _load():
    """The native extension, loaded and initialised (metal_backend.py:76-108).

    Returns the module of the reference's thirteen tensor-level functions
    (``metal_gauss_amd.ext``: rasterize_forward/backward, preprocess_forward/
    backward, bin_count, bin_write, adam_step, the five SSIM kernels, init)
    over libmgauss.so. The reference compiles Metal source at first use;
    libmgauss.so is built ahead of time, so this only loads it. Raises if it
    is missing.
    """
    from . import ext

    _lib.load()
    return ext


def _require_gpu(t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"hip backend requires ROCm (cuda) tensors, got device '{t.device}'. "
            "Refusing to silently move data or fall back to another backend.")


def _tile_grid(W: int, H: int, tile: int) -> tuple[int, int]:
    return math.ceil(W / tile), math.ceil(H / tile)


_pinned_total = None


def _host_total() -> torch.Tensor:
    global _pinned_total
    if _pinned_total is None:
        _pinned_total = torch.zeros(1, dtype=torch.int64, pin_memory=True)
    return _pinned_total


def _empty_lists(n_tiles: int, tx: int, device):
    return (torch.zeros(0, dtype=torch.int32, device=device),
            torch.zeros(n_tiles + 1, dtype=torch.int32, device=device), tx)


def _bin(uv, rxy, depth, valid_i, conic, opacity, W, H, tile):
    """Tile lists on the GPU (mg_bin_lists_begin / _finish).

    Per-Gaussian counts with the exact ellipse test and their scan, then the
    (tile, Gaussian) pairs emitted in Gaussian order, a stable counting sort
    of the pairs by tile (radix passes past 4096 tiles) and a stable sort of
    every tile's list by depth: the order of a stable sort of the
    (tile << 32 | depth bits) keys. Returns (gauss_ids, tile_offsets,
    tiles_x). One device->host read per call: the intersection total that
    sizes the pair buffers (the reference's .item(), metal_backend.py:247-248).
    """
    lib = _lib.load()
    device = uv.device
    tx, ty = _tile_grid(W, H, tile)
    n_tiles = tx * ty
    N = uv.shape[0]
    if N == 0:
        return _empty_lists(n_tiles, tx, device)
    s = _lib.stream(uv)
    ptrs = (N, _lib.dev_tensor(uv, "uv"), _lib.dev_tensor(rxy, "rxy"),
            _lib.dev_tensor(conic, "conic") if conic is not None else None,
            _lib.dev_tensor(opacity, "opacity") if opacity is not None else None,
            _lib.dev_tensor(valid_i, "valid", torch.int32), _lib.dev_tensor(depth, "depth"),
            W, H, tile, tx, ty)
    ws = torch.empty(lib.mg_bin_lists_workspace_bytes(N), dtype=torch.uint8, device=device)
    host = _host_total()
    _lib.check(lib.mg_bin_lists_begin(*ptrs, ws.data_ptr(), ws.numel(), host.data_ptr(), s))
    total = int(host[0])
    if total >= 2 ** 31:
        raise RuntimeError(f"{total} tile intersections exceed the int32 index range")
    gauss_ids = torch.empty(total, dtype=torch.int32, device=device)
    tile_offsets = torch.empty(n_tiles + 1, dtype=torch.int32, device=device)
    fws = torch.empty(lib.mg_bin_lists_finish_workspace_bytes(total), dtype=torch.uint8,
                      device=device)
    _lib.check(lib.mg_bin_lists_finish(*ptrs, ws.data_ptr(), ws.numel(), total,
                                       gauss_ids.data_ptr() if total else None,
                                       tile_offsets.data_ptr(), fws.data_ptr(), fws.numel(), s))
    return gauss_ids, tile_offsets, tx


# Tile count past which render orders the capacity lists' binning blocks by
# their estimated work: below it the heavy blocks are not long enough to
# trail the count and write passes.
_BLOCK_ORDER_TILES = 4096


def _bin_capped(uv, rxy, depth, valid_i, conic, opacity, W, H, tile, capacity,
                host_slot=None, tag=0, block_work=None):
    """The lists of ``_bin`` with no host read (mg_bin_lists_capped): ids in a
    (capacity,) buffer, and a device int64 (2,) status = (intersection
    total, 1 if it exceeded ``capacity`` else 0). After an overflow every
    list is empty. ``host_slot`` (an address of 3 int64 of pinned host
    memory) also receives the two words and then ``tag``. ``block_work``
    (int32, one per 256 Gaussians, or None) orders the passes' blocks
    heaviest first; it does not change the lists. Returns
    (gauss_ids, tile_offsets, tiles_x, status)."""
    lib = _lib.load()
    device = uv.device
    tx, ty = _tile_grid(W, H, tile)
    N = uv.shape[0]
    capacity = int(capacity)
    if capacity < 0 or capacity >= 2 ** 31:
        raise ValueError(f"list capacity {capacity} outside [0, 2^31)")
    s = _lib.stream(uv)
    gauss_ids = torch.empty(capacity, dtype=torch.int32, device=device)
    tile_offsets = torch.empty(tx * ty + 1, dtype=torch.int32, device=device)
    status = torch.empty(2, dtype=torch.int64, device=device)
    ws = torch.empty(lib.mg_bin_lists_capped_workspace_bytes(N, capacity), dtype=torch.uint8,
                     device=device)
    _lib.check(lib.mg_bin_lists_capped(
        N, _lib.dev_tensor(uv, "uv"), _lib.dev_tensor(rxy, "rxy"),
        _lib.dev_tensor(conic, "conic") if conic is not None else None,
        _lib.dev_tensor(opacity, "opacity") if opacity is not None else None,
        _lib.dev_tensor(valid_i, "valid", torch.int32), _lib.dev_tensor(depth, "depth"),
        W, H, tile, tx, ty, capacity, gauss_ids.data_ptr() if capacity else None,
        tile_offsets.data_ptr(), status.data_ptr(), host_slot, int(tag), ws.data_ptr(),
        ws.numel(),
        None if block_work is None else _lib.dev_tensor(block_work, "block_work", torch.int32),
        s))
    return gauss_ids, tile_offsets, tx, status


class ListCapacity:
    """Sizes a render's tile lists without a host read in the render.

    Pass the object itself as ``render(..., list_capacity=cap)``: the lists
    are built in buffers of ``cap.value`` intersections, and the kernel that
    forms the intersection total also writes it, with an overflow word and a
    ticket's tag, into a pinned host slot of this object, so no copy or
    event joins the stream. ``cap.overflowed(ticket)`` (default: the latest
    render) polls that slot and, on overflow, raises ``value`` to
    ``headroom`` times the total seen, for that render to be run again. An
    overflowed render has empty lists (a background image), and optimizer
    steps given its ``info["lists_status"]`` as ``skip`` leave every
    parameter as it was. With an int capacity instead, ``watch(status)``
    queues a copy of the device status words to pinned memory behind an
    event, and ``overflowed`` waits for that event. Up to ``depth`` renders
    may be outstanding: issuing one more first polls the oldest, and
    raises if that render overflowed unchecked. The reference sizes its buffers by reading the total
    on the host in the middle of every render (metal_backend.py:246-248),
    which drains the queue once per render.
    """

    def __init__(self, initial: int = 0, headroom: float = 1.25, depth: int = 8):
        self.value = int(initial)
        self.headroom = float(headroom)
        self.depth = int(depth)
        self.last_total = None
        self.overflows = 0
        self._slots = None      # pinned (depth, 3) int64: total, overflow, tag
        self._view = None       # the same memory as a numpy array, for polling
        self._events = None
        self._event_mode = None
        self._issued = 0

    def _next(self, event_mode: bool) -> int:
        if self._slots is None:
            self._slots = torch.zeros(self.depth, 3, dtype=torch.int64, pin_memory=True)
            self._view = self._slots.numpy()
            self._events = [None] * self.depth
            self._event_mode = [False] * self.depth
            self._observed = [True] * self.depth
        ticket = self._issued
        k = ticket % self.depth
        if not self._observed[k]:
            # The slot still holds a render nobody polled (more than
            # ``depth`` outstanding): read it before its status is
            # overwritten. An overflow there means an optimizer step that
            # changed nothing on the device while the host counted it.
            old = ticket - self.depth
            if self.overflowed(old):
                raise RuntimeError(
                    f"ListCapacity: render {old} overflowed its lists and was never checked; "
                    f"more than depth={self.depth} renders were outstanding. Poll each "
                    "render with overflowed(ticket) (and rewind() its optimizer step on "
                    "overflow) within depth renders, or raise depth.")
        self._issued += 1
        self._view[k, 2] = -1
        self._event_mode[k] = event_mode
        self._observed[k] = False
        return ticket

    def claim(self) -> tuple[int, int, int]:
        """(host slot address, tag, ticket) for the next render; render()
        calls this when given the object."""
        ticket = self._next(False)
        k = ticket % self.depth
        return self._slots[k].data_ptr(), ticket + 1, ticket

    def watch(self, status: torch.Tensor) -> int:
        ticket = self._next(True)
        k = ticket % self.depth
        self._slots[k, :2].copy_(status, non_blocking=True)
        if self._events[k] is None:
            self._events[k] = torch.cuda.Event()
        self._events[k].record(torch.cuda.current_stream(status.device))
        return ticket

    def overflowed(self, ticket: int | None = None, timeout_s: float = 60.0) -> bool:
        """Whether the render under ``ticket`` (default: the latest)
        overflowed; waits for its status."""
        if ticket is None:
            ticket = self._issued - 1
        if ticket < 0 or ticket >= self._issued or ticket < self._issued - self.depth:
            raise RuntimeError(f"ListCapacity: no outstanding render for ticket {ticket}")
        k = ticket % self.depth
        if self._event_mode[k]:
            self._events[k].synchronize()
        else:
            end = time.perf_counter() + timeout_s
            spins = 0
            while self._view[k, 2] != ticket + 1:
                # Spin briefly (a status is usually there within microseconds
                # of the render's binning), then yield the GIL and back off.
                spins += 1
                if spins > 64:
                    time.sleep(0.0 if spins < 1024 else 2e-5)
                if time.perf_counter() > end:
                    raise RuntimeError("ListCapacity: the lists' status never arrived")
        total, over = int(self._view[k, 0]), int(self._view[k, 1])
        self._observed[k] = True
        self.last_total = total
        if over:
            self.overflows += 1
            self.value = max(self.value, int(math.ceil(total * self.headroom)), total)
            if self.value >= 2 ** 31:
                raise RuntimeError(f"{total} tile intersections exceed the int32 index range")
        return bool(over)


def _bin_keys64(uv, rxy, depth, valid_i, conic, opacity, W, H, tile):
    """The same lists through the reference's ABI pipeline: mg_bin_count ->
    mg_exclusive_scan_i32 -> mg_bin_write (64-bit (tile|depth) keys) ->
    mg_sort_pairs_u64 -> mg_tile_ranges. Returns (gauss_ids, tile_offsets,
    tiles_x, sorted keys as int64)."""
    lib = _lib.load()
    device = uv.device
    tx, ty = _tile_grid(W, H, tile)
    n_tiles = tx * ty
    N = uv.shape[0]
    if N == 0:
        return _empty_lists(n_tiles, tx, device) + (torch.zeros(0, dtype=torch.int64,
                                                                device=device),)
    s = _lib.stream(uv)
    p_uv = _lib.dev_tensor(uv, "uv")
    p_rxy = _lib.dev_tensor(rxy, "rxy")
    p_valid = _lib.dev_tensor(valid_i, "valid", torch.int32)
    p_conic = _lib.dev_tensor(conic, "conic") if conic is not None else None
    p_op = _lib.dev_tensor(opacity, "opacity") if opacity is not None else None
    p_depth = _lib.dev_tensor(depth, "depth")

    counts = torch.empty(N, dtype=torch.int32, device=device)
    _lib.check(lib.mg_bin_count(N, p_uv, p_rxy, p_conic, p_op, p_valid, W, H, tile, tx, ty,
                                counts.data_ptr(), s))
    offsets = torch.empty(N, dtype=torch.int32, device=device)
    scan_ws = torch.empty(lib.mg_scan_workspace_bytes(N), dtype=torch.uint8, device=device)
    total_dev = torch.empty(1, dtype=torch.int64, device=device)
    host = _host_total()
    _lib.check(lib.mg_exclusive_scan_i32(counts.data_ptr(), N, offsets.data_ptr(),
                                         total_dev.data_ptr(), host.data_ptr(),
                                         scan_ws.data_ptr(), scan_ws.numel(), s))
    total = int(host[0])
    if total == 0:
        return _empty_lists(n_tiles, tx, device) + (torch.zeros(0, dtype=torch.int64,
                                                                device=device),)
    if total >= 2 ** 31:
        raise RuntimeError(f"{total} tile intersections exceed the int32 index range")

    keys = torch.empty(2 * total, dtype=torch.int64, device=device)
    ids = torch.empty(2 * total, dtype=torch.int32, device=device)
    k_in, k_out = keys[:total], keys[total:]
    i_in, i_out = ids[:total], ids[total:]
    _lib.check(lib.mg_bin_write(N, p_uv, p_rxy, p_conic, p_op, p_valid, p_depth,
                                offsets.data_ptr(), total, W, H, tile, tx, ty,
                                k_in.data_ptr(), i_in.data_ptr(), s))
    sort_ws = torch.empty(lib.mg_sort_workspace_bytes(total), dtype=torch.uint8, device=device)
    end_bit = 32 + max(1, (n_tiles - 1).bit_length())
    _lib.check(lib.mg_sort_pairs_u64(k_in.data_ptr(), i_in.data_ptr(), k_out.data_ptr(),
                                     i_out.data_ptr(), total, 0, end_bit, sort_ws.data_ptr(),
                                     sort_ws.numel(), s))
    tile_offsets = torch.empty(n_tiles + 1, dtype=torch.int32, device=device)
    _lib.check(lib.mg_tile_ranges(k_out.data_ptr(), total, n_tiles, tile_offsets.data_ptr(), s))
    return i_out, tile_offsets, tx, k_out


def _cap_per_tile(gauss_ids, tile_offsets, max_per_tile):
    """Nearest `max_per_tile` per tile (metal_backend.py:262-283); off by default."""
    n_tiles = tile_offsets.numel() - 1
    counts = (tile_offsets[1:] - tile_offsets[:-1]).to(torch.int64)
    tile_of = torch.repeat_interleave(torch.arange(n_tiles, device=gauss_ids.device), counts)
    rank = torch.arange(gauss_ids.numel(), device=gauss_ids.device) - \
        tile_offsets[:-1].to(torch.int64)[tile_of]
    keep = rank < max_per_tile
    kept = torch.minimum(counts, torch.tensor(max_per_tile, device=counts.device))
    offs = torch.zeros(n_tiles + 1, dtype=torch.int64, device=counts.device)
    offs[1:] = torch.cumsum(kept, 0)
    return gauss_ids[keep].contiguous(), offs.to(torch.int32).contiguous()


def build_tile_lists_metal(uv, rxy, depth, valid, conic, opacity, W, H, tile,
                           max_per_tile: int = 0):
    """Tile lists with the exact ellipse-vs-tile test (metal_backend.py:217-285).

    Returns (gauss_ids int32 sorted by (tile, depth), tile_offsets int32
    (n_tiles+1), tiles_x). Equal keys keep emission order (Gaussian, row,
    column): both sorts are stable.
    """
    _require_gpu(uv)
    valid_i = valid.to(torch.int32).contiguous()
    out = _bin(uv.detach().contiguous(), rxy.detach().contiguous(), depth.detach().contiguous(),
               valid_i, conic.detach().contiguous(), opacity.detach().contiguous(), W, H, tile)
    gauss_ids, tile_offsets, tx = out[0], out[1], out[2]
    if max_per_tile > 0 and gauss_ids.numel() > 0:
        gauss_ids, tile_offsets = _cap_per_tile(gauss_ids, tile_offsets, max_per_tile)
    return gauss_ids, tile_offsets, tx


# The reference's name describes its kernel language; this is the same call.
build_tile_lists_hip = build_tile_lists_metal


def build_tile_lists(uv, radius, depth, valid, W, H, tile, ry=None, conic=None, opacity=None):
    """Tile lists from rectangular bounds (metal_backend.py:111-214).

    ``radius`` is the x half-extent and ``ry`` the y half-extent (default
    ``radius``). With ``conic`` and ``opacity`` the exact ellipse test is
    applied as in build_tile_lists_metal; without them every tile of the
    rectangle is listed.
    """
    _require_gpu(uv)
    if ry is None:
        ry = radius
    rxy = torch.stack([radius.detach(), ry.detach()], dim=-1).to(torch.float32).contiguous()
    valid_i = valid.to(torch.int32).contiguous()
    if (conic is None) != (opacity is None):
        conic = opacity = None
    out = _bin(uv.detach().contiguous(), rxy, depth.detach().contiguous(), valid_i,
               None if conic is None else conic.detach().contiguous(),
               None if opacity is None else opacity.detach().contiguous(), W, H, tile)
    return out[0], out[1], out[2]


def _camera(K, viewmat):
    K_h = K if K.device.type == "cpu" else K.detach().cpu()
    fx, fy = float(K_h[0, 0]), float(K_h[1, 1])
    cx, cy = float(K_h[0, 2]), float(K_h[1, 2])
    vm_h = viewmat.detach()
    if vm_h.device.type != "cpu":
        vm_h = vm_h.cpu()
    vm_h = vm_h.to(torch.float32).contiguous()
    cam_center = (-vm_h[:3, :3].T @ vm_h[:3, 3]).contiguous()
    return fx, fy, cx, cy, vm_h, cam_center


# Slots of the rasteriser backward's per-Gaussian gradient record
# (mg_rasterize_backward): d_uv 0-1, d_conic 2-4, d_opacity 5, d_color 6-8,
# sum |d_uv| 9.
_REC = 10


def _grad_inputs(N, dev, d_uv, d_conic, d_color, d_oe, want_color, want_oe):
    """Pointers and record stride for the preprocess backward's incoming
    gradients. Row views of one gradient record (what the raster backward
    hands autograd) are read in place with the record's stride; anything else
    becomes separate contiguous arrays (zeros for a missing gradient)."""
    mats = [d_uv, d_conic] + ([d_color] if want_color else [])
    ts = mats + ([d_oe] if want_oe else [])
    if all(t is not None and t.device.type == "cuda" and t.dtype == torch.float32 for t in ts):
        k = d_uv.stride(0)
        ok = k >= 3 and all(t.dim() == 2 and t.shape[0] == N and t.stride(0) == k and
                            t.stride(1) == 1 for t in mats)
        if want_oe:
            ok = ok and d_oe.dim() == 1 and d_oe.shape[0] == N and d_oe.stride(0) == k
        if ok:
            return ([d_uv.data_ptr(), d_conic.data_ptr(),
                     d_color.data_ptr() if want_color else None,
                     d_oe.data_ptr() if want_oe else None], k, ())

    def dense(t, shape):
        return torch.zeros(*shape, device=dev) if t is None else t.contiguous()
    keep = (dense(d_uv, (N, 2)), dense(d_conic, (N, 3)),
            dense(d_color, (N, 3)) if want_color else None,
            dense(d_oe, (N,)) if want_oe else None)
    ptrs = [None if t is None else _lib.dev_tensor(t, what)
            for t, what in zip(keep, ("d_uv", "d_conic", "d_color", "d_opacity"))]
    return ptrs, 0, keep


class _PreprocessMetal(torch.autograd.Function):
    """Fused projection + SH colour, forward and analytic backward.

    Same bridge as metal_backend.py:288-333. ``sh_rest is None`` means ``sh``
    is one (N,16,3) tensor; otherwise sh is the (N,1,3) DC band and sh_rest
    the (N,15,3) bands 1+. ``sh is None`` is the explicit-colour route: only
    the projection runs and no colour is returned.
    """

    @staticmethod
    def forward(ctx, means, quats, scales, sh, sh_rest, ctx_opac, viewmat, fx, fy, cx, cy,
                W, H, near, far, blur, max_radius, cam_center, sh_degree, valid_mask=None):
        # valid_mask: an optional (N,) bool buffer the kernel also fills with
        # the visibility flags (render's info["valid_mask"]).
        lib = _lib.load()
        N = means.shape[0]
        dev = means.device
        means, quats, scales = (t.contiguous() for t in (means, quats, scales))
        fused = sh_rest is None
        if sh is not None:
            sh = sh.contiguous()
            rest = None if fused else sh_rest.contiguous()
            if fused and tuple(sh.shape[1:]) != (16, 3) or (not fused and (
                    tuple(sh.shape[1:]) != (1, 3) or tuple(rest.shape[1:]) != (15, 3))):
                raise RuntimeError(
                    "SH must be either one (N,16,3) tensor or (N,1,3)+(N,15,3); got "
                    f"{tuple(sh.shape)} and {None if rest is None else tuple(rest.shape)}")
        else:
            rest = None
        opac = ctx_opac.contiguous()
        uv = torch.empty(N, 2, device=dev)
        conic = torch.empty(N, 3, device=dev)
        depth = torch.empty(N, device=dev)
        rxy = torch.empty(N, 2, device=dev)
        valid = torch.empty(N, dtype=torch.int32, device=dev)
        color = torch.empty(N, 3, device=dev) if sh is not None else None
        vm = _lib.host_f32(viewmat)
        cc = _lib.host_f32(cam_center)
        _lib.check(lib.mg_preprocess_forward(
            N, _lib.dev_tensor(means, "means"), _lib.dev_tensor(quats, "quats"),
            _lib.dev_tensor(scales, "scales"),
            None if sh is None else _lib.dev_tensor(sh, "sh"),
            None if rest is None else _lib.dev_tensor(rest, "sh_rest"), int(fused),
            _lib.dev_tensor(opac, "opacities"), vm, fx, fy, cx, cy, W, H, near, far, blur,
            max_radius, cc, sh_degree, uv.data_ptr(), conic.data_ptr(), depth.data_ptr(),
            rxy.data_ptr(), valid.data_ptr(),
            None if valid_mask is None else _lib.dev_tensor(valid_mask, "valid_mask", torch.bool),
            None if color is None else color.data_ptr(), _lib.stream(means)))
        ctx.save_for_backward(means, quats, scales, sh, rest, valid)
        # depth, rxy and valid carry no gradient: no zeros are materialised
        # for them (or for an unused output) in the backward.
        ctx.set_materialize_grads(False)
        ctx.fused = fused
        ctx.has_sh = sh is not None
        ctx.meta = (viewmat, fx, fy, cx, cy, W, H, near, far, blur, max_radius, cam_center,
                    sh_degree)
        ctx.mark_non_differentiable(depth, rxy, valid)
        if color is None:
            return uv, conic, depth, rxy, valid
        return uv, conic, depth, rxy, valid, color

    @staticmethod
    def backward(ctx, d_uv, d_conic, d_depth, d_rxy, d_valid, d_color=None):
        lib = _lib.load()
        means, quats, scales, sh, rest, valid = ctx.saved_tensors
        viewmat, fx, fy, cx, cy, W, H, near, far, blur, max_radius, cam_center, deg = ctx.meta
        N = means.shape[0]
        dev = means.device
        d_means = torch.empty(N, 3, device=dev)
        d_quats = torch.empty(N, 4, device=dev)
        d_scales = torch.empty(N, 3, device=dev)
        d_sh = d_rest = None
        if ctx.has_sh:
            d_sh = torch.empty_like(sh)
            d_rest = None if ctx.fused else torch.empty_like(rest)
        (p_uv, p_conic, p_color, _), stride, keep = _grad_inputs(
            N, dev, d_uv, d_conic, d_color, None, ctx.has_sh, False)
        _lib.check(lib.mg_preprocess_backward(
            N, means.data_ptr(), quats.data_ptr(), scales.data_ptr(),
            None if sh is None else sh.data_ptr(), None if rest is None else rest.data_ptr(),
            int(ctx.fused), p_uv, p_conic, p_color, stride, valid.data_ptr(),
            _lib.host_f32(viewmat), fx, fy, cx, cy, W, H, near, far, blur, max_radius,
            _lib.host_f32(cam_center), deg, d_means.data_ptr(), d_quats.data_ptr(),
            d_scales.data_ptr(), None if d_sh is None else d_sh.data_ptr(),
            None if d_rest is None else d_rest.data_ptr(), _lib.stream(means)))
        return (d_means, d_quats, d_scales, d_sh, d_rest) + (None,) * 15


class _RasterizeMetal(torch.autograd.Function):
    """Compositing forward/backward bridge (metal_backend.py:336-364)."""

    @staticmethod
    def forward(ctx, uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, tiles_x,
                absgrad_out=None, t_min=DEFAULT_T_MIN, background=None, chunked=False):
        """``background`` is None or three host floats blended in the kernel
        (rgb + max(1 - alpha, 0) * background); the backward then carries the
        blend's gradient too. ``chunked`` runs the backward as independent
        512-entry units per tile from checkpoints the forward records, which
        pays when a few tiles hold most of the intersections."""
        lib = _lib.load()
        dev = uv.device
        uv, conic, opacity, color = (t.contiguous() for t in (uv, conic, opacity, color))
        N = uv.shape[0]
        rgb = torch.empty(H, W, 3, device=dev)
        alpha = torch.empty(H, W, device=dev)
        T = torch.empty(H, W, device=dev)
        stop = torch.empty(H, W, dtype=torch.int32, device=dev)
        # Plan + per-chunk pixel states for the chunked backward.
        n_isect = gauss_ids.numel()
        chunk_ws = torch.empty(
            lib.mg_rasterize_chunk_workspace_bytes(n_isect, tile_offsets.numel() - 1, tile)
            if chunked else 0, dtype=torch.uint8, device=dev)
        # The backward's gradient records, cleared by the forward kernel on
        # the way (the backward then skips its own fill), when a backward can
        # follow.
        rec = (torch.empty(N, _REC, device=dev) if N and any(ctx.needs_input_grad[:4])
               else None)
        # With a backward to come, the forward records each tile's walk
        # length so that the backward can run the longest walks first.
        sched = (torch.empty(lib.mg_rasterize_sched_ints(W, H, tile), dtype=torch.int32,
                             device=dev) if rec is not None and not chunked else None)
        _lib.check(lib.mg_rasterize_forward(
            N, _lib.dev_tensor(uv, "uv"), _lib.dev_tensor(conic, "conic"),
            _lib.dev_tensor(opacity, "opacity"), _lib.dev_tensor(color, "color"),
            _lib.dev_tensor(gauss_ids, "gauss_ids", torch.int32),
            _lib.dev_tensor(tile_offsets, "tile_offsets", torch.int32), W, H, tile, tiles_x,
            float(t_min), None if background is None else _lib.f32_array(background),
            n_isect, chunk_ws.data_ptr() if chunked else None, chunk_ws.numel(), rgb.data_ptr(),
            alpha.data_ptr(), T.data_ptr(), stop.data_ptr(),
            None if rec is None else rec.data_ptr(),
            None if sched is None else sched.data_ptr(), _lib.stream(uv)))
        ctx.save_for_backward(uv, conic, opacity, color, gauss_ids, tile_offsets, T, stop,
                              alpha if background is not None else None, chunk_ws)
        ctx.rec = rec
        ctx.sched = sched
        ctx.dims = (W, H, tile, tiles_x)
        ctx.background = background
        # An output nobody differentiates (alpha, most often) gets no
        # materialised zeros: the kernel reads a missing grad_alpha as 0.
        ctx.set_materialize_grads(False)
        # absgrad is a statistic of the backward, not a gradient: the caller
        # hands in a buffer and the backward accumulates into it.
        ctx.absgrad_out = absgrad_out
        return rgb, alpha

    @staticmethod
    def backward(ctx, grad_rgb, grad_alpha):
        lib = _lib.load()
        (uv, conic, opacity, color, gauss_ids, tile_offsets, T, stop, alpha,
         chunk_ws) = ctx.saved_tensors
        W, H, tile, tiles_x = ctx.dims
        bg = ctx.background
        N = uv.shape[0]
        dev = uv.device
        # One gradient record per Gaussian; autograd gets row views of it.
        rec, zeroed = ctx.rec, ctx.rec is not None
        ctx.rec = None
        sched = ctx.sched
        if rec is None:
            rec = torch.empty(N, _REC, device=dev)
        if grad_rgb is None and grad_alpha is None:
            return (None,) * 14
        grad_rgb = torch.zeros(H, W, 3, device=dev) if grad_rgb is None else grad_rgb.contiguous()
        grad_alpha = None if grad_alpha is None else grad_alpha.contiguous()
        _lib.check(lib.mg_rasterize_backward(
            N, uv.data_ptr(), conic.data_ptr(), opacity.data_ptr(), color.data_ptr(),
            gauss_ids.data_ptr(), tile_offsets.data_ptr(), T.data_ptr(), stop.data_ptr(),
            _lib.dev_tensor(grad_rgb, "grad_rgb"),
            None if grad_alpha is None else _lib.dev_tensor(grad_alpha, "grad_alpha"),
            None if bg is None else alpha.data_ptr(), None if bg is None else _lib.f32_array(bg),
            gauss_ids.numel(), chunk_ws.data_ptr() if chunk_ws.numel() else None,
            chunk_ws.numel(), W, H, tile, tiles_x, rec.data_ptr(),
            int(ctx.absgrad_out is not None), int(zeroed),
            None if sched is None else sched.data_ptr(), _lib.stream(uv)))
        if ctx.absgrad_out is not None:
            ctx.absgrad_out[:N] += rec[:, 9]
        return (rec[:, 0:2], rec[:, 2:5], rec[:, 5], rec[:, 6:9]) + (None,) * 10


class _PreprocessMip(torch.autograd.Function):
    """Preprocess with Mip-Splatting's filters folded into the kernel.

    The reference applies the 3D filter as a torch reparameterisation of
    scales and opacity before render (train.py:214-229, mipfilter.py:76-93)
    and the 2D antialias compensation as torch ops on the conic after
    preprocess (metal_backend.py:367-393, 506-511). Here both run inside the
    projection kernel: it takes the unfiltered scales and opacity (and
    ``filter_3d`` as a constant) and returns, after the usual outputs, the
    opacity binning and compositing use. The backward carries that opacity's
    gradient to the opacity, the scales and the projected covariance.
    ``activations`` (bit 0: scales are log scales, bit 1: opacities are
    logits) moves the trainer's torch.exp / torch.sigmoid (train.py:221-222)
    into the same kernels; the gradients then land on the log scales and
    logits. ``reg`` = (opacity weight, scale weight) adds the gradient of
    w_o * mean(opacity) + w_s * mean(scale) over the activated values, the
    trainer's regularisers (train.py:396-398), to every row in the kernel.
    """

    @staticmethod
    def forward(ctx, means, quats, scales, opacities, sh, sh_rest, filter_3d, antialias,
                viewmat, fx, fy, cx, cy, W, H, near, far, blur, max_radius, cam_center,
                sh_degree, valid_mask=None, activations=0, optimizer=None, reg=None,
                lists=None, block_work=None):
        lib = _lib.load()
        N = means.shape[0]
        dev = means.device
        means, quats, scales, opacities = (t.contiguous() for t in
                                           (means, quats, scales, opacities))
        fused = sh_rest is None
        if sh is not None:
            sh = sh.contiguous()
            rest = None if fused else sh_rest.contiguous()
        else:
            rest = None
        filt = None
        if filter_3d is not None:
            filt = filter_3d.detach().to(torch.float32).contiguous()
            if filt.shape != (N,):
                raise ValueError(f"filter_3d must be ({N},), got {tuple(filt.shape)}")
        uv = torch.empty(N, 2, device=dev)
        conic = torch.empty(N, 3, device=dev)
        depth = torch.empty(N, device=dev)
        rxy = torch.empty(N, 2, device=dev)
        valid = torch.empty(N, dtype=torch.int32, device=dev)
        color = torch.empty(N, 3, device=dev) if sh is not None else None
        op_eff = torch.empty(N, device=dev)
        _lib.check(lib.mg_preprocess_forward_mip(
            N, _lib.dev_tensor(means, "means"), _lib.dev_tensor(quats, "quats"),
            _lib.dev_tensor(scales, "scales"),
            None if sh is None else _lib.dev_tensor(sh, "sh"),
            None if rest is None else _lib.dev_tensor(rest, "sh_rest"), int(fused),
            _lib.dev_tensor(opacities, "opacities"), _lib.host_f32(viewmat), fx, fy, cx, cy,
            W, H, near, far, blur, max_radius, _lib.host_f32(cam_center), sh_degree,
            None if filt is None else _lib.dev_tensor(filt, "filter_3d"), int(bool(antialias)),
            int(activations), uv.data_ptr(), conic.data_ptr(), depth.data_ptr(), rxy.data_ptr(), valid.data_ptr(),
            None if valid_mask is None else _lib.dev_tensor(valid_mask, "valid_mask", torch.bool),
            None if color is None else color.data_ptr(), op_eff.data_ptr(),
            block_work[0] if block_work else 0,
            block_work[1].data_ptr() if block_work else None, _lib.stream(means)))
        ctx.save_for_backward(means, quats, scales, opacities, sh, rest, filt, valid)
        ctx.set_materialize_grads(False)
        ctx.fused = fused
        ctx.has_sh = sh is not None
        ctx.antialias = bool(antialias)
        ctx.activations = int(activations)
        ctx.optimizer = optimizer
        ctx.reg = _reg_coefficients(reg, N)
        # render() puts the status of capacity-bounded lists here once they
        # are built: the epilogue's update is skipped if they overflowed.
        ctx.lists = lists
        ctx.meta = (viewmat, fx, fy, cx, cy, W, H, near, far, blur, max_radius, cam_center,
                    sh_degree)
        ctx.mark_non_differentiable(depth, rxy, valid)
        if color is None:
            return uv, conic, depth, rxy, valid, op_eff
        return uv, conic, depth, rxy, valid, color, op_eff

    @staticmethod
    def backward(ctx, d_uv, d_conic, d_depth, d_rxy, d_valid, *rest_grads):
        lib = _lib.load()
        means, quats, scales, opacities, sh, rest, filt, valid = ctx.saved_tensors
        viewmat, fx, fy, cx, cy, W, H, near, far, blur, max_radius, cam_center, deg = ctx.meta
        if ctx.has_sh:
            d_color, d_oe = rest_grads
        else:
            d_color, (d_oe,) = None, rest_grads
        N = means.shape[0]
        dev = means.device
        params = (means, quats, scales, opacities, sh, None if ctx.fused else rest)
        epi = _epilogue(ctx, params, deg)
        (p_uv, p_conic, p_color, p_oe), stride, keep = _grad_inputs(
            N, dev, d_uv, d_conic, d_color, d_oe, ctx.has_sh, True)
        if epi is not None:
            # The optimizer's step for these parameters runs inside the kernel;
            # no gradient tensor is formed and autograd gets none.
            _lib.check(lib.mg_preprocess_backward_mip(
                N, means.data_ptr(), quats.data_ptr(), scales.data_ptr(), sh.data_ptr(),
                None if rest is None else rest.data_ptr(), int(ctx.fused), p_uv, p_conic,
                p_color, stride, valid.data_ptr(), _lib.host_f32(viewmat), fx, fy, cx, cy, W,
                H, near, far, blur, max_radius, _lib.host_f32(cam_center), deg,
                opacities.data_ptr(), None if filt is None else filt.data_ptr(),
                int(ctx.antialias), ctx.activations, *ctx.reg, p_oe, None, None, None, None,
                None, None, ctypes.byref(epi), _lib.stream(means)))
            return (None,) * 27
        d_means = torch.empty(N, 3, device=dev)
        d_quats = torch.empty(N, 4, device=dev)
        d_scales = torch.empty(N, 3, device=dev)
        d_op = torch.empty(N, device=dev)
        d_sh = d_rest = None
        if ctx.has_sh:
            d_sh = torch.empty_like(sh)
            d_rest = None if ctx.fused else torch.empty_like(rest)
        _lib.check(lib.mg_preprocess_backward_mip(
            N, means.data_ptr(), quats.data_ptr(), scales.data_ptr(),
            None if sh is None else sh.data_ptr(), None if rest is None else rest.data_ptr(),
            int(ctx.fused), p_uv, p_conic, p_color, stride, valid.data_ptr(),
            _lib.host_f32(viewmat), fx, fy, cx, cy, W, H, near, far, blur, max_radius,
            _lib.host_f32(cam_center), deg, opacities.data_ptr(),
            None if filt is None else filt.data_ptr(), int(ctx.antialias), ctx.activations,
            *ctx.reg, p_oe, d_means.data_ptr(), d_quats.data_ptr(),
            d_scales.data_ptr(), None if d_sh is None else d_sh.data_ptr(),
            None if d_rest is None else d_rest.data_ptr(), d_op.data_ptr(), None,
            _lib.stream(means)))
        return (d_means, d_quats, d_scales, d_op, d_sh, d_rest) + (None,) * 21


def _reg_coefficients(reg, n):
    """Per-element gradients (reg_opacity, reg_scale) of the regulariser
    weights (w_o, w_s) on mean(opacity) over n rows and mean(scale) over 3n
    elements, rounded as torch's float32 mean backward forms them
    (weight / count)."""
    if reg is None or n == 0:
        return (0.0, 0.0)
    w_o, w_s = (float(np.float32(w)) for w in reg)
    return (float(np.float32(w_o) / np.float32(n)), float(np.float32(w_s) / np.float32(3 * n)))


def _epilogue(ctx, params, sh_degree):
    """The optimizer's step as the preprocess backward's epilogue, or None
    when the ordinary gradients must be returned: no optimizer given, the
    explicit-colour route, SH degree below 3, a parameter that does not
    require grad, SH tensors or moments the kernel cannot stage (16-byte
    alignment), or whatever the optimizer's own ``epilogue`` refuses."""
    opt = ctx.optimizer
    if opt is None or not ctx.has_sh or sh_degree != 3 or not hasattr(opt, "epilogue"):
        return None
    for t, need in zip(params, ctx.needs_input_grad[:6]):
        if t is not None and not need:
            return None
    sh, rest = params[4], params[5]
    if sh.data_ptr() % 16 or (rest is not None and rest.data_ptr() % 16):
        return None
    skip = ctx.lists[0] if ctx.lists else None
    if skip is None:
        return opt.epilogue(list(params))
    return opt.epilogue(list(params), skip=skip)


# Names that describe this backend rather than the reference's.
_PreprocessHIP = _PreprocessMetal
_RasterizeHIP = _RasterizeMetal


def _host_background(background):
    """Three host floats for the in-kernel blend, or None when the torch
    expression must do it (no background, a device tensor, or one that
    requires grad)."""
    if background is None:
        return None
    if isinstance(background, torch.Tensor):
        if background.device.type != "cpu" or background.requires_grad:
            return None
        vals = background.detach().to(torch.float32).reshape(-1).tolist()
    else:
        vals = [float(v) for v in background]
    if len(vals) != 3:
        return None
    return tuple(vals)


def antialias_scale(conic: torch.Tensor, blur: float) -> torch.Tensor:
    """Mip-Splatting opacity compensation sqrt(det_before / det_after).

    Recovered from the conic, the inverse of the dilated covariance
    (metal_backend.py:367-393): det_after = 1/det(conic), the dilated
    covariance is (conic_z, -conic_y, conic_x) * det_after, and the undilated
    determinant subtracts ``blur`` from the diagonal. Torch autograd carries
    its gradient into the conic.
    """
    cxx, cxy, cyy = conic[:, 0], conic[:, 1], conic[:, 2]
    det_conic = (cxx * cyy - cxy * cxy).clamp_min(1e-12)
    det_after = 1.0 / det_conic
    a = cyy * det_after
    b = -cxy * det_after
    c = cxx * det_after
    det_before = (a - blur) * (c - blur) - b * b
    return (det_before.clamp_min(0.0) / det_after).clamp(0.0, 1.0).sqrt()


def _sh_inputs(sh, sh_rest):
    """(sh_in, rest_in) for the kernel: fused (N,16,3) with rest None, or the
    (N,1,3) + (N,15,3) pair; narrower inputs are zero-padded
    (metal_backend.py:482-497)."""
    if sh_rest is None:
        sh_in = sh
        if sh_in.shape[1] < 16:
            pad = torch.zeros(sh_in.shape[0], 16 - sh_in.shape[1], 3, device=sh_in.device,
                              dtype=sh_in.dtype)
            sh_in = torch.cat([sh_in, pad], dim=1)
        return sh_in, None
    if sh.shape[1] != 1:
        raise ValueError(
            f"with sh_rest given, sh must be the DC band (N,1,3); got {tuple(sh.shape)}")
    rest_in = sh_rest
    if rest_in.shape[1] < 15:
        pad = torch.zeros(rest_in.shape[0], 15 - rest_in.shape[1], 3, device=rest_in.device,
                          dtype=rest_in.dtype)
        rest_in = torch.cat([rest_in, pad], dim=1)
    return sh, rest_in


def render(means, quats, scales, opacities, sh, K, viewmat, W, H,
           sh_degree: int = 3, tile: int | None = None,
           near: float = 0.01, far: float = 100.0,
           background=(0.0, 0.0, 0.0), colors=None, max_radius_frac: float = 1.0,
           sh_rest=None, antialias: bool = False, absgrad_out=None,
           min_transmittance: float = DEFAULT_T_MIN, chunked_backward: bool = False,
           filter_3d=None, activations: bool = False, optimizer=None,
           opacity_reg: float = 0.0, scale_reg: float = 0.0, list_capacity=None,
           **_ignored):
    """Render Gaussians from one camera; same signature as the reference's.

    means (N,3) world; quats (N,4) wxyz (need not be normalised); scales (N,3)
    linear; opacities (N,) in [0,1]; sh (N,B,3) or the (N,1,3) DC band with
    ``sh_rest`` (N,15,3); K (3,3); viewmat (4,4) world->camera. Returns
    (rgb (H,W,3), alpha (H,W), info). ``colors`` (N,3) bypasses SH.
    ``min_transmittance`` is the per-pixel early-stop threshold (the
    reference's fixed 1e-4); 0 composites every listed Gaussian.
    ``chunked_backward`` splits each tile's backward into 512-entry units run
    in parallel (same gradients up to rounding); it helps when a few tiles hold
    most of the intersections.
    ``filter_3d`` (N,) applies Mip-Splatting's 3D filter inside the
    projection kernel: the result equals rendering
    ``apply_3d_filter(scales, opacities, filter_3d)`` (what the reference's
    trainer does in torch, train.py:223-227), with the filter a constant.
    ``antialias`` likewise runs in the kernel.
    ``activations=True`` takes ``scales`` as log scales and ``opacities`` as
    logits: the exp and sigmoid the reference's trainer applies in torch
    before render (train.py:221-222) run inside the projection kernel and
    their derivatives in its backward, so the gradients land on the log
    scales and logits (the same values as torch.exp / torch.sigmoid in
    front of ``render``).
    ``opacity_reg`` and ``scale_reg`` add the trainer's regularisers
    opacity_reg * mean(opacity) + scale_reg * mean(scale) of the activated
    values (with ``activations``: mean(sigmoid(logit)) and
    mean(exp(log_scales)), train.py:396-398) to the loss this render's
    backward differentiates: their gradient is added to every row inside the
    projection backward, and ``info["regularizer"]()`` returns their value
    (a device scalar) for the loss the caller reports.
    ``optimizer`` (a FusedAdam over these parameters) moves its step for
    means, quats, scales, opacities and the SH into the projection
    backward: the kernel updates the parameters and moments in place, no
    gradient tensors are formed, their ``.grad`` stays unset and the
    optimizer's ``step()`` skips them. That equals the backward followed by
    ``step()`` when this render (with its regularisers) is the only use of
    those parameters in the loss. Any other use would reach them as a
    ``.grad`` after their update: ``step()`` then raises instead of updating
    them a second time. When the optimizer or the tensors do not allow the
    epilogue, the ordinary gradients are returned.
    ``list_capacity`` (a ``ListCapacity``, or an int) builds the tile lists
    in buffers of that many intersections with no host read, so the render
    enqueues without waiting for the GPU. ``info["lists_status"]`` is then a
    device int64 (2,): the intersection total, and 1 if it exceeded the
    capacity, in which case every list is empty (the image is the
    background), the epilogue of ``optimizer`` does nothing, and the caller
    renders again with a larger capacity; with a ``ListCapacity`` the same
    words reach its host slot and ``info["lists_ticket"]`` is the ticket to
    check with ``overflowed``. ``info["isect_total"]`` is then that device
    total (0-d) instead of an int.
    """
    explicit_colors = colors is not None
    opacities_in = opacities
    _require_gpu(means)
    if tile is None:
        tile = 16
    W, H, tile = int(W), int(H), int(tile)
    mt = _lib.open_library().mg_max_tile()
    if tile * tile > mt * mt:
        raise RuntimeError(
            f"tile {tile} needs {tile * tile} threads per threadgroup; rasterize_forward "
            f"allows at most {mt * mt} on this GPU")
    fx, fy, cx, cy, vm_h, cam_center = _camera(K, viewmat)
    max_radius = max_radius_frac * max(W, H)
    # info["valid_mask"], written by the projection kernel itself.
    valid_b = torch.empty(means.shape[0], dtype=torch.bool, device=means.device)

    reg = None
    if opacity_reg or scale_reg:
        reg = (float(opacity_reg), float(scale_reg))
    # The epilogue's skip word, filled in once the lists are built.
    lists = [None] if list_capacity is not None else None
    # Past _BLOCK_ORDER_TILES tiles the capacity lists' count and write passes
    # take their blocks of 256 Gaussians heaviest first, from a per-block
    # work estimate the projection kernel writes (the mip projection only).
    block_work = None
    if (filter_3d is not None or antialias or activations or optimizer is not None
            or reg is not None):
        if list_capacity is not None and means.shape[0] > 0:
            tx, ty = _tile_grid(W, H, tile)
            if tx * ty > _BLOCK_ORDER_TILES:
                block_work = (tile, torch.empty((means.shape[0] + 255) // 256,
                                                dtype=torch.int32, device=means.device))
        # Both filters (and the activations) in the projection kernel; the
        # compensated opacity is binned too, which gives a tighter, still
        # exact, ellipse bound (metal_backend.py:506-511).
        act = 3 if activations else 0
        if explicit_colors:
            uv, conic, depth, rxy, valid_i, opacities = _PreprocessMip.apply(
                means, quats, scales, opacities, None, None, filter_3d, antialias, vm_h, fx,
                fy, cx, cy, W, H, near, far, 0.3, max_radius, cam_center, sh_degree, valid_b,
                act, None, reg, None, block_work)
            colors = colors.contiguous()
        else:
            sh_in, rest_in = _sh_inputs(sh, sh_rest)
            uv, conic, depth, rxy, valid_i, colors, opacities = _PreprocessMip.apply(
                means, quats, scales, opacities, sh_in, rest_in, filter_3d, antialias, vm_h,
                fx, fy, cx, cy, W, H, near, far, 0.3, max_radius, cam_center, sh_degree,
                valid_b, act, optimizer, reg, lists, block_work)
    elif explicit_colors:
        uv, conic, depth, rxy, valid_i = _PreprocessMetal.apply(
            means, quats, scales, None, None, opacities.detach(), vm_h, fx, fy, cx, cy, W, H,
            near, far, 0.3, max_radius, cam_center, sh_degree, valid_b)
        colors = colors.contiguous()
    else:
        sh_in, rest_in = _sh_inputs(sh, sh_rest)
        uv, conic, depth, rxy, valid_i, colors = _PreprocessMetal.apply(
            means, quats, scales, sh_in, rest_in, opacities.detach(), vm_h, fx, fy, cx, cy,
            W, H, near, far, 0.3, max_radius, cam_center, sh_degree, valid_b)

    status = None
    ticket = None
    if list_capacity is None:
        gauss_ids, tile_offsets, tiles_x = build_tile_lists_metal(
            uv.detach(), rxy.detach(), depth.detach(), valid_i, conic.detach(),
            opacities.detach(), W, H, tile)
    else:
        slot, tag, capacity = None, 0, list_capacity
        if isinstance(list_capacity, ListCapacity):
            slot, tag, ticket = list_capacity.claim()
            capacity = list_capacity.value
        gauss_ids, tile_offsets, tiles_x, status = _bin_capped(
            uv.detach().contiguous(), rxy.detach().contiguous(), depth.detach().contiguous(),
            valid_i.contiguous(), conic.detach().contiguous(), opacities.detach().contiguous(),
            W, H, tile, capacity, slot, tag, None if block_work is None else block_work[1])
        lists[0] = status

    # A constant background (tuple, list or CPU tensor without grad) is
    # blended inside the raster kernels; a device or trainable one by the
    # reference's torch expression (metal_backend.py:539-541).
    bg_host = _host_background(background)
    rgb, alpha = _RasterizeMetal.apply(
        uv, conic, opacities, colors, gauss_ids, tile_offsets, W, H, tile, tiles_x,
        absgrad_out, min_transmittance, bg_host, chunked_backward)

    if background is not None and bg_host is None:
        bg = torch.as_tensor(background, device=rgb.device, dtype=rgb.dtype)
        rgb = rgb + (1.0 - alpha).clamp_min(0)[..., None] * bg

    if uv.requires_grad:
        _retain_grad_in_place(uv)

    info_reg = None
    if reg is not None:
        info_reg = _regularizer_value(scales, opacities_in, reg, bool(activations))
    return rgb, alpha, {
        "uv": uv,
        "tiles": int(tile_offsets.numel() - 1),
        "isect_total": int(gauss_ids.numel()) if status is None else status[0],
        "lists_status": status,
        "lists_ticket": ticket,
        "isect_dropped": 0,
        "isect_dropped_frac": 0.0,
        "valid_mask": valid_b,
        "backend": "hip",
        "regularizer": info_reg,
    }


def _retain_grad_in_place(t):
    """``t.retain_grad()`` (metal_backend.py:548-549) without its copy:
    retain_grad stores a contiguous clone of the incoming gradient, which for
    uv is a strided (N,2) view of the raster backward's gradient record (a
    gather of 8 bytes out of every 40, about 10 us at 1M Gaussians per
    backward). Here t.grad becomes that view itself, summed over repeated
    backwards as retain_grad sums. The hook holds t weakly."""
    ref = weakref.ref(t)
    seen = [False]

    def hook(g):
        x = ref()
        if x is None:
            return
        cur = None
        if seen[0]:
            # Defined unless the caller reset it (reading an unset .grad of a
            # non-leaf warns, hence the flag).
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                cur = x.grad
        x.grad = g if cur is None else cur + g
        seen[0] = True
    t.register_hook(hook)


def _regularizer_value(scales, opacities, reg, activations):
    """A callable returning the regularisers' value w_o * mean(opacity) +
    w_s * mean(scale) (activated values) as a device scalar, computed when
    called; its gradient is already part of render's backward."""
    w_o, w_s = reg

    def value():
        with torch.no_grad():
            op = torch.sigmoid(opacities) if activations else opacities
            sc = torch.exp(scales) if activations else scales
            return w_o * op.mean() + w_s * sc.mean()
    return value
