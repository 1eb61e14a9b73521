"""The reference's native-extension surface over libmgauss.so.

metal_gauss/metal_backend.py:_load() returns a pybind11 module whose
functions take and return torch tensors (metal_gauss/csrc/rasterize.mm:
79-533). This module has the same thirteen functions, with the same argument
order, output shapes, dtypes and in-place behaviour, so code written against
that module - the reference's autograd bridges (metal_backend.py:288-364),
its tile-list builder (217-285) and its trainer's fused SSIM
(train.py:67-105) - runs unchanged on gfx950: ``backend._load()`` returns this
module.

Each function allocates its outputs on the inputs' device, as the reference
does with ``torch::zeros/empty``, launches on torch's current HIP stream and
raises RuntimeError with the library's message on failure. Tensors must be
ROCm (``cuda``) tensors: the reference's "must be an MPS tensor" check becomes
"must be a HIP (ROCm) tensor". ``pack_intersections`` (rasterize.mm:115-145),
which the reference never calls, is not provided.
"""

from __future__ import annotations

import torch

from . import _lib
from .ssim import blur15 as _blur15
from .ssim import chain_backward as _chain_backward
from .ssim import stack_blur_h as _stack_blur_h
from .ssim import tail_backward as _tail_backward
from .ssim import tail_forward as _tail_forward

# The reference kernel's per-pixel stop transmittance (rasterize.metal:149).
_T_MIN = 1e-4

__all__ = ["init", "rasterize_forward", "rasterize_backward", "preprocess_forward",
           "preprocess_backward", "adam_step", "ssim_tail_forward", "ssim_tail_backward",
           "ssim_stack_blur_h", "ssim_blur15", "ssim_chain_backward", "bin_count",
           "bin_write"]


def _dev(t: torch.Tensor, what: str, dtype=torch.float32) -> int:
    return _lib.dev_tensor(t, what, dtype)


def init(src: str = "") -> None:
    """rasterize.mm:196. The reference compiles Metal source here; the gfx950
    code objects are built ahead of time, so this only loads the library and
    checks that it runs on the current device. ``src`` is ignored."""
    _lib.load()


def _check_tile(tile: int) -> None:
    mt = _lib.open_library().mg_max_tile()
    if tile * tile > mt * mt:
        raise RuntimeError(f"tile {tile} needs {tile * tile} threads per threadgroup; "
                           f"rasterize_forward allows at most {mt * mt} on this GPU")


def rasterize_forward(uv, conic, opacity, color, gauss_ids, tile_offsets, W, H, tile, tiles_x):
    """rasterize.mm:79-113 -> [rgb (H,W,3), alpha (H,W), T (H,W), n_contrib
    (H,W) int32]. n_contrib is the per-pixel stop index into gauss_ids that
    rasterize_backward replays from."""
    lib = _lib.load()
    W, H, tile, tiles_x = int(W), int(H), int(tile), int(tiles_x)
    _check_tile(tile)
    dev = uv.device
    rgb = torch.empty(H, W, 3, device=dev)
    alpha = torch.empty(H, W, device=dev)
    T = torch.empty(H, W, device=dev)
    n_contrib = torch.empty(H, W, dtype=torch.int32, device=dev)
    _lib.check(lib.mg_rasterize_forward(
        uv.shape[0], _dev(uv, "input"), _dev(conic, "input"), _dev(opacity, "input"),
        _dev(color, "input"), _dev(gauss_ids, "input", torch.int32),
        _dev(tile_offsets, "input", torch.int32), W, H, tile, tiles_x, _T_MIN, None,
        gauss_ids.numel(), None, 0, rgb.data_ptr(), alpha.data_ptr(), T.data_ptr(),
        n_contrib.data_ptr(), None, None, _lib.stream(uv)))
    return [rgb, alpha, T, n_contrib]


def rasterize_backward(uv, conic, opacity, color, gauss_ids, tile_offsets, final_T, n_contrib,
                       grad_rgb, grad_alpha, W, H, tile, tiles_x, want_absgrad):
    """rasterize.mm:147-194 -> [d_uv (N,2), d_conic (N,3), d_opacity (N,),
    d_color (N,3), d_absuv (N,) or (1,) when want_absgrad is false], each a
    new contiguous tensor. The kernel accumulates them in one 10-float record
    per Gaussian; the five tensors are copied out of it."""
    lib = _lib.load()
    W, H, tile, tiles_x = int(W), int(H), int(tile), int(tiles_x)
    _check_tile(tile)
    N = uv.shape[0]
    dev = uv.device
    rec = torch.empty(N, 10, device=dev)
    grad_rgb = grad_rgb.contiguous()
    grad_alpha = grad_alpha.contiguous()
    _lib.check(lib.mg_rasterize_backward(
        N, _dev(uv, "input"), _dev(conic, "input"), _dev(opacity, "input"),
        _dev(color, "input"), _dev(gauss_ids, "input", torch.int32),
        _dev(tile_offsets, "input", torch.int32), _dev(final_T, "final_T"),
        _dev(n_contrib, "n_contrib", torch.int32), _dev(grad_rgb, "grad_rgb"),
        _dev(grad_alpha, "grad_alpha"), None, None, gauss_ids.numel(), None, 0, W, H, tile,
        tiles_x, rec.data_ptr(), int(bool(want_absgrad)), 0, None, _lib.stream(uv)))
    d_absuv = rec[:, 9].contiguous() if want_absgrad else torch.zeros(1, device=dev)
    return [rec[:, 0:2].contiguous(), rec[:, 2:5].contiguous(), rec[:, 5].contiguous(),
            rec[:, 6:9].contiguous(), d_absuv]


def _sh_layout(sh, sh_rest):
    """(fused, sh, rest) with the reference's layout check (rasterize.mm:214-224):
    sh (N,16,3), or sh (N,1,3) with sh_rest (N,15,3)."""
    fused = sh.dim() == 3 and sh.shape[1] == 16
    if not fused and not (sh.dim() == 3 and sh.shape[1] == 1 and sh_rest is not None and
                          sh_rest.dim() == 3 and sh_rest.shape[1] == 15):
        raise RuntimeError(
            "SH must be either one (N,16,3) tensor or (N,1,3)+(N,15,3); got "
            f"{tuple(sh.shape)} and {None if sh_rest is None else tuple(sh_rest.shape)}")
    return fused, sh.contiguous(), None if fused else sh_rest.contiguous()


def _host_pose(viewmat, cam_center):
    return _lib.host_f32(viewmat), _lib.host_f32(cam_center)


def preprocess_forward(means, quats, scales, sh, sh_rest, opacities, viewmat, fx, fy, cx, cy,
                       W, H, near, far, blur, max_radius, cam_center, sh_degree):
    """rasterize.mm:244-284 -> [uv (N,2), conic (N,3), depth (N,), rxy (N,2),
    valid (N,) int32, color (N,3)]. viewmat (4,4) and cam_center (3,) are read
    on the host, as the reference reads them."""
    lib = _lib.load()
    N = means.shape[0]
    dev = means.device
    fused, sh, rest = _sh_layout(sh, sh_rest)
    means, quats, scales = means.contiguous(), quats.contiguous(), scales.contiguous()
    opacities = opacities.contiguous()
    uv = torch.empty(N, 2, device=dev)
    conic = torch.empty(N, 3, device=dev)
    depth = torch.empty(N, device=dev)
    rxy = torch.empty(N, 2, device=dev)
    valid = torch.empty(N, dtype=torch.int32, device=dev)
    color = torch.empty(N, 3, device=dev)
    vm, cc = _host_pose(viewmat, cam_center)
    _lib.check(lib.mg_preprocess_forward(
        N, _dev(means, "means"), _dev(quats, "quats"), _dev(scales, "scales"), _dev(sh, "sh"),
        None if fused else _dev(rest, "sh_rest"), int(fused), _dev(opacities, "opacities"), vm,
        float(fx), float(fy), float(cx), float(cy), int(W), int(H), float(near), float(far),
        float(blur), float(max_radius), cc, int(sh_degree), uv.data_ptr(), conic.data_ptr(),
        depth.data_ptr(), rxy.data_ptr(), valid.data_ptr(), None, color.data_ptr(),
        _lib.stream(means)))
    return [uv, conic, depth, rxy, valid, color]


def preprocess_backward(means, quats, scales, sh, sh_rest, d_uv, d_conic, d_color, valid,
                        viewmat, fx, fy, cx, cy, W, H, near, far, blur, max_radius, cam_center,
                        sh_degree):
    """rasterize.mm:286-327 -> [d_means (N,3), d_quats (N,4), d_scales (N,3),
    d_sh, d_sh_rest] in the input's SH layout; with one (N,16,3) SH tensor
    d_sh_rest IS d_sh (the same tensor), as in the reference."""
    lib = _lib.load()
    N = means.shape[0]
    dev = means.device
    fused, sh, rest = _sh_layout(sh, sh_rest)
    d_means = torch.empty(N, 3, device=dev)
    d_quats = torch.empty(N, 4, device=dev)
    d_scales = torch.empty(N, 3, device=dev)
    d_sh = torch.empty(N, 16 if fused else 1, 3, device=dev)
    d_sh_rest = d_sh if fused else torch.empty(N, 15, 3, device=dev)
    d_uv, d_conic, d_color = d_uv.contiguous(), d_conic.contiguous(), d_color.contiguous()
    vm, cc = _host_pose(viewmat, cam_center)
    _lib.check(lib.mg_preprocess_backward(
        N, _dev(means.contiguous(), "means"), _dev(quats.contiguous(), "quats"),
        _dev(scales.contiguous(), "scales"), _dev(sh, "sh"),
        None if fused else _dev(rest, "sh_rest"), int(fused), _dev(d_uv, "d_uv"),
        _dev(d_conic, "d_conic"), _dev(d_color, "d_color"), 0,
        _dev(valid.contiguous(), "valid", torch.int32), vm, float(fx), float(fy), float(cx),
        float(cy), int(W), int(H), float(near), float(far), float(blur), float(max_radius), cc,
        int(sh_degree), d_means.data_ptr(), d_quats.data_ptr(), d_scales.data_ptr(),
        d_sh.data_ptr(), None if fused else d_sh_rest.data_ptr(), _lib.stream(means)))
    return [d_means, d_quats, d_scales, d_sh, d_sh_rest]


def adam_step(p, g, m, v, lr, b1, b2, eps, step):
    """rasterize.mm:329-360: one Adam step of p, m, v in place (contiguous,
    same number of elements as g)."""
    lib = _lib.load()
    n = p.numel()
    if g.numel() != n or m.numel() != n or v.numel() != n:
        raise RuntimeError("adam_step: parameter/grad/moment numel mismatch")
    if n == 0:
        return
    _lib.check(lib.mg_adam_step(_dev(p, "adam tensor"), _dev(g.contiguous(), "adam tensor"),
                                _dev(m, "adam tensor"), _dev(v, "adam tensor"), n, float(lr),
                                float(b1), float(b2), float(eps), int(step), _lib.stream(p)))


def ssim_tail_forward(b, H, W):
    """rasterize.mm:383-389: SSIM map (1,3,H,W) of a blurred (15,H,W) stack."""
    return _tail_forward(b, int(H), int(W))


def ssim_tail_backward(b, gout, H, W):
    """rasterize.mm:391-397: gradient of the blurred stack, shaped like b."""
    return _tail_backward(b, gout, int(H), int(W))


def ssim_stack_blur_h(x, y, w, H, W):
    """rasterize.mm:399-419: the (1,15,H,W) moment stack of two (H,W,3)
    images, blurred along rows by the 11-tap window w."""
    if x.numel() != 3 * H * W or y.numel() != x.numel():
        raise RuntimeError("expected (H,W,3)")
    return _stack_blur_h(x, y, w, int(H), int(W))


def ssim_blur15(src, w, dir, H, W):  # noqa: A002  (the reference's argument name)
    """rasterize.mm:421-440: the 15-channel stack blurred along columns
    (dir 1) or rows (dir 0)."""
    return _blur15(src, w, int(dir), int(H), int(W))


def ssim_chain_backward(x, y, d_stack, H, W):
    """rasterize.mm:442-461: the gradient of x through the moment stack."""
    return _chain_backward(x, y, d_stack, int(H), int(W))


def bin_count(uv, rxy, conic, opacity, valid, W, H, tile, tiles_x, tiles_y):
    """rasterize.mm:485-497 -> counts (N,) int32 of tiles passing the exact
    ellipse test."""
    lib = _lib.load()
    N = uv.shape[0]
    counts = torch.empty(N, dtype=torch.int32, device=uv.device)
    if N == 0:
        return counts
    _lib.check(lib.mg_bin_count(N, _dev(uv, "uv"), _dev(rxy, "rxy"), _dev(conic, "conic"),
                                _dev(opacity, "opacity"), _dev(valid, "valid", torch.int32),
                                int(W), int(H), int(tile), int(tiles_x), int(tiles_y),
                                counts.data_ptr(), _lib.stream(uv)))
    return counts


def bin_write(uv, rxy, conic, opacity, valid, depth, offsets, total, W, H, tile, tiles_x,
              tiles_y):
    """rasterize.mm:499-516 -> [keys (total,) int64 = (tile << 32) | depth
    bits, ids (total,) int32], one pair per surviving (Gaussian, tile) at the
    Gaussian's offset, rows then columns."""
    lib = _lib.load()
    N = uv.shape[0]
    total = int(total)
    keys = torch.empty(total, dtype=torch.int64, device=uv.device)
    ids = torch.empty(total, dtype=torch.int32, device=uv.device)
    if total == 0 or N == 0:
        return [keys, ids]
    _lib.check(lib.mg_bin_write(N, _dev(uv, "uv"), _dev(rxy, "rxy"), _dev(conic, "conic"),
                                _dev(opacity, "opacity"), _dev(valid, "valid", torch.int32),
                                _dev(depth, "depth"), _dev(offsets, "offsets", torch.int32),
                                total, int(W), int(H), int(tile), int(tiles_x), int(tiles_y),
                                keys.data_ptr(), ids.data_ptr(), _lib.stream(uv)))
    return [keys, ids]
