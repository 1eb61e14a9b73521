"""Fused SSIM loss on the GPU (11-tap Gaussian window, sigma 1.5).

The reference computes SSIM for the loss with five Metal kernels driven from
``train._SSIMFused`` (metal_gauss/train.py:52-105): stack + horizontal blur,
vertical blur, tail; and in the backward tail adjoint, two blurs and a chain
kernel. Here the forward is one LDS-tiled kernel that produces the mean SSIM
and the three adjoint maps, and the backward is one kernel that blurs them and
chains through the moments (mg_ssim_fused_forward / _backward). The five
kernels of the reference's ABI are also exported (``stack_blur_h``,
``blur15``, ``tail_forward``, ``tail_backward``, ``chain_backward``) for
callers that drive them directly.
"""

from __future__ import annotations

import torch

from . import _lib


def gaussian_kernel(size: int = 11, sigma: float = 1.5, device="cuda", groups: int = 1):
    """Normalised 1-D Gaussian window shaped (groups, 1, 1, size) (ssim.py:29-32)."""
    x = torch.arange(size, dtype=torch.float32, device=device) - size // 2
    g = torch.exp(-x ** 2 / (2 * sigma ** 2))
    return (g / g.sum()).view(1, 1, 1, size).expand(groups, 1, 1, size).contiguous()


def _gaussian_kernel(size: int = 11, sigma: float = 1.5, device="cuda", groups: int = 15):
    """The trainer's 15-group window (train.py:40-49)."""
    return gaussian_kernel(size, sigma, device, groups)


def _check_image(t: torch.Tensor, what: str) -> None:
    if t.dim() != 3 or t.shape[2] != 3:
        raise ValueError(f"{what} must be (H,W,3), got {tuple(t.shape)}")


class _SSIMFused(torch.autograd.Function):
    """Mean SSIM of a (H,W,3) render against a target; gradient to the render."""

    @staticmethod
    def forward(ctx, a, b, w):
        lib = _lib.load()
        _check_image(a, "render")
        _check_image(b, "target")
        a, b = a.contiguous(), b.contiguous()
        w = w.reshape(-1).contiguous().to(torch.float32)
        if w.numel() != 11:
            raise ValueError(f"SSIM window must have 11 taps, got {w.numel()}")
        H, W = a.shape[0], a.shape[1]
        partials = torch.empty(9, H, W, device=a.device)
        mean = torch.empty((), device=a.device)
        ws = torch.empty(lib.mg_ssim_fused_workspace_bytes(H, W), dtype=torch.uint8,
                         device=a.device)
        _lib.check(lib.mg_ssim_fused_forward(
            _lib.dev_tensor(a, "render"), _lib.dev_tensor(b, "target"),
            _lib.dev_tensor(w, "window"), H, W, partials.data_ptr(), mean.data_ptr(),
            ws.data_ptr(), ws.numel(), _lib.stream(a)))
        ctx.save_for_backward(a, b, w, partials)
        return mean

    @staticmethod
    def backward(ctx, grad_out):
        lib = _lib.load()
        a, b, w, partials = ctx.saved_tensors
        H, W = a.shape[0], a.shape[1]
        scale = grad_out.detach().to(torch.float32).reshape(1).contiguous()
        d_a = torch.empty_like(a)
        _lib.check(lib.mg_ssim_fused_backward(
            a.data_ptr(), b.data_ptr(), w.data_ptr(), partials.data_ptr(),
            _lib.dev_tensor(scale, "grad"), H, W, d_a.data_ptr(), _lib.stream(a)))
        return d_a, None, None


class _PhotometricLoss(torch.autograd.Function):
    """(loss, [L1 mean, SSIM mean]) with loss = (1 - w) * mean|a - b| +
    w * (1 - mean SSIM(a, b)). Only the loss carries a gradient (to ``a``);
    the parts are non-differentiable, and no zero gradient is materialised
    for them."""

    @staticmethod
    def forward(ctx, a, b, win, ssim_weight):
        lib = _lib.load()
        _check_image(a, "render")
        _check_image(b, "target")
        a, b = a.contiguous(), b.contiguous()
        win = win.reshape(-1).contiguous().to(torch.float32)
        if win.numel() != 11:
            raise ValueError(f"SSIM window must have 11 taps, got {win.numel()}")
        H, W = a.shape[0], a.shape[1]
        partials = torch.empty(9, H, W, device=a.device)
        out = torch.empty(3, device=a.device)
        ws = torch.empty(lib.mg_ssim_fused_workspace_bytes(H, W), dtype=torch.uint8,
                         device=a.device)
        _lib.check(lib.mg_photometric_loss_forward(
            _lib.dev_tensor(a, "render"), _lib.dev_tensor(b, "target"),
            _lib.dev_tensor(win, "window"), H, W, float(ssim_weight), partials.data_ptr(),
            out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(a)))
        ctx.save_for_backward(a, b, win, partials)
        ctx.ssim_weight = float(ssim_weight)
        ctx.set_materialize_grads(False)
        loss, parts = out[0], out[1:]
        ctx.mark_non_differentiable(parts)
        return loss, parts

    @staticmethod
    def backward(ctx, grad_loss, grad_parts):
        if grad_loss is None:
            return None, None, None, None
        lib = _lib.load()
        a, b, win, partials = ctx.saved_tensors
        H, W = a.shape[0], a.shape[1]
        g = grad_loss.detach().to(torch.float32).reshape(1).contiguous()
        d_a = torch.empty_like(a)
        _lib.check(lib.mg_photometric_loss_backward(
            a.data_ptr(), b.data_ptr(), win.data_ptr(), partials.data_ptr(),
            _lib.dev_tensor(g, "grad"), H, W, ctx.ssim_weight, d_a.data_ptr(), _lib.stream(a)))
        return d_a, None, None, None


def photometric_loss(a: torch.Tensor, b: torch.Tensor, kernel: torch.Tensor,
                     ssim_weight: float = 0.2):
    """The trainer's loss (train.py:389-390) in one fused pass:
    ``(1 - ssim_weight) * (a - b).abs().mean() + ssim_weight * (1 - ssim(a, b))``.

    Returns (loss, parts), where parts is a detached device tensor holding
    [L1 mean, SSIM mean]. Differentiable w.r.t. ``a`` only. The value and the
    gradient equal the two-term torch expression up to float rounding.
    """
    w = kernel.reshape(-1, kernel.shape[-1])[0] if kernel.dim() > 1 else kernel
    return _PhotometricLoss.apply(a, b, w, ssim_weight)


def ssim(a: torch.Tensor, b: torch.Tensor, kernel: torch.Tensor) -> torch.Tensor:
    """Mean SSIM of a, b (H,W,3) in [0,1]; differentiable w.r.t. ``a`` only.

    ``kernel`` is the trainer's window, (groups,1,1,11) or a flat 11-vector
    (train.py:52-64 passes kernel[0, 0, 0]).
    """
    w = kernel.reshape(-1, kernel.shape[-1])[0] if kernel.dim() > 1 else kernel
    return _SSIMFused.apply(a, b, w)


# ------------------------------------------------ the reference's five kernels

def _img_ptrs(*ts):
    return [_lib.dev_tensor(t, "image") for t in ts]


def stack_blur_h(x, y, w, H, W):
    lib = _lib.load()
    out = torch.empty(1, 15, H, W, device=x.device)
    px, py, pw = _img_ptrs(x.contiguous(), y.contiguous(), w.contiguous())
    _lib.check(lib.mg_ssim_stack_blur_h(px, py, pw, H, W, out.data_ptr(), _lib.stream(x)))
    return out


def blur15(src, w, direction, H, W):
    lib = _lib.load()
    src = src.contiguous()
    out = torch.empty_like(src)
    _lib.check(lib.mg_ssim_blur15(_lib.dev_tensor(src, "src"), _lib.dev_tensor(w.contiguous(), "w"),
                                  int(direction), H, W, out.data_ptr(), _lib.stream(src)))
    return out


def tail_forward(b, H, W):
    lib = _lib.load()
    b = b.contiguous()
    if b.numel() != 15 * H * W:
        raise RuntimeError("ssim_tail_forward: expected 15*H*W")
    out = torch.empty(1, 3, H, W, device=b.device)
    _lib.check(lib.mg_ssim_tail_forward(_lib.dev_tensor(b, "blurred stack"), H, W,
                                        out.data_ptr(), _lib.stream(b)))
    return out


def tail_backward(b, gout, H, W):
    lib = _lib.load()
    b, gout = b.contiguous(), gout.contiguous()
    gb = torch.empty_like(b)
    _lib.check(lib.mg_ssim_tail_backward(_lib.dev_tensor(b, "blurred stack"),
                                         _lib.dev_tensor(gout, "grad"), H, W, gb.data_ptr(),
                                         _lib.stream(b)))
    return gb


def chain_backward(x, y, d_stack, H, W):
    lib = _lib.load()
    x, y, d_stack = x.contiguous(), y.contiguous(), d_stack.contiguous()
    d_x = torch.empty_like(x)
    _lib.check(lib.mg_ssim_chain_backward(_lib.dev_tensor(x, "x"), _lib.dev_tensor(y, "y"),
                                          _lib.dev_tensor(d_stack, "d_stack"), H, W,
                                          d_x.data_ptr(), _lib.stream(x)))
    return d_x
