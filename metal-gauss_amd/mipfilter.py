"""Mip-Splatting's 3D smoothing filter (metal_gauss/mipfilter.py).

Same two functions, same arguments and results:

* ``compute_3d_filter(means, views, near=0.2, margin=0.15)`` - per-Gaussian
  low-pass size, min seen depth / max focal * sqrt(0.2) (mipfilter.py:29-73).
  Here one HIP kernel pass over all views (mg_compute_3d_filter) instead of a
  torch loop with one projection per view.
* ``apply_3d_filter(scales, opacities, filter_3d)`` - the reparameterisation
  scales' = sqrt(scales^2 + f^2), opacity * sqrt(prod s^2 / prod s'^2)
  (mipfilter.py:76-93), kept as the reference's torch expression for callers
  that want the filtered tensors themselves (a ply export bakes them in).

For training, pass ``filter_3d`` to ``render`` instead: the projection kernel
applies the filter and its adjoint itself, with no extra passes over the
scales and opacities.
"""

from __future__ import annotations

import torch

from . import _lib


def _view_records(views, near: float, margin: float):
    """(V, 20) float32 per-view records and the largest focal length."""
    rows = []
    focal = 0.0
    for v in views:
        vm = v.viewmat.detach().to("cpu", torch.float64)
        K = v.K.detach().to("cpu", torch.float64)
        H, W = v.image.shape[:2]
        fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])
        rows.append(vm[:3, :3].reshape(-1).tolist() + vm[:3, 3].tolist() +
                    [fx, fy, cx, cy, -margin * W, (1.0 + margin) * W,
                     -margin * H, (1.0 + margin) * H])
        focal = max(focal, fx, fy)
    rec = torch.tensor(rows, dtype=torch.float32) if rows else torch.zeros(0, 20)
    return rec, focal


@torch.no_grad()
def compute_3d_filter(means: torch.Tensor, views, near: float = 0.2,
                      margin: float = 0.15) -> torch.Tensor:
    """Per-Gaussian low-pass scale, one value per Gaussian (mipfilter.py:29-73).

    ``views`` need ``.K``, ``.viewmat`` and an ``.image`` for the frame size.
    A Gaussian seen by no camera gets the largest distance any Gaussian got;
    with none seen at all every distance is 1.
    """
    if means.device.type != "cuda":
        raise RuntimeError(
            f"hip backend requires ROCm (cuda) tensors, got device '{means.device}'. "
            "Refusing to silently move data or fall back to another backend.")
    lib = _lib.load()
    means = means.detach().to(torch.float32).contiguous()
    N = means.shape[0]
    rec, focal = _view_records(views, near, margin)
    rec = rec.to(means.device)
    out = torch.empty(N, device=means.device)
    scratch = torch.empty(1, dtype=torch.int32, device=means.device)
    _lib.check(lib.mg_compute_3d_filter(
        N, _lib.dev_tensor(means, "means"), rec.shape[0],
        rec.data_ptr() if rec.numel() else None, float(focal), float(near), out.data_ptr(),
        scratch.data_ptr(), _lib.stream(means)))
    return out


def apply_3d_filter(scales: torch.Tensor, opacities: torch.Tensor,
                    filter_3d: torch.Tensor):
    """Widen the Gaussians and dim them to match (mipfilter.py:76-93).

    Returns (scales, opacities); differentiable in both, with ``filter_3d`` a
    constant.
    """
    f2 = (filter_3d ** 2).unsqueeze(-1)
    s2 = scales ** 2
    s2f = s2 + f2
    coef = torch.sqrt((s2.prod(dim=-1) / s2f.prod(dim=-1)).clamp(0.0, 1.0))
    return torch.sqrt(s2f), opacities * coef
