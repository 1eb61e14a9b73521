"""SSIM as the reference's tests define it. TEST INFRASTRUCTURE ONLY.

Restates the F.conv2d expression of metal_gauss/tests/test_fused_ssim.py:19-30
(and ssim.py:54-108): five stacked moments (x, y, x^2, y^2, xy) blurred with
a separable 11-tap Gaussian window (sigma 1.5, train.py:40-49) under zero
padding, then S = (2 mx my + C1)(2 sxy + C2) / ((mx^2 + my^2 + C1)(sxx + syy
+ C2)), mean over pixels and channels. Gradient by torch autograd.

Pinned by tests/test_oracle_adam_ssim_raster.py: SSIM(a, a) = 1; the
separable blur against a direct 11x11 2-D convolution in float64; the window
against scipy's Gaussian window and its second moment sigma^2 = 2.25; C1 by
the closed form of constant images, C2 by that of a checkerboard pair, and
the window's width inside SSIM by that of a ramp pair; float64 gradcheck.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

C1 = 0.01 ** 2
C2 = 0.03 ** 2


def window(size: int = 11, sigma: float = 1.5, dtype=torch.float32) -> torch.Tensor:
    x = torch.arange(size, dtype=dtype) - size // 2
    g = torch.exp(-x ** 2 / (2 * sigma ** 2))
    return g / g.sum()


def _blur(t: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Separable zero-padded blur of a (1,G,H,W) stack."""
    G = t.shape[1]
    k = w.view(1, 1, 1, -1).expand(G, 1, 1, w.numel()).contiguous()
    r = w.numel() // 2
    t = F.conv2d(t, k, padding=(0, r), groups=G)
    return F.conv2d(t, k.transpose(2, 3), padding=(r, 0), groups=G)


def moments(a: torch.Tensor, b: torch.Tensor, w: torch.Tensor):
    """(mx, my, exx, eyy, exy), each (1,3,H,W), for (H,W,3) images."""
    x = a.permute(2, 0, 1)[None]
    y = b.permute(2, 0, 1)[None]
    bl = _blur(torch.cat([x, y, x * x, y * y, x * y], dim=1), w)
    return bl.split(3, dim=1)


def ssim_map(a: torch.Tensor, b: torch.Tensor, w: torch.Tensor | None = None) -> torch.Tensor:
    if w is None:
        w = window(dtype=a.dtype)
    mx, my, exx, eyy, exy = moments(a, b, w)
    sxx, syy, sxy = exx - mx * mx, eyy - my * my, exy - mx * my
    return ((2 * mx * my + C1) * (2 * sxy + C2)) / ((mx * mx + my * my + C1) * (sxx + syy + C2))


def ssim(a: torch.Tensor, b: torch.Tensor, w: torch.Tensor | None = None) -> torch.Tensor:
    return ssim_map(a, b, w).mean()
