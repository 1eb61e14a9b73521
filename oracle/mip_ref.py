"""Restatement of Mip-Splatting's filters. TEST INFRASTRUCTURE ONLY.

* ``apply_3d_filter`` restates metal_gauss/mipfilter.py:76-93 (torch, any
  dtype, differentiable): s' = sqrt(s^2 + f^2), opacity * sqrt(clamp(prod s^2
  / prod s'^2, 0, 1)).
* ``compute_3d_filter`` restates metal_gauss/mipfilter.py:29-73 in numpy
  float64: min depth over the views that see each Gaussian, / max focal,
  * sqrt(0.2); unseen Gaussians take the largest seen depth, none seen gives 1.
* ``preprocess_mip`` is the contract of the fused projection with both
  filters: the 3D filter applied to scales and opacity first (train.py:223-227
  does it before render), the SnugBox extents and validity from that opacity
  (preprocess.metal:180-195 is handed it), then the 2D antialias factor of
  torch_ref.py:100-124 (det of the projected covariance before / after the
  blur), applied after (metal_backend.py:506-511). Returns the preprocess
  outputs plus the effective opacity.

Pinned by tests/test_oracle_mip.py:
  * apply_3d_filter: the filtered covariance R diag(s'^2) R^T equals
    Sigma + f^2 I, and the opacity factor equals sqrt(det Sigma /
    det(Sigma + f^2 I)) from torch.linalg.det; plus the reference's own known
    answers (tests/test_mipfilter.py:33-105);
  * the 2D factor: against sqrt(det(J Sigma J^T) / det(J Sigma J^T + blur I))
    with J from autograd of the projection, and the isotropic closed form
    sigma^2 / (sigma^2 + blur);
  * compute_3d_filter: the on-axis closed form depth / f * sqrt(0.2) and the
    reference's ordering and unseen cases (tests/test_mipfilter.py:108-144).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import render_ref as R


def apply_3d_filter(scales: torch.Tensor, opacities: torch.Tensor, filter_3d: torch.Tensor):
    """mipfilter.py:76-93."""
    f2 = (filter_3d ** 2).unsqueeze(-1)
    s2 = scales ** 2
    s2f = s2 + f2
    coef = torch.sqrt((s2.prod(dim=-1) / s2f.prod(dim=-1)).clamp(0.0, 1.0))
    return torch.sqrt(s2f), opacities * coef


def compute_3d_filter(means, views, near: float = 0.2, margin: float = 0.15) -> np.ndarray:
    """mipfilter.py:29-73, float64. ``views``: iterable of (K (3,3), viewmat
    (4,4), W, H)."""
    m = np.asarray(means, dtype=np.float64)
    n = m.shape[0]
    dist = np.full(n, np.inf)
    seen = np.zeros(n, dtype=bool)
    focal = 0.0
    for K, vm, W, H in views:
        K = np.asarray(K, dtype=np.float64)
        vm = np.asarray(vm, dtype=np.float64)
        pc = m @ vm[:3, :3].T + vm[:3, 3]
        z = pc[:, 2]
        fx, fy, cx, cy = K[0, 0], K[1, 1], K[0, 2], K[1, 2]
        zc = np.maximum(z, 1e-6)
        u = fx * pc[:, 0] / zc + cx
        w = fy * pc[:, 1] / zc + cy
        inview = ((z > near) & (u > -margin * W) & (u < (1.0 + margin) * W)
                  & (w > -margin * H) & (w < (1.0 + margin) * H))
        dist = np.where(inview, np.minimum(dist, z), dist)
        seen |= inview
        focal = max(focal, fx, fy)
    if seen.any():
        dist[~seen] = dist[seen].max()
    else:
        dist[:] = 1.0
    if focal <= 0.0:
        focal = 1.0
    return (dist / focal) * math.sqrt(0.2)


def antialias_factor(cov2d: torch.Tensor, blur: float) -> torch.Tensor:
    """sqrt(clamp(max(det0, 0) / max(det, 1e-12), 0, 1)) of an undilated
    (N,2,2) covariance and its blurred version (torch_ref.py:110-124)."""
    det0 = cov2d[:, 0, 0] * cov2d[:, 1, 1] - cov2d[:, 0, 1] * cov2d[:, 1, 0]
    a = cov2d[:, 0, 0] + blur
    c = cov2d[:, 1, 1] + blur
    b = cov2d[:, 0, 1]
    det = a * c - b * b
    return (det0.clamp_min(0.0) / det.clamp_min(1e-12)).clamp(0.0, 1.0).sqrt()


def preprocess_mip(means, quats, scales, opacities, sh, viewmat, fx, fy, cx, cy, W, H,
                   near=0.01, far=100.0, blur=0.3, max_radius=None, sh_degree=3,
                   filter_3d=None, antialias=False):
    """-> (uv, conic, depth, rxy, valid, color, opacity_eff)."""
    if filter_3d is not None:
        scales, opacities = apply_3d_filter(scales, opacities, filter_3d)
    uv, conic, depth, rxy, valid, color = R.preprocess(
        means, quats, scales, opacities, sh, viewmat, fx, fy, cx, cy, W, H, near=near, far=far,
        blur=blur, max_radius=max_radius, sh_degree=sh_degree)
    op_eff = opacities
    if antialias:
        _, _, cov = R._cov2d(means, R.build_cov3d(quats, scales), viewmat, fx, fy, W, H, near)
        op_eff = opacities * antialias_factor(cov, blur)
    return uv, conic, depth, rxy, valid, color, op_eff
