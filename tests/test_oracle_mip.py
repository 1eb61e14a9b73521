"""Pins of oracle/mip_ref.py (CPU): Mip-Splatting's 3D filter and the 2D
antialias factor, each against a computation that does not reuse the
restated formula, plus the reference's own known answers
(tests/test_mipfilter.py, tests/test_antialias.py)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import intrinsics
from oracle import mip_ref as M
from oracle import render_ref as R


def test_filtered_covariance_is_sigma_plus_f2_identity():
    """R diag(s'^2) R^T = R diag(s^2) R^T + f^2 I since R is orthonormal: the
    3D filter convolves with an isotropic Gaussian of variance f^2."""
    g = torch.Generator().manual_seed(0)
    n = 64
    q = torch.randn(n, 4, generator=g).double()
    s = (torch.rand(n, 3, generator=g) * 0.3 + 1e-3).double()
    f = (torch.rand(n, generator=g) * 0.1).double()
    s2, _ = M.apply_3d_filter(s, torch.ones(n, dtype=torch.float64), f)
    want = R.build_cov3d(q, s) + (f ** 2)[:, None, None] * torch.eye(3, dtype=torch.float64)
    assert torch.allclose(R.build_cov3d(q, s2), want, rtol=1e-12, atol=1e-15)


def test_opacity_factor_is_the_determinant_ratio():
    """opacity' / opacity = sqrt(det Sigma / det(Sigma + f^2 I)), from
    torch.linalg.det of the full 3x3 matrices."""
    g = torch.Generator().manual_seed(1)
    n = 64
    q = torch.randn(n, 4, generator=g).double()
    s = (torch.rand(n, 3, generator=g) * 0.3 + 1e-2).double()
    f = (torch.rand(n, generator=g) * 0.1).double()
    op = (torch.rand(n, generator=g) * 0.9 + 0.05).double()
    _, op2 = M.apply_3d_filter(s, op, f)
    sig = R.build_cov3d(q, s)
    sigf = sig + (f ** 2)[:, None, None] * torch.eye(3, dtype=torch.float64)
    want = op * torch.sqrt(torch.linalg.det(sig) / torch.linalg.det(sigf))
    assert torch.allclose(op2, want, rtol=1e-10)


def test_reference_known_answers_of_the_3d_filter():
    """tests/test_mipfilter.py:33-105."""
    s = torch.tensor([[0.10, 0.20, 0.30]], dtype=torch.float64)
    o = torch.tensor([0.8], dtype=torch.float64)
    f = torch.tensor([0.05], dtype=torch.float64)
    ns, no = M.apply_3d_filter(s, o, f)
    assert torch.allclose(ns ** 2, s ** 2 + f ** 2)
    assert torch.allclose(no, (0.8 * torch.sqrt((s ** 2).prod() / (s ** 2 + f ** 2).prod()))[None])
    z = torch.zeros(8, dtype=torch.float64)
    s8 = torch.rand(8, 3, dtype=torch.float64) + 0.01
    o8 = torch.rand(8, dtype=torch.float64)
    ns, no = M.apply_3d_filter(s8, o8, z)
    assert torch.allclose(ns, s8) and torch.allclose(no, o8)
    tiny, big = torch.full((1, 3), 1e-3, dtype=torch.float64), torch.full((1, 3), 1.0,
                                                                           dtype=torch.float64)
    one = torch.ones(1, dtype=torch.float64)
    assert M.apply_3d_filter(tiny, one, f)[1].item() < 0.01
    assert M.apply_3d_filter(big, one, f)[1].item() > 0.99


def test_antialias_factor_matches_autograd_jacobian_determinants():
    """The factor of torch_ref.py:100-124 against det(J Sigma J^T) with J
    from autograd of the perspective map (no closed-form Jacobian reused)."""
    g = torch.Generator().manual_seed(4)
    n = 12
    means = (torch.randn(n, 3, generator=g) * 0.3 + torch.tensor([0.0, 0.0, 3.0])).double()
    sig = R.build_cov3d(torch.randn(n, 4, generator=g).double(),
                        (torch.rand(n, 3, generator=g) * 0.01 + 0.002).double())
    fx, fy, W, H, blur = 300.0, 280.0, 640, 480, 0.3
    vm = torch.eye(4, dtype=torch.float64)
    _, _, cov = R._cov2d(means, sig, vm, fx, fy, W, H, 0.01)
    got = M.antialias_factor(cov, blur)

    def uv_of(p):
        return torch.stack([fx * p[0] / p[2], fy * p[1] / p[2]])

    for i in range(n):
        J = torch.autograd.functional.jacobian(uv_of, means[i])
        c2 = J @ sig[i] @ J.T
        want = math.sqrt(torch.linalg.det(c2).item() /
                         torch.linalg.det(c2 + blur * torch.eye(2, dtype=torch.float64)).item())
        assert got[i].item() == pytest.approx(want, rel=1e-9)


def test_antialias_factor_isotropic_closed_form():
    """An isotropic 2D covariance sigma^2 I: the factor is sigma^2 / (sigma^2 + blur)."""
    s2 = torch.tensor([0.01, 0.3, 2.0, 100.0], dtype=torch.float64)
    cov = torch.zeros(4, 2, 2, dtype=torch.float64)
    cov[:, 0, 0] = cov[:, 1, 1] = s2
    got = M.antialias_factor(cov, 0.3)
    assert torch.allclose(got, s2 / (s2 + 0.3), rtol=1e-14)
    assert torch.allclose(M.antialias_factor(cov, 0.0), torch.ones(4, dtype=torch.float64))


def test_preprocess_mip_matches_render_project():
    """preprocess_mip's effective opacity equals opacity * project's
    opacity_scale (render_ref.project, torch_ref.py:49-144) on filtered inputs."""
    g = torch.Generator().manual_seed(2)
    n, W, H = 200, 64, 48
    means = (torch.randn(n, 3, generator=g) * 0.5 + torch.tensor([0.0, 0.0, 4.0])).double()
    quats = torch.randn(n, 4, generator=g).double()
    scales = (torch.rand(n, 3, generator=g) * 0.03 + 0.004).double()
    op = (torch.rand(n, generator=g) * 0.7 + 0.15).double()
    f = (torch.rand(n, generator=g) * 0.01).double()
    K = intrinsics(W, H).double()
    vm = torch.eye(4, dtype=torch.float64)
    fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])
    out = M.preprocess_mip(means, quats, scales, op, None, vm, fx, fy, cx, cy, W, H,
                           filter_3d=f, antialias=True)
    s2, o2 = M.apply_3d_filter(scales, op, f)
    *_, scale = R.project(means, R.build_cov3d(quats, s2), vm, fx, fy, cx, cy, W, H, 0.01, 100.0,
                          antialias=True)
    assert torch.allclose(out[6], o2 * scale, rtol=1e-12)
    assert bool((out[6] <= op + 1e-15).all())


class _View:
    """The reference's test camera (tests/test_mipfilter.py:23-31): identity
    rotation, pushed back by z along +z."""

    def __init__(self, z, f=1000.0, hw=(400, 400)):
        self.K = np.array([[f, 0, hw[1] / 2], [0, f, hw[0] / 2], [0, 0, 1.0]])
        self.vm = np.eye(4)
        self.vm[2, 3] = z
        self.W, self.H = hw[1], hw[0]

    def tup(self):
        return self.K, self.vm, self.W, self.H


def test_3d_filter_on_axis_closed_form():
    """A Gaussian on the optical axis at camera depth d, one view of focal f:
    d / f * sqrt(0.2)."""
    means = np.array([[0.0, 0.0, 0.0], [0.0, 0.0, 3.0]])
    got = M.compute_3d_filter(means, [_View(5.0, f=800.0).tup()])
    assert got == pytest.approx(np.array([5.0, 8.0]) / 800.0 * math.sqrt(0.2), rel=1e-15)


def test_3d_filter_reference_known_answers():
    """tests/test_mipfilter.py:108-144: farther -> larger; sharper camera ->
    smaller; unseen -> the largest seen distance, finite and positive; min
    over views."""
    m = np.array([[0.0, 0.0, 0.0], [0.0, 0.0, 3.0]])
    f = M.compute_3d_filter(m, [_View(5.0).tup()])
    assert f[1] > f[0] > 0
    lo = M.compute_3d_filter(np.zeros((1, 3)), [_View(5.0, f=500.0).tup()])
    hi = M.compute_3d_filter(np.zeros((1, 3)), [_View(5.0, f=2000.0).tup()])
    assert hi[0] < lo[0]
    m = np.array([[0.0, 0.0, 0.0], [0.0, 0.0, -100.0]])   # the second is behind the camera
    f = M.compute_3d_filter(m, [_View(5.0).tup()])
    assert np.isfinite(f).all() and (f > 0).all() and f[1] == f[0]
    # Two views: the nearer one decides; focal is the larger of the two.
    f2 = M.compute_3d_filter(np.zeros((1, 3)), [_View(5.0, f=500.0).tup(),
                                                _View(2.0, f=1000.0).tup()])
    assert f2[0] == pytest.approx(2.0 / 1000.0 * math.sqrt(0.2), rel=1e-15)
    # None seen: every distance is 1.
    f3 = M.compute_3d_filter(np.array([[0.0, 0.0, -50.0]]), [_View(5.0, f=400.0).tup()])
    assert f3[0] == pytest.approx(1.0 / 400.0 * math.sqrt(0.2), rel=1e-15)
