"""Pins oracle/render_ref.py (the CPU restatement of torch_ref.py / sh.py).

Each check is chosen so a plausible restatement mistake fails it:
  * known answers of tests/test_torch_ref.py:36-147, 255-284 (principal point,
    occlusion, culling, opacity linearity, clamp, area, translation, off-axis);
  * float64 gradcheck on the reference's own 2-Gaussian 12x12 scene;
  * an independent per-pixel float64 loop (sequential compositing written
    from the definition) - catches a wrong cumprod/exclusive product, a
    dropped transmittance carry, or a wrong cutoff;
  * the SH basis against scipy's complex spherical harmonics - catches any
    wrong constant, sign or polynomial;
  * the EWA covariance against J Sigma J^T with J from autograd of the
    perspective map - catches a transposed or wrong closed-form Jacobian;
  * the preprocess contract's SnugBox extents against a direct level-set
    computation.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import intrinsics
from oracle import render_ref as R


def one(z=3.0, scale=0.15, opacity=1.0, color=(1, 0, 0), dtype=torch.float32):
    return (torch.tensor([[0.0, 0.0, z]], dtype=dtype), torch.tensor([[1.0, 0, 0, 0]], dtype=dtype),
            torch.full((1, 3), scale, dtype=dtype), torch.tensor([opacity], dtype=dtype),
            torch.tensor([color], dtype=dtype))


def rend(m, q, s, o, c, W, H, vm=None, **kw):
    return R.render(m, q, s, o, None, intrinsics(W, H), torch.eye(4) if vm is None else vm, W, H,
                    colors=c, **kw)


def test_single_gaussian_lands_at_principal_point():
    W = H = 64
    rgb, alpha, info = rend(*one(), W, H)
    assert info["visible_gaussians"] == 1
    peak = torch.nonzero(alpha == alpha.max())[0]
    assert abs(peak[0].item() - H / 2) <= 1 and abs(peak[1].item() - W / 2) <= 1
    assert alpha.max() > 0.9 and alpha[0, 0] < 1e-3
    assert rgb[H // 2, W // 2, 0] > 0.9 and rgb[H // 2, W // 2, 2] < 1e-3


def test_front_occludes_back():
    W = H = 32
    means = torch.tensor([[0.0, 0.0, 5.0], [0.0, 0.0, 2.0]])
    rgb, _, _ = rend(means, torch.tensor([[1.0, 0, 0, 0]] * 2), torch.full((2, 3), 0.3),
                     torch.tensor([1.0, 1.0]), torch.tensor([[0.0, 0, 1], [1.0, 0, 0]]), W, H)
    c = rgb[H // 2, W // 2]
    assert c[0] > 0.9 and c[2] < 0.1


def test_behind_camera_is_culled():
    _, alpha, info = rend(*one(z=-3.0), 32, 32)
    assert info["visible_gaussians"] == 0 and alpha.max() == 0


def test_alpha_is_linear_in_opacity():
    peaks = [rend(*one(opacity=op), 32, 32)[1].max().item() for op in (0.25, 0.5, 1.0)]
    ratios = [p / o for p, o in zip(peaks, (0.25, 0.5, 1.0))]
    assert max(ratios) - min(ratios) < 1e-5


def test_alpha_saturates_at_the_clamp():
    _, alpha, _ = rend(*one(scale=0.5), 128, 128)
    assert alpha.max().item() == pytest.approx(0.999, abs=1e-3)


def test_farther_gaussian_is_smaller():
    areas = [(rend(*one(z=z), 64, 64)[1] > 0.05).sum().item() for z in (2.0, 4.0)]
    assert areas[0] > areas[1] * 2.5


def test_translating_camera_moves_the_splat():
    vm = torch.eye(4)
    vm[0, 3] = 0.5
    _, alpha, _ = rend(*one(), 64, 64, vm=vm)
    assert torch.nonzero(alpha == alpha.max())[0][1].item() > 64 / 2 + 2


def test_near_offaxis_gaussian_is_rejected_and_finite():
    K = intrinsics(128, 128)
    means = torch.tensor([[6.0, -4.0, 0.02], [0.0, 0.0, 3.0]])
    cov = R.build_cov3d(torch.tensor([[1.0, 0, 0, 0]] * 2), torch.full((2, 3), 0.1))
    _, _, _, radius, valid, _ = R.project(means, cov, torch.eye(4), float(K[0, 0]), float(K[1, 1]),
                                          float(K[0, 2]), float(K[1, 2]), 128, 128, 0.01, 100.0)
    assert torch.isfinite(radius).all() and not valid[0] and valid[1]
    assert radius[valid].max() <= 128


def test_gradients_flow_to_every_input():
    W = H = 32
    leaves = [torch.tensor([[0.05, -0.02, 3.0]]), torch.tensor([[1.0, 0.1, 0.0, 0.0]]),
              torch.tensor([[0.2, 0.15, 0.18]]), torch.tensor([0.7]),
              torch.randn(1, 16, 3, generator=torch.Generator().manual_seed(0)) * 0.3]
    for t in leaves:
        t.requires_grad_(True)
    rgb, _, _ = R.render(*leaves, intrinsics(W, H), torch.eye(4), W, H, sh_degree=3)
    rgb.square().mean().backward()
    for t in leaves:
        assert t.grad is not None and torch.isfinite(t.grad).all() and t.grad.abs().sum() > 0


def test_gradcheck_float64():
    """tests/test_torch_ref.py:218-251, the reference's own oracle certificate."""
    W = H = 12
    K = intrinsics(W, H).double()
    vm = torch.eye(4, dtype=torch.float64)
    args = [torch.tensor([[0.03, -0.05, 3.0], [-0.12, 0.08, 2.6]]),
            torch.tensor([[1.0, 0.05, -0.02, 0.03], [0.98, -0.1, 0.05, 0.0]]),
            torch.tensor([[0.22, 0.19, 0.2], [0.17, 0.21, 0.18]]), torch.tensor([0.55, 0.4]),
            torch.tensor([[0.7, 0.2, 0.1], [0.1, 0.3, 0.8]])]
    args = [a.double().requires_grad_(True) for a in args]

    def f(m, q, s, o, c):
        return R.render(m, q, s, o, None, K, vm, W, H, colors=c)[0]

    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6, rtol=1e-4)


def brute_force(means, quats, scales, op, colors, W, H, tile):
    """Per-pixel sequential compositing in float64 from the definition:
    C = sum_i c_i a_i prod_{j<i}(1 - a_j) over the Gaussians whose 3-sigma tile
    box contains the pixel's tile, in depth order; a_i = min(0.999, o_i
    exp(-q/2)), counted only above 1/255."""
    K = intrinsics(W, H).double()
    fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])
    cov = R.build_cov3d(quats.double(), scales.double())
    uv, conic, depth, radius, valid, _ = R.project(means.double(), cov, torch.eye(4).double(),
                                                   fx, fy, cx, cy, W, H, 0.01, 100.0)
    uv, conic, depth, radius = (t.numpy() for t in (uv, conic, depth, radius))
    tx_n = math.ceil(W / tile)
    ty_n = math.ceil(H / tile)
    order = [i for i in np.argsort(depth, kind="stable") if bool(valid[i])]
    img = np.zeros((H, W, 3))
    acc = np.zeros((H, W))
    for py in range(H):
        for px in range(W):
            t_x, t_y = px // tile, py // tile
            T = 1.0
            for i in order:
                x0 = min(max(math.floor((uv[i, 0] - radius[i]) / tile), 0), tx_n - 1)
                x1 = min(max(math.floor((uv[i, 0] + radius[i]) / tile), 0), tx_n - 1)
                y0 = min(max(math.floor((uv[i, 1] - radius[i]) / tile), 0), ty_n - 1)
                y1 = min(max(math.floor((uv[i, 1] + radius[i]) / tile), 0), ty_n - 1)
                if not (x0 <= t_x <= x1 and y0 <= t_y <= y1):
                    continue
                dx, dy = px + 0.5 - uv[i, 0], py + 0.5 - uv[i, 1]
                q = conic[i, 0] * dx * dx + 2 * conic[i, 1] * dx * dy + conic[i, 2] * dy * dy
                a = min(0.999, float(op[i]) * math.exp(-0.5 * q))
                if a <= 1.0 / 255.0:
                    continue
                img[py, px] += a * T * colors[i].double().numpy()
                acc[py, px] += a * T
                T *= 1.0 - a
    return img, acc


@pytest.mark.parametrize("seed,tile", [(0, 4), (1, 8), (2, 16)])
def test_compositing_matches_a_per_pixel_loop(seed, tile):
    from conftest import scene

    W, H = 20, 14
    s = scene(n=25, seed=seed, z=3.0, spread=0.3, scale=(0.03, 0.12))
    img, acc = brute_force(s["means"], s["quats"], s["scales"], s["opacities"], s["colors"], W, H,
                           tile)
    rgb, alpha, _ = R.render(s["means"].double(), s["quats"].double(), s["scales"].double(),
                             s["opacities"].double(), None, intrinsics(W, H).double(),
                             torch.eye(4).double(), W, H, colors=s["colors"].double(), tile=tile,
                             slab=4, min_transmittance=0.0)
    assert np.abs(rgb.numpy() - img).max() < 1e-10
    assert np.abs(alpha.numpy() - acc).max() < 1e-10


def test_slab_transmittance_carry_is_exact():
    """Slab size must not change the result (T carries across slabs)."""
    from conftest import scene

    s = scene(n=200, seed=9, z=3.0, spread=0.2)
    args = [s[k].double() for k in ("means", "quats", "scales", "opacities")]
    outs = [R.render(*args, None, intrinsics(32, 32).double(), torch.eye(4).double(), 32, 32,
                     colors=s["colors"].double(), slab=sl, min_transmittance=0.0)[0]
            for sl in (3, 256)]
    assert (outs[0] - outs[1]).abs().max() < 1e-12


def test_sh_basis_matches_textbook_real_harmonics():
    """Real SH with the Condon-Shortley phase, from scipy's complex Y_l^m:
    Y_{l,0} = Y_l^0, Y_{l,m>0} = sqrt2 (-1)^m Re Y_l^m,
    Y_{l,m<0} = sqrt2 (-1)^m Im Y_l^|m|; basis index l^2 + l + m."""
    sp = pytest.importorskip("scipy.special")
    g = np.random.default_rng(0)
    d = g.normal(size=(64, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    theta = np.arccos(d[:, 2])                 # polar
    phi = np.arctan2(d[:, 1], d[:, 0])         # azimuth
    B = R.sh_basis(3, torch.from_numpy(d)).numpy()
    for l in range(4):
        for m in range(-l, l + 1):
            if hasattr(sp, "sph_harm_y"):
                Y = sp.sph_harm_y(l, abs(m), theta, phi)
            else:
                Y = sp.sph_harm(abs(m), l, phi, theta)
            if m == 0:
                want = Y.real
            elif m > 0:
                want = math.sqrt(2) * (-1) ** m * Y.real
            else:
                want = math.sqrt(2) * (-1) ** m * Y.imag
            got = B[:, l * l + l + m]
            # 3DGS stores the basis with the opposite sign convention for
            # odd m (the .ply format's); magnitudes and shapes must agree.
            sign = np.sign(np.dot(got, want))
            assert np.allclose(got, sign * want, atol=1e-12), (l, m)
            assert sign == (-1.0 if m % 2 else 1.0), (l, m, sign)


def test_ewa_covariance_matches_autograd_jacobian():
    g = torch.Generator().manual_seed(4)
    n = 16
    means = (torch.randn(n, 3, generator=g) * 0.3 + torch.tensor([0.0, 0.0, 3.0])).double()
    cov3d = R.build_cov3d(torch.randn(n, 4, generator=g).double(),
                          (torch.rand(n, 3, generator=g) * 0.2 + 0.05).double())
    ang = 0.3
    vm = torch.eye(4, dtype=torch.float64)
    vm[:3, :3] = torch.tensor([[math.cos(ang), 0, math.sin(ang)], [0, 1, 0],
                               [-math.sin(ang), 0, math.cos(ang)]], dtype=torch.float64)
    vm[:3, 3] = torch.tensor([0.1, -0.2, 0.3], dtype=torch.float64)
    fx, fy, W, H = 300.0, 280.0, 640, 480
    _, _, cov = R._cov2d(means, cov3d, vm, fx, fy, W, H, 0.01)

    def uv_of(p):
        x = vm[:3, :3] @ p + vm[:3, 3]
        return torch.stack([fx * x[0] / x[2], fy * x[1] / x[2]])

    for i in range(n):
        J = torch.autograd.functional.jacobian(uv_of, means[i])      # (2,3), world coords
        want = J @ cov3d[i] @ J.T
        assert torch.allclose(cov[i], want, rtol=1e-9, atol=1e-12)


def test_snugbox_extent_is_the_alpha_level_set():
    """rxy = sqrt(2 ln(255 op) * cov_axis): along x through the centre the
    alpha = 1/255 crossing of op exp(-1/2 q) lies exactly at u +- rx (when the
    3-sigma cap does not bind)."""
    W = H = 64
    means = torch.tensor([[0.0, 0.0, 3.0]], dtype=torch.float64)
    quats = torch.tensor([[0.9, 0.1, 0.3, -0.2]], dtype=torch.float64)
    scales = torch.tensor([[0.05, 0.08, 0.03]], dtype=torch.float64)
    op = torch.tensor([0.2], dtype=torch.float64)   # rs < 3: the 3-sigma cap cannot bind
    K = intrinsics(W, H)
    uv, conic, _, rxy, valid, _ = R.preprocess(means, quats, scales, op, None,
                                               torch.eye(4, dtype=torch.float64), float(K[0, 0]),
                                               float(K[1, 1]), float(K[0, 2]), float(K[1, 2]), W, H)
    assert bool(valid[0])
    a, b, c = conic[0].tolist()
    # On the horizontal line through the centre, q(dx, dy*) minimised over dy
    # is dx^2 (a - b^2/c) = dx^2 / cov_xx; the level set q = 2 ln(255 op).
    cov_xx = c / (a * c - b * b)
    rx_want = math.sqrt(2 * math.log(255 * 0.2) * cov_xx)
    assert rxy[0, 0].item() == pytest.approx(rx_want, rel=1e-9)
