"""Pins oracle/adam_ref.py, oracle/ssim_ref.py and oracle/raster_seq.c.

Adam: step-1 closed form, torch.optim.Adam over 30 and 101 steps, and the
selective variant against a float64 per-row brute force (each row runs plain
Adam over exactly its visible steps with its own step count).
SSIM: SSIM(a, a) = 1, the separable zero-padded blur against a direct 11x11
2-D convolution, float64 gradcheck.
Raster contract (C): forward against the torch restatement of torch_ref on
the same tile lists with every Gaussian composited, backward against torch
autograd of that restatement.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import intrinsics, rel_l2, scene
from oracle import adam_ref, raster_ref, render_ref, ssim_ref


# -------------------------------------------------------------------- Adam

def test_adam_step_one_closed_form():
    g = np.random.default_rng(0)
    p = g.normal(size=1000).astype(np.float32)
    grad = (g.normal(size=1000) * 1e-3).astype(np.float32)
    p0 = p.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    adam_ref.adam_step(p, grad, m, v, 1e-3, 0.9, 0.999, 1e-15, 1)
    want = p0 - 1e-3 * grad / (np.abs(grad) + 1e-15)
    assert np.abs(p - want).max() <= 2 * np.finfo(np.float32).eps * np.abs(p0).max()


@pytest.mark.parametrize("steps", [30, 101])
def test_adam_matches_torch(steps):
    g = torch.Generator().manual_seed(7)
    t = torch.randn(3000, generator=g)
    a = t.clone().requires_grad_(True)
    opt = torch.optim.Adam([a], lr=2e-3, eps=1e-15)
    p, m, v = t.numpy().copy(), np.zeros(3000, np.float32), np.zeros(3000, np.float32)
    for k in range(1, steps + 1):
        gr = torch.randn(3000, generator=g) * 1e-2
        a.grad = gr.clone()
        opt.step()
        adam_ref.adam_step(p, gr.numpy(), m, v, 2e-3, 0.9, 0.999, 1e-15, k)
    assert np.abs(a.detach().numpy() - p).max() / np.abs(p).max() < 1e-6


def test_selective_adam_matches_per_row_brute_force():
    rows, width, steps = 200, 3, 15
    g = np.random.default_rng(1)
    p0 = g.normal(size=(rows, width)).astype(np.float32)
    grads = (g.normal(size=(steps, rows, width)) * 1e-3).astype(np.float32)
    vis = g.random(size=(steps, rows - 20)) < 0.6           # 20 rows of padding
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    st = np.zeros(rows, np.float32)
    lr, b1, b2, eps = 1e-2, 0.9, 0.999, 1e-15
    for k in range(steps):
        adam_ref.selective_adam_step(p, grads[k], m, v, st, vis[k], lr, b1, b2, eps)
    for r in range(rows):
        pr, mr, vr, n = p0[r].astype(np.float64), np.zeros(width), np.zeros(width), 0
        for k in range(steps):
            if r < rows - 20 and vis[k, r]:
                n += 1
                gk = grads[k, r].astype(np.float64)
                mr = b1 * mr + (1 - b1) * gk
                vr = b2 * vr + (1 - b2) * gk * gk
                pr = pr - lr * math.sqrt(1 - b2 ** n) / (1 - b1 ** n) * mr / (np.sqrt(vr) + eps)
        assert st[r] == n
        assert np.abs(p[r] - pr).max() < 2e-6 * max(1.0, np.abs(pr).max())
    assert np.array_equal(p[rows - 20:], p0[rows - 20:])


# -------------------------------------------------------------------- SSIM

def test_ssim_of_an_image_with_itself_is_one():
    a = torch.rand(40, 50, 3, generator=torch.Generator().manual_seed(0)).double()
    assert abs(ssim_ref.ssim(a, a).item() - 1.0) < 1e-12


def test_separable_blur_equals_direct_2d_convolution():
    g = torch.Generator().manual_seed(1)
    img = torch.rand(1, 2, 23, 31, generator=g).double()
    w = ssim_ref.window(dtype=torch.float64)
    got = ssim_ref._blur(img, w)
    k2 = torch.outer(w, w)
    want = torch.zeros_like(img)
    H, W = img.shape[2:]
    for y in range(H):
        for x in range(W):
            for dy in range(-5, 6):
                for dx in range(-5, 6):
                    yy, xx = y + dy, x + dx
                    if 0 <= yy < H and 0 <= xx < W:
                        want[0, :, y, x] += k2[dy + 5, dx + 5] * img[0, :, yy, xx]
    assert (got - want).abs().max() < 1e-12


def _scipy_window():
    """The 11-tap sigma-1.5 Gaussian from scipy's own window routine,
    normalised: an implementation independent of ssim_ref.window."""
    from scipy.signal import windows

    w = windows.gaussian(11, std=1.5, sym=True)
    return torch.from_numpy(w / w.sum())


def test_ssim_window_is_the_sigma_1_5_gaussian():
    """train.py:40-49: 11 taps, sigma 1.5. Against scipy's Gaussian window,
    and its discrete second moment sum k^2 w_k is sigma^2 = 2.25 up to the
    truncation at +-5 taps (a window of sigma 1.0 or 2.0 gives about 1.0 or
    3.4)."""
    w = ssim_ref.window(dtype=torch.float64)
    assert (w - _scipy_window()).abs().max() < 1e-15
    k = torch.arange(-5, 6, dtype=torch.float64)
    m2 = float((k * k * w).sum())
    assert abs(m2 - 2.25) < 0.05, m2
    assert abs(float(w.sum()) - 1.0) < 1e-15


def _interior(t, r=5):
    return t[..., r:-r, r:-r]


def test_ssim_constants_from_constant_images():
    """Constant images a = alpha, b = beta: away from the zero-padded border
    the local variances and covariance vanish, so SSIM = (2 alpha beta + C1) /
    (alpha^2 + beta^2 + C1) with C1 = (0.01 L)^2, L = 1 (Wang et al. 2004,
    the constants of ssim.py:35-36). With alpha, beta of order 0.01 a C1 off
    by a factor of two moves the value in the second digit."""
    for alpha, beta in ((0.01, 0.02), (0.3, 0.7), (0.05, 0.05)):
        a = torch.full((24, 30, 3), alpha, dtype=torch.float64)
        b = torch.full((24, 30, 3), beta, dtype=torch.float64)
        got = _interior(ssim_ref.ssim_map(a, b))
        want = (2 * alpha * beta + 1e-4) / (alpha ** 2 + beta ** 2 + 1e-4)
        assert (got - want).abs().max() < 1e-12, (alpha, beta)


def test_ssim_c2_from_a_checkerboard_pair():
    """x = mu + s c, y = mu + t c with c = (-1)^(i+j): with rho = sum_k w_k
    (-1)^k of the window, the interior moments are mu_x = mu + s rho^2 c,
    var_x = s^2 (1 - rho^4), var_y = t^2 (1 - rho^4), cov = s t (1 - rho^4),
    so SSIM = (2 mu_x mu_y + C1)(2 cov + C2) / ((mu_x^2 + mu_y^2 + C1)
    (var_x + var_y + C2)) with C2 = (0.03 L)^2. s = 0.01, t = 0.03 give 0.79
    with that C2 and 0.64 with C2 = 1e-4."""
    w = _scipy_window()
    rho = float((w * torch.tensor([(-1.0) ** k for k in range(11)], dtype=torch.float64)).sum())
    mu, s, t = 0.4, 0.01, 0.03
    i = torch.arange(26, dtype=torch.float64)[:, None]
    j = torch.arange(33, dtype=torch.float64)[None, :]
    c = 1.0 - 2.0 * ((i + j) % 2)
    a = (mu + s * c)[..., None].expand(26, 33, 3).contiguous()
    b = (mu + t * c)[..., None].expand(26, 33, 3).contiguous()
    got = _interior(ssim_ref.ssim_map(a, b))[0, 0]
    mx, my = mu + s * rho ** 2 * c, mu + t * rho ** 2 * c
    q = 1 - rho ** 4
    want = ((2 * mx * my + 1e-4) * (2 * s * t * q + 9e-4)) / \
        ((mx * mx + my * my + 1e-4) * ((s * s + t * t) * q + 9e-4))
    assert (got - _interior(want)).abs().max() < 1e-12


def test_ssim_window_second_moment_from_a_ramp_pair():
    """Horizontal ramps x = a j, y = b j: the window is symmetric and sums to
    1, so the interior means stay a j and b j while var_x = a^2 m2, var_y =
    b^2 m2, cov = a b m2 with m2 = sum_k k^2 w_k of the (scipy) window. The
    closed form pins the window's width inside the SSIM itself."""
    w = _scipy_window()
    m2 = float((torch.arange(-5, 6, dtype=torch.float64) ** 2 * w).sum())
    ca, cb = 0.01, 0.015
    j = torch.arange(40, dtype=torch.float64)[None, :].expand(20, 40)
    a = (ca * j)[..., None].expand(20, 40, 3).contiguous()
    b = (cb * j)[..., None].expand(20, 40, 3).contiguous()
    got = _interior(ssim_ref.ssim_map(a, b))[0, 0]
    jj = _interior(j)
    want = ((2 * ca * cb * jj * jj + 1e-4) * (2 * ca * cb * m2 + 9e-4)) / \
        (((ca * ca + cb * cb) * jj * jj + 1e-4) * ((ca * ca + cb * cb) * m2 + 9e-4))
    assert (got - want).abs().max() < 1e-12


def test_ssim_gradcheck():
    g = torch.Generator().manual_seed(2)
    a = torch.rand(9, 11, 3, generator=g).double().requires_grad_(True)
    b = torch.rand(9, 11, 3, generator=g).double()
    assert torch.autograd.gradcheck(lambda x: ssim_ref.ssim(x, b), (a,), eps=1e-6, atol=1e-7)


# ------------------------------------------------------ raster contract (C)

def _lists_from_ref(uv, radius, valid, depth, W, H, tile):
    tx, ty, buf, _ = render_ref.tile_lists(uv, radius, valid, depth, W, H, tile)
    ids, offs = [], [0]
    for t in range(tx * ty):
        row = [int(g) for g in buf[t].tolist() if g >= 0]
        ids += row
        offs.append(len(ids))
    return np.array(ids, np.int32), np.array(offs, np.int32)


def _projected(n, seed, W, H, dtype):
    s = scene(n=n, seed=seed)
    K = intrinsics(W, H)
    leaves = {k: s[k].to(dtype) for k in ("means", "quats", "scales", "opacities", "colors")}
    cov = render_ref.build_cov3d(leaves["quats"], leaves["scales"])
    uv, conic, depth, radius, valid, _ = render_ref.project(
        leaves["means"], cov, torch.eye(4, dtype=dtype), float(K[0, 0]), float(K[1, 1]),
        float(K[0, 2]), float(K[1, 2]), W, H, 0.01, 100.0)
    return uv, conic, depth, radius, valid, leaves


@pytest.mark.parametrize("tile", [8, 16])
def test_c_forward_matches_the_torch_restatement(tile):
    W, H = 72, 56
    uv, conic, depth, radius, valid, lv = _projected(400, 5, W, H, torch.float64)
    ids, offs = _lists_from_ref(uv, radius, valid, depth, W, H, tile)
    rgb, alpha, _ = render_ref.rasterize(uv, conic, lv["opacities"], lv["colors"], depth, radius,
                                         valid, W, H, tile=tile, min_transmittance=0.0)
    c = raster_ref.forward(uv.numpy(), conic.numpy(), lv["opacities"].numpy(),
                           lv["colors"].numpy(), ids, offs, W, H, tile, t_min=0.0)
    ok = ~c[4]
    assert c[4].mean() < 1e-2
    assert np.abs(c[0] - rgb.numpy())[ok].max() < 2e-5
    assert np.abs(c[1] - alpha.numpy())[ok].max() < 2e-5


def test_c_backward_matches_autograd_of_the_restatement():
    W, H, tile = 64, 48, 16
    uv, conic, depth, radius, valid, lv = _projected(300, 6, W, H, torch.float64)
    uv, conic = uv.detach().requires_grad_(True), conic.detach().requires_grad_(True)
    op = lv["opacities"].clone().requires_grad_(True)
    col = lv["colors"].clone().requires_grad_(True)
    ids, offs = _lists_from_ref(uv.detach(), radius, valid, depth, W, H, tile)
    rgb, alpha, _ = render_ref.rasterize(uv, conic, op, col, depth, radius, valid, W, H,
                                         tile=tile, min_transmittance=0.0)
    g = torch.Generator().manual_seed(0)
    grgb = torch.randn(H, W, 3, generator=g).double()
    galpha = torch.randn(H, W, generator=g).double()
    torch.autograd.backward([rgb, alpha], [grgb, galpha])
    f = raster_ref.forward(uv.detach().numpy(), conic.detach().numpy(), op.detach().numpy(),
                           col.detach().numpy(), ids, offs, W, H, tile, t_min=0.0)
    d = raster_ref.backward(uv.detach().numpy(), conic.detach().numpy(), op.detach().numpy(),
                            col.detach().numpy(), ids, offs, f[2], f[3], grgb.numpy(),
                            galpha.numpy(), W, H, tile)
    for name, got, want in zip(("uv", "conic", "opacity", "color"), d[:4],
                               (uv.grad, conic.grad, op.grad, col.grad)):
        assert rel_l2(got, want) < 1e-4, f"{name}: {rel_l2(got, want):.2e}"


def test_c_forward_stops_at_t_min_and_reports_the_stop_index():
    """Two stacked opaque splats: the pixel under both stops after the second
    (T = 0.001^2 < 1e-4) and its stop index is 2."""
    W = H = 16
    uv = np.array([[8.0, 8.0], [8.0, 8.0], [8.0, 8.0]], np.float32)
    conic = np.array([[0.01, 0.0, 0.01]] * 3, np.float32)
    op = np.array([1.0, 1.0, 1.0], np.float32)
    col = np.eye(3, dtype=np.float32)
    ids = np.array([0, 1, 2], np.int32)
    offs = np.array([0, 3], np.int32)
    rgb, alpha, T, stop, _ = raster_ref.forward(uv, conic, op, col, ids, offs, W, H, 16, 1e-4)
    assert stop[8, 8] == 2 and T[8, 8] < 1e-4
    assert rgb[8, 8, 2] == 0.0                  # the third splat never blends
