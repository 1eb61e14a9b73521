"""SSIM on the GPU against the F.conv2d expression the reference's own test
uses as oracle (tests/test_fused_ssim.py:19-61; oracle/ssim_ref.py).
Bars: value within 1e-6, gradient max relative error below 1e-4."""

from __future__ import annotations

import pytest
import torch

from oracle import ssim_ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H,W", [(64, 64), (200, 300), (97, 131), (800, 800)])
def test_fused_value_and_gradient(dev, H, W):
    from metal_gauss_amd import gaussian_kernel, ssim

    g = torch.Generator().manual_seed(H * W)
    a = torch.rand(H, W, 3, generator=g)
    b = torch.rand(H, W, 3, generator=g)
    ag = a.to(dev).requires_grad_(True)
    v1 = ssim(ag, b.to(dev), gaussian_kernel(device=dev, groups=15))
    g1, = torch.autograd.grad(v1, ag)
    a2 = a.double().requires_grad_(True)
    v2 = ssim_ref.ssim(a2, b.double(), ssim_ref.window(dtype=torch.float64))
    g2, = torch.autograd.grad(v2, a2)
    assert abs(v1.item() - v2.item()) < 1e-6
    rel = ((g1.cpu().double() - g2).abs().max() / g2.abs().max()).item()
    assert rel < 1e-4, f"gradient rel err {rel:.2e}"


def test_identical_images_give_one(dev):
    from metal_gauss_amd import gaussian_kernel, ssim

    a = torch.rand(80, 80, 3, generator=torch.Generator().manual_seed(3)).to(dev)
    assert abs(ssim(a, a, gaussian_kernel(device=dev)).item() - 1.0) < 1e-5


def test_upstream_gradient_scales_linearly(dev):
    from metal_gauss_amd import gaussian_kernel, ssim

    g = torch.Generator().manual_seed(5)
    a = torch.rand(50, 70, 3, generator=g).to(dev).requires_grad_(True)
    b = torch.rand(50, 70, 3, generator=g).to(dev)
    w = gaussian_kernel(device=dev)
    g1, = torch.autograd.grad(ssim(a, b, w), a)
    g3, = torch.autograd.grad(-3.0 * ssim(a, b, w), a)
    assert torch.allclose(g3, -3.0 * g1, rtol=1e-5, atol=1e-12)


def test_reference_abi_kernels(dev):
    """The five kernels of the reference ABI compose to the same SSIM and
    gradient (train.py:86-105)."""
    import importlib

    S = importlib.import_module("metal_gauss_amd.ssim")

    H, W = 97, 131
    g = torch.Generator().manual_seed(11)
    a = torch.rand(H, W, 3, generator=g)
    b = torch.rand(H, W, 3, generator=g)
    w = ssim_ref.window().to(dev)
    ad, bd = a.to(dev), b.to(dev)
    inter = S.stack_blur_h(ad, bd, w, H, W)
    blurred = S.blur15(inter, w, 1, H, W)
    smap = S.tail_forward(blurred, H, W)
    want = ssim_ref.ssim_map(a.double(), b.double(), ssim_ref.window(dtype=torch.float64))
    assert float((smap.cpu().double() - want).abs().max()) < 1e-5
    gout = torch.full((1, 3, H, W), 1.0 / (3 * H * W), device=dev)
    d_blur = S.tail_backward(blurred, gout, H, W)
    d_inter = S.blur15(d_blur, w, 1, H, W)
    d_stack = S.blur15(d_inter, w, 0, H, W)
    dx = S.chain_backward(ad, bd, d_stack, H, W)
    a2 = a.double().requires_grad_(True)
    g2, = torch.autograd.grad(ssim_ref.ssim(a2, b.double(), ssim_ref.window(dtype=torch.float64)), a2)
    assert ((dx.cpu().double() - g2).abs().max() / g2.abs().max()).item() < 1e-4


@pytest.mark.parametrize("H,W,lam", [(64, 64, 0.2), (97, 131, 0.2), (800, 800, 0.2),
                                     (50, 70, 0.0), (50, 70, 1.0)])
def test_photometric_loss_matches_the_trainer_expression(dev, H, W, lam):
    """photometric_loss equals (1 - lam) * |a - b|.mean() + lam * (1 - ssim)
    (train.py:389-390), with the SSIM term from the float64 conv2d oracle.
    Value within 1e-6; gradient max error within 1e-4 of its magnitude. Some
    pixels have a == b exactly, so the L1 term's sign(0) = 0 is exercised."""
    from metal_gauss_amd import gaussian_kernel, photometric_loss

    g = torch.Generator().manual_seed(H + W)
    a = torch.rand(H, W, 3, generator=g)
    b = torch.rand(H, W, 3, generator=g)
    b[: H // 4] = a[: H // 4]
    ag = a.to(dev).requires_grad_(True)
    loss, parts = photometric_loss(ag, b.to(dev), gaussian_kernel(device=dev, groups=15), lam)
    g1, = torch.autograd.grad(loss, ag)
    a2 = a.double().requires_grad_(True)
    l1 = (a2 - b.double()).abs().mean()
    s2 = ssim_ref.ssim(a2, b.double(), ssim_ref.window(dtype=torch.float64))
    want = (1.0 - lam) * l1 + lam * (1.0 - s2)
    g2, = torch.autograd.grad(want, a2)
    assert abs(loss.item() - want.item()) < 1e-6
    assert abs(parts[0].item() - l1.item()) < 1e-6
    assert abs(parts[1].item() - s2.item()) < 1e-6
    err = ((g1.cpu().double() - g2).abs().max() / g2.abs().max()).item()
    assert err < 1e-4, f"gradient rel err {err:.2e}"


def test_photometric_loss_upstream_gradient(dev):
    from metal_gauss_amd import gaussian_kernel, photometric_loss

    g = torch.Generator().manual_seed(8)
    a = torch.rand(40, 60, 3, generator=g).to(dev).requires_grad_(True)
    b = torch.rand(40, 60, 3, generator=g).to(dev)
    w = gaussian_kernel(device=dev)
    g1, = torch.autograd.grad(photometric_loss(a, b, w)[0], a)
    g2, = torch.autograd.grad(2.5 * photometric_loss(a, b, w)[0], a)
    assert torch.allclose(g2, 2.5 * g1, rtol=1e-5, atol=1e-12)
