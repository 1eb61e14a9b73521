"""The allocation-free loss entry point, mg_photometric_loss_forward_noalloc,
against mg_photometric_loss_forward with a caller workspace, called through
the C ABI: the same kernels on the same inputs, so the loss, its L1 and
SSIM parts and the adjoint maps must be identical. Two calls in a row, the
second on a smaller, ragged image (the static block sums keep the first
call's values beyond the second's range), and a size past the static
scratch's limit refused before anything is launched."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(H, W, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(H, W, 3, generator=g).to(dev)
    y = torch.rand(H, W, 3, generator=g).to(dev)
    return x, y


def test_noalloc_loss_forward_equals_the_workspace_entry(dev):
    from metal_gauss_amd import _lib, gaussian_kernel

    lib = _lib.load()
    win = gaussian_kernel(device=dev).reshape(-1).contiguous()
    for H, W, seed in ((800, 800, 1), (301, 457, 2)):
        x, y = _inputs(H, W, seed, dev)
        s = _lib.stream(x)
        part_a = torch.empty(9, H, W, device=dev)
        out_a = torch.empty(3, device=dev)
        ws = torch.empty(lib.mg_ssim_fused_workspace_bytes(H, W), dtype=torch.uint8, device=dev)
        _lib.check(lib.mg_photometric_loss_forward(
            x.data_ptr(), y.data_ptr(), win.data_ptr(), H, W, 0.2, part_a.data_ptr(),
            out_a.data_ptr(), ws.data_ptr(), ws.numel(), s))
        part_b = torch.full((9, H, W), 7.0, device=dev)
        out_b = torch.full((3,), 7.0, device=dev)
        _lib.check(lib.mg_photometric_loss_forward_noalloc(
            x.data_ptr(), y.data_ptr(), win.data_ptr(), H, W, 0.2, part_b.data_ptr(),
            out_b.data_ptr(), s))
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), (H, W, out_a.tolist(), out_b.tolist())
        assert torch.equal(part_a, part_b), (H, W)
        l1 = (x - y).abs().mean().item()
        assert abs(out_b[1].item() - l1) <= 1e-6 * l1


def test_noalloc_loss_forward_refuses_images_past_its_scratch(dev):
    from metal_gauss_amd import _lib, gaussian_kernel

    lib = _lib.load()
    win = gaussian_kernel(device=dev).reshape(-1).contiguous()
    x, y = _inputs(16, 32, 3, dev)
    out = torch.zeros(3, device=dev)
    # 8192 x 8192 needs 3 * 256 * 512 block sums, past the 2^18 held: refused
    # on the host, nothing is launched (the pointers are never read).
    rc = lib.mg_photometric_loss_forward_noalloc(
        x.data_ptr(), y.data_ptr(), win.data_ptr(), 8192, 8192, 0.2, x.data_ptr(),
        out.data_ptr(), _lib.stream(x))
    assert rc == 1
    assert "static scratch" in lib.mg_last_error().decode()
    torch.cuda.synchronize()
    assert float(out.abs().max()) == 0.0
