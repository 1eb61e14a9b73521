"""The reference's extension surface (metal_gauss_amd.ext, what
backend._load() returns) driven through the reference's own call sequences,
against the CPU oracle:

* the tile-list builder's sequence (metal_backend.py:217-285): bin_count,
  cumsum, bin_write, a sort of the 64-bit keys, searchsorted - bit-exact
  against oracle/binning_ref.py (the reference's torch.argsort leaves equal
  keys in no particular order; a stable sort is used here, as the oracle's);
* the trainer's fused SSIM (train.py:86-105): stack_blur_h, blur15, tail
  forward; tail backward, two blur15 adjoints, chain backward - against
  float64 autograd of oracle/ssim_ref.py;
* the projection and raster bridges (metal_backend.py:288-364) as autograd
  Functions over preprocess_forward/backward and rasterize_forward/backward,
  with both SH layouts - image within 1e-4 and gradients within 1e-3
  relative L2 of float64 autograd of oracle/render_ref.py;
* adam_step against oracle/adam_ref.py, and the absgrad slot's shapes.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import intrinsics, rel_l2, scene
from oracle import adam_ref, binning_ref, render_ref, ssim_ref

pytestmark = pytest.mark.gpu


def _ext():
    from metal_gauss_amd import backend

    return backend._load()


def _camera_args(K, vm):
    cam_center = -vm[:3, :3].T @ vm[:3, 3]
    return float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2]), cam_center


def test_load_returns_the_thirteen_functions(dev):
    ext = _ext()
    names = ("init rasterize_forward rasterize_backward preprocess_forward "
             "preprocess_backward adam_step ssim_tail_forward ssim_tail_backward "
             "ssim_stack_blur_h ssim_blur15 ssim_chain_backward bin_count bin_write").split()
    assert all(callable(getattr(ext, n)) for n in names)
    ext.init("")     # the reference passes Metal source; accepted and ignored


def _lists_by_reference_sequence(ext, uv, rxy, depth, valid, conic, opacity, W, H, tile):
    """metal_backend.py:217-285 step by step, through the extension."""
    tx, ty = math.ceil(W / tile), math.ceil(H / tile)
    counts = ext.bin_count(uv.contiguous(), rxy.contiguous(), conic.contiguous(),
                           opacity.contiguous(), valid.to(torch.int32).contiguous(),
                           W, H, tile, tx, ty)
    offs = torch.cumsum(counts, 0, dtype=torch.int64) - counts
    total = int(offs[-1].item()) + int(counts[-1].item())
    keys, ids = ext.bin_write(uv.contiguous(), rxy.contiguous(), conic.contiguous(),
                              opacity.contiguous(), valid.to(torch.int32).contiguous(),
                              depth.contiguous(), offs.to(torch.int32).contiguous(), total,
                              W, H, tile, tx, ty)
    assert keys.dtype == torch.int64 and ids.dtype == torch.int32
    skeys, order = torch.sort(keys, stable=True)
    tiles = skeys >> 32
    offsets = torch.searchsorted(tiles, torch.arange(tx * ty + 1, device=uv.device,
                                                     dtype=tiles.dtype))
    return ids[order], offsets.to(torch.int32), tx, skeys


@pytest.mark.parametrize("tile", [16, 12])
def test_tile_list_sequence_bit_exact(dev, tile):
    ext = _ext()
    W, H = 240, 320
    s = scene(n=20000, seed=3, z=3.0, spread=0.5, scale=(0.005, 0.085))
    fx, fy, cx, cy, cc = _camera_args(intrinsics(W, H, f=200.0), torch.eye(4))
    m, q, sc, op = (s[k].to(dev) for k in ("means", "quats", "scales", "opacities"))
    sh = s["sh"].to(dev)
    uv, conic, depth, rxy, valid, _ = ext.preprocess_forward(
        m, q, sc, sh, sh, op, torch.eye(4), fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
        float(max(W, H)), cc, 3)
    ids, offs, tx, skeys = _lists_by_reference_sequence(ext, uv, rxy, depth, valid, conic, op,
                                                        W, H, tile)
    cpu = [t.cpu().numpy() for t in (uv, rxy, conic, op, valid, depth)]
    rids, roffs, rtx, rkeys = binning_ref.build_tile_lists(*cpu, W, H, tile)
    assert tx == rtx and rids.size > 20000
    assert np.array_equal(skeys.cpu().numpy().view(np.uint64), rkeys)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(offs.cpu().numpy(), roffs)


def test_fused_ssim_sequence_against_the_oracle(dev):
    """train.py:86-105: five kernels forward, four backward."""
    ext = _ext()
    H, W = 61, 77
    g = torch.Generator().manual_seed(4)
    a64 = torch.rand(H, W, 3, generator=g, dtype=torch.float64)
    b64 = (a64 + 0.1 * torch.randn(H, W, 3, generator=g, dtype=torch.float64)).clamp(0, 1)
    a, b = a64.float().to(dev), b64.float().to(dev)
    w = ssim_ref.window().to(dev)
    inter = ext.ssim_stack_blur_h(a, b, w, H, W)
    blurred = ext.ssim_blur15(inter, w, 1, H, W)
    smap = ext.ssim_tail_forward(blurred, H, W)
    assert tuple(inter.shape) == (1, 15, H, W) and tuple(smap.shape) == (1, 3, H, W)
    ar = a64.clone().requires_grad_(True)
    want = ssim_ref.ssim(ar, b64)
    want.backward()
    assert abs(float(smap.mean()) - float(want)) < 1e-5
    # d mean / d map = 1 / (3 H W), as autograd hands it to the reference.
    gout = torch.full_like(smap, 1.0 / smap.numel())
    d_blur = ext.ssim_tail_backward(blurred, gout, H, W)
    d_inter = ext.ssim_blur15(d_blur, w, 1, H, W)
    d_stack = ext.ssim_blur15(d_inter, w, 0, H, W)
    d_a = ext.ssim_chain_backward(a, b, d_stack, H, W)
    assert tuple(d_a.shape) == (H, W, 3)
    assert rel_l2(d_a.cpu(), ar.grad) < 1e-4


class _Project(torch.autograd.Function):
    """The reference's projection bridge (metal_backend.py:288-333) over ext."""

    @staticmethod
    def forward(ctx, means, quats, scales, sh, sh_rest, opac, viewmat, fx, fy, cx, cy, W, H,
                cam_center):
        ext = _ext()
        outs = ext.preprocess_forward(means, quats, scales, sh, sh_rest, opac, viewmat, fx, fy,
                                      cx, cy, W, H, 0.01, 100.0, 0.3, float(max(W, H)),
                                      cam_center, 3)
        ctx.save_for_backward(means, quats, scales, sh, sh_rest, outs[4])
        ctx.fused = sh_rest is sh
        ctx.meta = (viewmat, fx, fy, cx, cy, W, H, cam_center)
        ctx.mark_non_differentiable(outs[2], outs[3], outs[4])
        return tuple(outs)

    @staticmethod
    def backward(ctx, d_uv, d_conic, d_depth, d_rxy, d_valid, d_color):
        ext = _ext()
        means, quats, scales, sh, rest, valid = ctx.saved_tensors
        viewmat, fx, fy, cx, cy, W, H, cc = ctx.meta
        d = ext.preprocess_backward(means, quats, scales, sh, rest, d_uv, d_conic, d_color,
                                    valid, viewmat, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
                                    float(max(W, H)), cc, 3)
        if ctx.fused:
            assert d[4] is d[3]
        return (d[0], d[1], d[2], d[3], None if ctx.fused else d[4]) + (None,) * 9


class _Raster(torch.autograd.Function):
    """The reference's raster bridge (metal_backend.py:336-364) over ext."""

    @staticmethod
    def forward(ctx, uv, conic, opacity, color, ids, offs, W, H, tile, tx):
        ext = _ext()
        rgb, alpha, T, n = ext.rasterize_forward(uv, conic, opacity, color, ids, offs, W, H,
                                                 tile, tx)
        ctx.save_for_backward(uv, conic, opacity, color, ids, offs, T, n)
        ctx.dims = (W, H, tile, tx)
        return rgb, alpha

    @staticmethod
    def backward(ctx, g_rgb, g_alpha):
        ext = _ext()
        uv, conic, opacity, color, ids, offs, T, n = ctx.saved_tensors
        d = ext.rasterize_backward(uv, conic, opacity, color, ids, offs, T, n, g_rgb, g_alpha,
                                   *ctx.dims, False)
        assert tuple(d[4].shape) == (1,)
        return (d[0], d[1], d[2], d[3]) + (None,) * 6


@pytest.mark.parametrize("fused", [True, False])
def test_projection_and_raster_bridges_against_the_oracle(dev, fused):
    """A render through the reference's bridges and tile-list sequence, with
    the loss mean(rgb^2) + 0.1 mean(alpha^2), against float64 autograd of
    render_ref, which composites every listed Gaussian."""
    ext = _ext()
    W, H, tile, n = 96, 72, 16, 400
    s = scene(n=n, seed=12)
    K, vm = intrinsics(W, H), torch.eye(4)
    fx, fy, cx, cy, cc = _camera_args(K, vm)
    leaves = [s[k].to(dev).clone().requires_grad_(True) for k in ("means", "quats", "scales")]
    op = s["opacities"].to(dev).requires_grad_(True)
    if fused:
        shl = [s["sh"].to(dev).clone().requires_grad_(True)]
        sh_args = (shl[0], shl[0])
    else:
        shl = [s["sh"][:, :1].contiguous().to(dev).requires_grad_(True),
               s["sh"][:, 1:].contiguous().to(dev).requires_grad_(True)]
        sh_args = tuple(shl)
    uv, conic, depth, rxy, valid, color = _Project.apply(*leaves, *sh_args, op.detach(), vm,
                                                         fx, fy, cx, cy, W, H, cc)
    ids, offs, tx, _ = _lists_by_reference_sequence(ext, uv.detach(), rxy, depth, valid,
                                                    conic.detach(), op.detach(), W, H, tile)
    rgb, alpha = _Raster.apply(uv, conic, op, color, ids, offs, W, H, tile, tx)
    (rgb.square().mean() + 0.1 * alpha.square().mean()).backward()

    ref = [s[k].double().requires_grad_(True) for k in ("means", "quats", "scales", "opacities",
                                                       "sh")]
    r_rgb, r_alpha, _ = render_ref.render(*ref, K.double(), vm.double(), W, H, sh_degree=3,
                                          tile=16, min_transmittance=0.0)
    (r_rgb.square().mean() + 0.1 * r_alpha.square().mean()).backward()
    # The extension stops each pixel at T < 1e-4, as the reference kernel
    # does; what the rest of the list would add is below 1e-4 of the largest
    # colour.
    bar = 1e-4 * max(1.0, float(color.detach().max())) + 1e-6
    assert float((rgb.detach().cpu().double() - r_rgb.detach()).abs().max()) < bar
    assert float((alpha.detach().cpu().double() - r_alpha.detach()).abs().max()) < 1e-4
    got = [t.grad for t in leaves] + [op.grad,
                                      shl[0].grad if fused else torch.cat([shl[0].grad,
                                                                           shl[1].grad], 1)]
    for name, a, b in zip(("means", "quats", "scales", "opacities", "sh"), got, ref):
        assert rel_l2(a.cpu(), b.grad) < 1e-3, f"{name}: {rel_l2(a.cpu(), b.grad):.2e}"


def test_adam_step_in_place_against_the_restatement(dev):
    ext = _ext()
    g = torch.Generator().manual_seed(8)
    p = torch.randn(5000, generator=g)
    want = [p.numpy().copy(), np.zeros(5000, np.float32), np.zeros(5000, np.float32)]
    pd, m, v = p.to(dev), torch.zeros(5000, device=dev), torch.zeros(5000, device=dev)
    for k in range(1, 6):
        grad = torch.randn(5000, generator=g) * 1e-2
        ext.adam_step(pd, grad.to(dev), m, v, 1e-3, 0.9, 0.999, 1e-15, k)
        adam_ref.adam_step(want[0], grad.numpy(), want[1], want[2], 1e-3, 0.9, 0.999, 1e-15, k)
    assert np.abs(pd.cpu().numpy() - want[0]).max() < 1e-6 * np.abs(want[0]).max()
    with pytest.raises(RuntimeError, match="numel mismatch"):
        ext.adam_step(pd, grad[:10].to(dev), m, v, 1e-3, 0.9, 0.999, 1e-15, 6)


def test_rasterize_backward_absgrad_slot(dev):
    """d_absuv is (N,) with want_absgrad and a single zero otherwise
    (rasterize.mm:162-164); the other four outputs do not depend on it."""
    ext = _ext()
    W, H, tile = 64, 48, 16
    s = scene(n=200, seed=5)
    fx, fy, cx, cy, cc = _camera_args(intrinsics(W, H), torch.eye(4))
    m, q, sc, op = (s[k].to(dev) for k in ("means", "quats", "scales", "opacities"))
    sh = s["sh"].to(dev)
    uv, conic, depth, rxy, valid, color = ext.preprocess_forward(
        m, q, sc, sh, sh, op, torch.eye(4), fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
        float(max(W, H)), cc, 3)
    ids, offs, tx, _ = _lists_by_reference_sequence(ext, uv, rxy, depth, valid, conic, op, W, H,
                                                    tile)
    rgb, alpha, T, n = ext.rasterize_forward(uv, conic, op, color, ids, offs, W, H, tile, tx)
    assert n.dtype == torch.int32 and tuple(T.shape) == (H, W)
    g_rgb = (2.0 * rgb).contiguous()
    g_a = torch.zeros(H, W, device=dev)
    on = ext.rasterize_backward(uv, conic, op, color, ids, offs, T, n, g_rgb, g_a, W, H, tile,
                                tx, True)
    off = ext.rasterize_backward(uv, conic, op, color, ids, offs, T, n, g_rgb, g_a, W, H, tile,
                                 tx, False)
    assert tuple(on[4].shape) == (200,) and tuple(off[4].shape) == (1,)
    assert float(off[4].abs().max()) == 0.0 and float(on[4].max()) > 0
    for a, b in zip(on[:4], off[:4]):
        assert a.is_contiguous() and rel_l2(a.cpu(), b.cpu()) < 1e-6
    assert bool((on[4] + 1e-6 >= on[0].norm(dim=1)).all())
