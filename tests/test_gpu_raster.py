"""The rasteriser kernels in isolation against the C restatement of their
per-pixel contract (oracle/raster_seq.c), on identical inputs and tile lists.

Bars: images within 1e-4 max-abs, gradients within
1e-3 relative L2. Pixels the oracle marks ill-conditioned (an alpha within
1e-5 relative of the 1/255 cutoff, or the stopping T within 1e-5 of t_min,
where one ulp of exp flips a discrete decision) are counted and bounded
separately rather than compared at 1e-4."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import intrinsics, rel_l2, scene
from oracle import raster_ref

pytestmark = pytest.mark.gpu


def prepare(n, seed, W, H, tile, dev, elongate=False, sh=False):
    from metal_gauss_amd.backend import _PreprocessMetal, _camera, build_tile_lists_metal

    s = scene(n=n, seed=seed)
    if elongate:
        s["scales"] = s["scales"] * torch.tensor([4.0, 0.5, 1.0])
    fx, fy, cx, cy, vm_h, cc = _camera(intrinsics(W, H), torch.eye(4))
    with torch.no_grad():
        uv, conic, depth, rxy, valid = _PreprocessMetal.apply(
            s["means"].to(dev), s["quats"].to(dev), s["scales"].to(dev), None, None,
            s["opacities"].to(dev), vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
            float(max(W, H)), cc, 3)
        op = s["opacities"].to(dev)
        col = s["colors"].to(dev)
        gids, offs, tx = build_tile_lists_metal(uv, rxy, depth, valid, conic, op, W, H, tile)
    return uv, conic, op, col, gids, offs, tx


def gpu_forward(args, W, H, tile, t_min, background=None, chunked=True, sched=None):
    """mg_rasterize_forward; returns (rgb, alpha, T, stop, chunk workspace or None)."""
    from metal_gauss_amd import _lib

    uv, conic, op, col, gids, offs, tx = args
    dev = uv.device
    rgb = torch.empty(H, W, 3, device=dev)
    alpha = torch.empty(H, W, device=dev)
    T = torch.empty(H, W, device=dev)
    stop = torch.empty(H, W, dtype=torch.int32, device=dev)
    lib = _lib.load()
    ws = None
    if chunked:
        ws = torch.empty(lib.mg_rasterize_chunk_workspace_bytes(gids.numel(), offs.numel() - 1,
                                                                tile),
                         dtype=torch.uint8, device=dev)
    _lib.check(lib.mg_rasterize_forward(uv.shape[0], uv.data_ptr(), conic.data_ptr(),
                                        op.data_ptr(), col.data_ptr(), gids.data_ptr(),
                                        offs.data_ptr(), W, H, tile, tx, t_min,
                                        None if background is None else
                                        _lib.f32_array(background), gids.numel(),
                                        None if ws is None else ws.data_ptr(),
                                        0 if ws is None else ws.numel(), rgb.data_ptr(),
                                        alpha.data_ptr(), T.data_ptr(), stop.data_ptr(),
                                        None, None if sched is None else sched.data_ptr(),
                                        _lib.stream(uv)))
    return rgb, alpha, T, stop, ws


def gpu_backward(args, fwd, grad_rgb, grad_alpha, W, H, tile, absgrad=True, background=None,
                 sched=None):
    from metal_gauss_amd import _lib

    uv, conic, op, col, gids, offs, tx = args
    _, alpha, T, stop, ws = fwd
    N, dev = uv.shape[0], uv.device
    rec = torch.full((N, 10), 7.0, device=dev)     # overwritten by the kernel
    lib = _lib.load()
    _lib.check(lib.mg_rasterize_backward(
        N, uv.data_ptr(), conic.data_ptr(), op.data_ptr(), col.data_ptr(), gids.data_ptr(),
        offs.data_ptr(), T.data_ptr(), stop.data_ptr(), grad_rgb.data_ptr(),
        None if grad_alpha is None else grad_alpha.data_ptr(),
        alpha.data_ptr() if background is not None else None,
        None if background is None else _lib.f32_array(background), gids.numel(),
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), W, H, tile, tx,
        rec.data_ptr(), int(absgrad), 0, None if sched is None else sched.data_ptr(),
        _lib.stream(uv)))
    # The record's slots as the reference's five tensors.
    return [rec[:, 0:2], rec[:, 2:5], rec[:, 5], rec[:, 6:9], rec[:, 9] if absgrad else None]


def np_(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("t_min", [0.0, 1e-4])
@pytest.mark.parametrize("tile", [8, 12, 16, 32])
def test_forward_matches_contract(dev, tile, t_min):
    W, H = 100, 63
    args = prepare(600, 17, W, H, tile, dev, elongate=True)
    rgb, alpha, T, stop, _ = gpu_forward(args, W, H, tile, t_min)
    r = raster_ref.forward(*[np_(a) for a in args[:6]], W, H, tile, t_min)
    amb = r[4]
    ok = ~amb
    assert amb.mean() < 1e-3, f"{amb.sum()} ill-conditioned pixels"
    assert np.abs(np_(rgb) - r[0])[ok].max() < 1e-4
    assert np.abs(np_(alpha) - r[1])[ok].max() < 1e-4
    assert np.abs(np_(T) - r[2])[ok].max() < 1e-4
    assert (np_(stop) == r[3])[ok].all(), "stop indices differ"


@pytest.mark.parametrize("chunked", [True, False])
@pytest.mark.parametrize("tile", [8, 12, 16, 32])
def test_backward_matches_contract(dev, tile, chunked):
    W, H = 100, 63
    args = prepare(600, 19, W, H, tile, dev, elongate=True)
    fwd = gpu_forward(args, W, H, tile, 1e-4, chunked=chunked)
    g = torch.Generator().manual_seed(3)
    grad_rgb = torch.randn(H, W, 3, generator=g).to(dev)
    grad_alpha = torch.randn(H, W, generator=g).to(dev)
    outs = gpu_backward(args, fwd, grad_rgb, grad_alpha, W, H, tile)
    ref = raster_ref.backward(*[np_(a) for a in args[:6]], np_(fwd[2]), np_(fwd[3]),
                              np_(grad_rgb), np_(grad_alpha), W, H, tile)
    for name, a, b in zip(("d_uv", "d_conic", "d_opacity", "d_color", "d_absuv"), outs, ref):
        assert torch.isfinite(a).all(), name
        assert rel_l2(np_(a), b) < 1e-3, f"tile {tile}: {name} rel L2 {rel_l2(np_(a), b):.2e}"


def test_absgrad_is_at_least_the_norm_of_the_summed_gradient(dev):
    """tests/test_absgrad.py:60-76: sum |d_uv_px| >= |sum d_uv_px|."""
    W, H, tile = 96, 64, 16
    args = prepare(300, 0, W, H, tile, dev)
    fwd = gpu_forward(args, W, H, tile, 1e-4)
    grad_rgb = (2.0 * fwd[0]).contiguous()           # d/drgb of mean(rgb^2) up to 1/n
    grad_alpha = torch.zeros(H, W, device=dev)
    d_uv, _, _, _, d_abs = gpu_backward(args, fwd, grad_rgb, grad_alpha, W, H, tile)
    slack = d_abs - d_uv.norm(dim=1)
    assert (d_abs >= 0).all() and d_abs.sum() > 0
    assert (slack >= -1e-4 * d_abs.max()).all()
    assert (slack > 1e-6 * d_abs.max()).any()


def test_gradients_are_overwritten_not_accumulated(dev):
    """The backward zero-fills its outputs (they arrive holding 7s)."""
    W, H, tile = 48, 32, 16
    args = prepare(50, 1, W, H, tile, dev)
    args = (args[0], args[1], args[2], args[3], args[4][:0].contiguous(),
            torch.zeros_like(args[5]), args[6])             # empty lists
    fwd = gpu_forward(args, W, H, tile, 1e-4)
    assert float(fwd[1].abs().max()) == 0.0 and float(fwd[2].min()) == 1.0
    outs = gpu_backward(args, fwd, torch.ones(H, W, 3, device=dev), torch.ones(H, W, device=dev),
                        W, H, tile)
    for o in outs:
        assert float(o.abs().max()) == 0.0


def test_oversized_tile_is_refused(dev):
    """tests/test_metal.py:205-213: one tile is one workgroup."""
    from metal_gauss_amd import render

    s = scene(n=50)
    with pytest.raises(RuntimeError, match="threads per threadgroup"):
        render(s["means"].to(dev), s["quats"].to(dev), s["scales"].to(dev),
               s["opacities"].to(dev), None, intrinsics(96, 64), torch.eye(4), 96, 64,
               colors=s["colors"].to(dev), tile=64)


def test_config2_scale_forward_and_backward(dev):
    """BASELINE configs[1] at full size: 300k Gaussians, 800x800, SH 3, white
    background; the raster kernels against the contract on the real lists."""
    from metal_gauss_amd import scenes
    from metal_gauss_amd.backend import _PreprocessMetal, _camera, build_tile_lists_metal

    sc, cam, _ = scenes.config2()
    m, q, sca, op, sh = (t.to(dev) for t in sc.activated())
    fx, fy, cx, cy, vm_h, cc = _camera(cam.K, cam.viewmat)
    W, H, tile = cam.W, cam.H, 16
    with torch.no_grad():
        uv, conic, depth, rxy, valid, col = _PreprocessMetal.apply(
            m, q, sca, sh, None, op, vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
            float(max(W, H)), cc, 3)
        gids, offs, tx = build_tile_lists_metal(uv, rxy, depth, valid, conic, op, W, H, tile)
    args = (uv, conic, op, col, gids, offs, tx)
    fwd = gpu_forward(args, W, H, tile, 1e-4)
    r = raster_ref.forward(*[np_(a) for a in args[:6]], W, H, tile, 1e-4)
    ok = ~r[4]
    print(f"config 2: {gids.numel()} intersections, {r[4].sum()} ill-conditioned pixels")
    assert r[4].mean() < 1e-3
    assert np.abs(np_(fwd[0]) - r[0])[ok].max() < 1e-4
    assert np.abs(np_(fwd[1]) - r[1])[ok].max() < 1e-4
    target = scenes.config2_target().to(dev)
    img = fwd[0] + (1.0 - fwd[1])[..., None]                # white background
    grad_rgb = (torch.sign(img - target) / img.numel()).contiguous()
    grad_alpha = (-(grad_rgb.sum(dim=-1))).contiguous()     # through the blend
    outs = gpu_backward(args, fwd, grad_rgb, grad_alpha, W, H, tile)
    ref = raster_ref.backward(*[np_(a) for a in args[:6]], np_(fwd[2]), np_(fwd[3]),
                              np_(grad_rgb), np_(grad_alpha), W, H, tile)
    for name, a, b in zip(("d_uv", "d_conic", "d_opacity", "d_color"), outs, ref):
        assert rel_l2(np_(a), b) < 1e-3, f"{name} rel L2 {rel_l2(np_(a), b):.2e}"


def _tile_of_block(b, tiles_x, tiles_y, sup=4, xcds=8):
    """The raster kernels' workgroup -> tile dealing (rasterize.hip
    tile_of_block): 4x4-tile super-tiles round-robin over the eight XCDs."""
    xcd, k = b % xcds, b // xcds
    s = (k // (sup * sup)) * xcds + xcd
    sx, sy = -(-tiles_x // sup), -(-tiles_y // sup)
    if s >= sx * sy:
        return -1
    loc = k % (sup * sup)
    x, y = (s % sx) * sup + loc % sup, (s // sx) * sup + loc // sup
    return y * tiles_x + x if x < tiles_x and y < tiles_y else -1


def _order_bin(w):
    """The schedule's counting-sort bin of a walk length (rasterize.hip
    order_bin): exact below 768, 32 entries a bin above, capped at 1023."""
    return w if w < 768 else min(1023, 768 + ((w - 768) >> 5))


def test_backward_schedule_config2(dev):
    """The backward schedule on config 2's full-size lists (2500 tiles):
    mg_rasterize_forward(sched=) leaves its outputs bit for bit as without it
    and records, for each workgroup, its tile's walk length max(stop) - first
    entry (-1 for a workgroup without a tile); the backward given the buffer
    writes, per XCD, the tiles tile_of_block deals it, each once, longest walk
    (bin) first, then -1 for the empty slots, and returns the unscheduled
    backward's gradients up to the order of the float atomics, also from a
    buffer of garbage the forward never wrote."""
    from metal_gauss_amd import _lib, scenes
    from metal_gauss_amd.backend import _PreprocessMetal, _camera, build_tile_lists_metal

    sc, cam, _ = scenes.config2()
    m, q, sca, op, sh = (t.to(dev) for t in sc.activated())
    fx, fy, cx, cy, vm_h, cc = _camera(cam.K, cam.viewmat)
    W, H, tile = cam.W, cam.H, 16
    with torch.no_grad():
        uv, conic, depth, rxy, valid, col = _PreprocessMetal.apply(
            m, q, sca, sh, None, op, vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
            float(max(W, H)), cc, 3)
        gids, offs, tx = build_tile_lists_metal(uv, rxy, depth, valid, conic, op, W, H, tile)
    args = (uv, conic, op, col, gids, offs, tx)
    lib = _lib.load()
    ty = -(-H // tile)
    grid = -(-(-(-tx // 4) * -(-ty // 4)) // 8) * 8 * 16
    assert lib.mg_rasterize_sched_ints(W, H, tile) == 2 * grid
    sched = torch.full((2 * grid,), -7, dtype=torch.int32, device=dev)
    plain = gpu_forward(args, W, H, tile, 1e-4, chunked=False)
    fwd = gpu_forward(args, W, H, tile, 1e-4, chunked=False, sched=sched)
    for a, b in zip(plain[:4], fwd[:4]):
        assert torch.equal(a, b)
    stop = np_(fwd[3]).astype(np.int64)
    o = np_(offs).astype(np.int64)
    tmax = stop.reshape(ty, tile, tx, tile).max(axis=(1, 3)).reshape(-1)
    work = np.maximum(tmax, o[:-1]) - o[:-1]
    dealt = [_tile_of_block(b, tx, ty) for b in range(grid)]
    assert np_(sched[:grid]).tolist() == [int(work[t]) if t >= 0 else -1 for t in dealt]

    g = torch.Generator().manual_seed(11)
    grad_rgb = torch.randn(H, W, 3, generator=g).to(dev)
    want = gpu_backward(args, fwd, grad_rgb, None, W, H, tile)
    got = gpu_backward(args, fwd, grad_rgb, None, W, H, tile, sched=sched)
    for name, a, b in zip(("d_uv", "d_conic", "d_opacity", "d_color", "absgrad"), got, want):
        assert rel_l2(np_(a), np_(b)) < 1e-5, f"{name} rel L2 {rel_l2(np_(a), np_(b)):.2e}"
    # A buffer the forward never filled only reorders the tiles.
    junk = torch.randint(-2**31, 2**31 - 1, (2 * grid,), generator=g, dtype=torch.int32).to(dev)
    got_junk = gpu_backward(args, fwd, grad_rgb, None, W, H, tile, sched=junk)
    for name, a, b in zip(("d_uv", "d_conic", "d_opacity", "d_color", "absgrad"), got_junk, want):
        assert rel_l2(np_(a), np_(b)) < 1e-5, f"junk schedule: {name}"

    order = np_(sched[grid:])
    for x in range(8):
        mine = [t for t in dealt[x::8] if t >= 0]
        lst = order[x::8].tolist()
        assert sorted(lst[:len(mine)]) == sorted(mine), f"XCD {x}: not its tiles"
        assert lst[len(mine):] == [-1] * (len(lst) - len(mine)), f"XCD {x}: empty slots"
        bins = [_order_bin(int(work[t])) for t in lst[:len(mine)]]
        assert all(a >= b for a, b in zip(bins, bins[1:])), f"XCD {x}: not longest first"


def test_background_blend_in_kernel(dev):
    """The in-kernel blend equals the reference's torch expression
    rgb + (1 - alpha).clamp_min(0) * bg (metal_backend.py:539-541), and its
    backward equals the plain backward with grad_alpha reduced by grad_rgb . bg
    (clamp_min passes the gradient wherever 1 - alpha >= 0)."""
    W, H, tile = 100, 63, 16
    bg = (0.25, 0.5, 1.0)
    args = prepare(600, 23, W, H, tile, dev, elongate=True)
    plain = gpu_forward(args, W, H, tile, 1e-4)
    blended = gpu_forward(args, W, H, tile, 1e-4, background=bg)
    bgt = torch.tensor(bg, device=dev)
    want = plain[0] + (1.0 - plain[1]).clamp_min(0)[..., None] * bgt
    assert torch.equal(blended[0], want)
    for a, b in zip(plain[1:4], blended[1:4]):
        assert torch.equal(a, b)
    g = torch.Generator().manual_seed(5)
    grad_rgb = torch.randn(H, W, 3, generator=g).to(dev)
    grad_alpha = torch.randn(H, W, generator=g).to(dev)
    got = gpu_backward(args, blended, grad_rgb, grad_alpha, W, H, tile, background=bg)
    ga = grad_alpha - torch.where(1.0 - plain[1] >= 0, (grad_rgb * bgt).sum(-1),
                                  torch.zeros_like(grad_alpha))
    ref = gpu_backward(args, plain, grad_rgb, ga.contiguous(), W, H, tile)
    for a, b in zip(got, ref):
        assert rel_l2(a.cpu(), b.cpu()) < 1e-5


@pytest.mark.parametrize("t_min", [0.0, 1e-4])
@pytest.mark.parametrize("tile", [16, 32])
def test_chunked_backward_on_long_lists(dev, tile, t_min):
    """Tiles with thousands of entries, so the backward runs several
    512-entry units per tile from the forward's checkpoints. Against the C
    contract (1e-3 relative L2) and against the one-chain-per-tile backward
    (1e-4: both recover T by division, but from different starting points)."""
    W, H = 64, 48
    args = prepare(6000, 29, W, H, tile, dev)
    offs = args[5]
    longest = int((offs[1:] - offs[:-1]).max())
    assert longest > 4 * 512, longest
    g = torch.Generator().manual_seed(4)
    grad_rgb = torch.randn(H, W, 3, generator=g).to(dev)
    grad_alpha = torch.randn(H, W, generator=g).to(dev)
    chunked = gpu_forward(args, W, H, tile, t_min, chunked=True)
    whole = gpu_forward(args, W, H, tile, t_min, chunked=False)
    for a, b in zip(chunked[:4], whole[:4]):
        assert torch.equal(a, b)             # the checkpoints do not touch the forward
    got = gpu_backward(args, chunked, grad_rgb, grad_alpha, W, H, tile)
    one = gpu_backward(args, whole, grad_rgb, grad_alpha, W, H, tile)
    ref = raster_ref.backward(*[np_(a) for a in args[:6]], np_(chunked[2]), np_(chunked[3]),
                              np_(grad_rgb), np_(grad_alpha), W, H, tile)
    for name, a, b, c in zip(("d_uv", "d_conic", "d_opacity", "d_color", "d_absuv"), got, one,
                             ref):
        assert torch.isfinite(a).all(), name
        assert rel_l2(np_(a), c) < 1e-3, f"{name} vs contract {rel_l2(np_(a), c):.2e}"
        assert rel_l2(a.cpu(), b.cpu()) < 1e-4, f"{name} chunked vs whole {rel_l2(a.cpu(), b.cpu()):.2e}"


def test_missing_alpha_gradient_reads_as_zero(dev):
    """grad_alpha NULL (the coverage feeds no loss; render's autograd passes
    no materialised zeros) equals an explicit zero gradient."""
    W, H, tile = 100, 63, 16
    args = prepare(600, 37, W, H, tile, dev, elongate=True)
    fwd = gpu_forward(args, W, H, tile, 1e-4, chunked=False)
    g = torch.Generator().manual_seed(9)
    grad_rgb = torch.randn(H, W, 3, generator=g).to(dev)
    none = gpu_backward(args, fwd, grad_rgb, None, W, H, tile)
    zero = gpu_backward(args, fwd, grad_rgb, torch.zeros(H, W, device=dev), W, H, tile)
    for a, b in zip(none, zero):
        assert rel_l2(a.cpu(), b.cpu()) < 1e-6


def test_forward_clears_the_backward_records(dev):
    """mg_rasterize_forward(zero_grads=rec) clears the (N,10) record buffer
    (here prefilled with 7.0, N odd so the slices end mid-float4), and the
    backward told so (grads_zeroed = 1) gives the records of a backward that
    fills its own buffer."""
    from metal_gauss_amd import _lib

    W, H, tile = 96, 70, 16
    args = prepare(601, 23, W, H, tile, dev, elongate=True)
    uv, conic, op, col, gids, offs, tx = args
    N = uv.shape[0]
    assert N % 2 == 1
    lib = _lib.load()
    rgb = torch.empty(H, W, 3, device=dev)
    alpha = torch.empty(H, W, device=dev)
    T = torch.empty(H, W, device=dev)
    stop = torch.empty(H, W, dtype=torch.int32, device=dev)
    rec = torch.full((N, 10), 7.0, device=dev)
    _lib.check(lib.mg_rasterize_forward(N, uv.data_ptr(), conic.data_ptr(), op.data_ptr(),
                                        col.data_ptr(), gids.data_ptr(), offs.data_ptr(), W, H,
                                        tile, tx, 1e-4, None, gids.numel(), None, 0,
                                        rgb.data_ptr(), alpha.data_ptr(), T.data_ptr(),
                                        stop.data_ptr(), rec.data_ptr(), None,
                                        _lib.stream(uv)))
    torch.cuda.synchronize()
    assert float(rec.abs().max()) == 0.0
    g = torch.Generator().manual_seed(5)
    grad_rgb = torch.randn(H, W, 3, generator=g).to(dev)
    want = gpu_backward(args, (rgb, alpha, T, stop, None), grad_rgb, None, W, H, tile,
                        absgrad=True)
    _lib.check(lib.mg_rasterize_backward(
        N, uv.data_ptr(), conic.data_ptr(), op.data_ptr(), col.data_ptr(), gids.data_ptr(),
        offs.data_ptr(), T.data_ptr(), stop.data_ptr(), grad_rgb.data_ptr(), None, None, None,
        gids.numel(), None, 0, W, H, tile, tx, rec.data_ptr(), 1, 1, None, _lib.stream(uv)))
    got = [rec[:, 0:2], rec[:, 2:5], rec[:, 5], rec[:, 6:9], rec[:, 9]]
    for a, b in zip(got, want):
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-7), float((a - b).abs().max())
