"""The ellipse test drops only pairs that cannot reach any pixel: rendering
the same projection with rectangle-bound tile lists and with ellipse-filtered
tile lists gives identical images.

The reference pins this property on its own kernels
(tests/test_metal_binning.py:44-59, tests/test_boundary_culling.py:100-114):
the binning drops a (Gaussian, tile) pair when the minimum of the conic's
quadratic form over the tile rectangle is at least 2 ln(255 opacity)
(binning.metal:25-90), the rasteriser skips a pixel's Gaussian when
opacity * exp(-Q/2) < 1/255 (rasterize.metal:136-140), and the two must
agree for every dropped pair. Here the HIP projection's outputs are binned
twice on the GPU (backend.build_tile_lists without the conic: every tile of
the SnugBox rectangle; build_tile_lists_metal: the ellipse test), and:

* the raster forward's images and alpha are ``torch.equal``;
* the raster backward's gradients agree up to the order of the float
  atomics (relative L2 below 1e-5; the same Gaussians receive gradient);
* the ellipse lists are a strict subset of the rectangle lists, with each
  tile's entries in the same order (checked on the reference scene).

Scenes: the reference's own (20k splats, 240x320, f = 200, tiles 16 and
32), one full config-4 view (1M Gaussians, 800x800), and the crowded
config-5 scene (3.6M Gaussians, 1920x1080, over 30M intersections).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _reference_scene(dev):
    """tests/test_boundary_culling.py:90-99 of the reference: rotated,
    elongated splats in front of an identity camera."""
    N = 20000
    g = torch.Generator(device="cpu").manual_seed(1)
    means = torch.randn(N, 3, generator=g) * 0.5
    means[:, 2] += 3.0
    quats = torch.randn(N, 4, generator=g)
    scales = torch.rand(N, 3, generator=g) * 0.08 + 0.005
    op = torch.rand(N, generator=g) * 0.9 + 0.05
    sh = torch.randn(N, 16, 3, generator=g) * 0.3
    return [t.to(dev) for t in (means, quats, scales, op, sh)]


def _both_lists(uv, rxy, depth, valid, conic, op, W, H, tile):
    from metal_gauss_amd.backend import build_tile_lists, build_tile_lists_metal

    rect = build_tile_lists(uv, rxy[:, 0], depth, valid.bool(), W, H, tile, ry=rxy[:, 1])
    ell = build_tile_lists_metal(uv, rxy, depth, valid, conic, op, W, H, tile)
    assert rect[2] == ell[2] and rect[1].shape == ell[1].shape
    return rect, ell


def _subset_per_tile(rect, ell):
    """Every tile's ellipse list is its rectangle list with entries removed,
    order kept (both are sorted by (depth, Gaussian id))."""
    r_ids, r_off = rect[0].cpu().numpy(), rect[1].cpu().numpy().astype(np.int64)
    e_ids, e_off = ell[0].cpu().numpy(), ell[1].cpu().numpy().astype(np.int64)
    T = r_off.size - 1
    r_tile = np.repeat(np.arange(T, dtype=np.int64), np.diff(r_off))
    e_tile = np.repeat(np.arange(T, dtype=np.int64), np.diff(e_off))
    n = max(int(r_ids.max(initial=0)), int(e_ids.max(initial=0))) + 1
    r_key = r_tile * n + r_ids
    e_key = e_tile * n + e_ids
    sorter = np.argsort(r_key, kind="stable")
    pos = np.clip(np.searchsorted(r_key[sorter], e_key), 0, r_key.size - 1)
    at = sorter[pos]                      # each ellipse entry's index in the rectangle lists
    assert np.array_equal(r_key[at], e_key), "an ellipse pair is not in the rectangle lists"
    same_tile = np.diff(e_tile) == 0
    assert np.all(np.diff(at)[same_tile] > 0), "order within a tile differs"


def _render_both(args_common, rect, ell, W, H, tile, grad_rgb, grad_alpha, label):
    """Forward with both lists (torch.equal), then backward with both."""
    from metal_gauss_amd import backend

    ext = backend._load()
    uv, conic, op, color = (x.contiguous() for x in args_common)
    fa = ext.rasterize_forward(uv, conic, op, color, rect[0], rect[1], W, H, tile, rect[2])
    fb = ext.rasterize_forward(uv, conic, op, color, ell[0], ell[1], W, H, tile, ell[2])
    print(f"{label}: rectangle lists {rect[0].numel()}, ellipse lists {ell[0].numel()} "
          f"({1 - ell[0].numel() / max(rect[0].numel(), 1):.1%} dropped), "
          f"max |d rgb| {(fa[0] - fb[0]).abs().max().item():.3e}", flush=True)
    assert ell[0].numel() < rect[0].numel(), "the ellipse test removed nothing"
    assert torch.equal(fa[0], fb[0]), f"image differs, max {(fa[0] - fb[0]).abs().max().item():.3e}"
    assert torch.equal(fa[1], fb[1]), "alpha differs"
    assert torch.equal(fa[2], fb[2]), "final transmittance differs"
    ga = ext.rasterize_backward(uv, conic, op, color, rect[0], rect[1], fa[2], fa[3], grad_rgb,
                                grad_alpha, W, H, tile, rect[2], True)
    gb = ext.rasterize_backward(uv, conic, op, color, ell[0], ell[1], fb[2], fb[3], grad_rgb,
                                grad_alpha, W, H, tile, ell[2], True)
    for name, a, b in zip(("d_uv", "d_conic", "d_opacity", "d_color", "d_absuv"), ga, gb):
        ra = a.reshape(a.shape[0], -1).abs().sum(1) > 0
        rb = b.reshape(b.shape[0], -1).abs().sum(1) > 0
        assert torch.equal(ra, rb), f"{name}: different Gaussians receive gradient"
        err = rel_l2(a.cpu(), b.cpu())
        assert err < 1e-5, f"{name}: relative L2 {err:.2e} between the two lists"


@pytest.mark.parametrize("tile", [16, 32])
def test_reference_scene_renders_identically(dev, tile):
    """The reference's 20k-splat, 240x320 scene (f = 200) through the
    extension surface, as tests/test_metal_binning.py:44-59 runs it."""
    from metal_gauss_amd import backend

    ext = backend._load()
    means, quats, scales, op, sh = _reference_scene(dev)
    W, H = 240, 320
    vm = torch.eye(4)
    cc = (-vm[:3, :3].T @ vm[:3, 3]).contiguous()
    uv, conic, depth, rxy, valid, color = ext.preprocess_forward(
        means, quats, scales, sh, sh, op, vm.contiguous(), 200.0, 200.0, W / 2, H / 2, W, H,
        0.01, 100.0, 0.3, 1.0 * max(W, H), cc, 3)
    rect, ell = _both_lists(uv, rxy, depth, valid, conic, op, W, H, tile)
    _subset_per_tile(rect, ell)
    g = torch.Generator(device=dev).manual_seed(11)
    grad_rgb = torch.randn(H, W, 3, device=dev, generator=g)
    grad_alpha = torch.randn(H, W, device=dev, generator=g)
    _render_both((uv, conic, op, color), rect, ell, W, H, tile, grad_rgb, grad_alpha,
                 f"reference scene tile {tile}")


def _product_projection(sc, cam, dev):
    from test_gpu_fullsize import _leaves, _project

    p = _leaves(sc, dev)
    with torch.no_grad():
        outs, _ = _project(p, cam)
    del p
    return outs


def test_config4_view_renders_identically(dev):
    """One config-4 view (1M Gaussians, SH 3, 800x800) with the trainer's
    activations, projected by the product's kernel."""
    from metal_gauss_amd import scenes

    sc, cams, _ = scenes.config4()
    cam = cams[23]
    W, H = cam.W, cam.H
    uv, conic, depth, rxy, valid, color, op_eff = _product_projection(sc, cam, dev)
    rect, ell = _both_lists(uv, rxy, depth, valid, conic, op_eff, W, H, 16)
    g = torch.Generator(device=dev).manual_seed(23)
    grad_rgb = torch.randn(H, W, 3, device=dev, generator=g) / (H * W)
    grad_alpha = torch.randn(H, W, device=dev, generator=g) / (H * W)
    _render_both((uv, conic, op_eff, color), rect, ell, W, H, 16, grad_rgb, grad_alpha,
                 "config 4 view 23")


def test_config5_crowded_renders_identically(dev):
    """The crowded config-5 scene (3.6M Gaussians, heavy-tailed scales,
    1920x1080 from inside the cloud: 8160 tiles, the radix route)."""
    from metal_gauss_amd import scenes

    sc, cam, _ = scenes.config5_crowded()
    W, H = cam.W, cam.H
    uv, conic, depth, rxy, valid, color, op_eff = _product_projection(sc, cam, dev)
    rect, ell = _both_lists(uv, rxy, depth, valid, conic, op_eff, W, H, 16)
    assert ell[0].numel() > 30_000_000
    g = torch.Generator(device=dev).manual_seed(5)
    grad_rgb = torch.randn(H, W, 3, device=dev, generator=g) / (H * W)
    grad_alpha = torch.randn(H, W, device=dev, generator=g) / (H * W)
    _render_both((uv, conic, op_eff, color), rect, ell, W, H, 16, grad_rgb, grad_alpha,
                 "config 5 crowded")
