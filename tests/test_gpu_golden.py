"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

config1 (10k Gaussians at 256x256) is checked in three ways:
  * The preprocess outputs must agree with the fixture's float32 contract.
    uv, conic, rxy and colour agree within float32 rounding; validity and
    depth ordering agree exactly.
  * Tile lists built on the GPU from the fixture's own preprocess outputs must
    equal the fixture's lists: every id, in order, and every offset.
  * The rendered image and alpha must agree within 1e-4 max-abs of the
    fixture's float64 render, with every listed Gaussian composited. Pixels
    the fixture flags as ill-conditioned at float32 are exempt: there some
    alpha sits within a relative 1e-5 of the 1/255 cutoff. They must be fewer
    than 0.1% of the image.
fwd_bwd_small checks the image within 1e-4 and every parameter gradient
within 1e-3 relative L2.
adam_small checks 20 FusedAdam steps (two eps values) and 20 SelectiveAdam
steps within 1e-6 relative to the parameters' magnitude, with step counts
exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2
from golden import make_golden as G

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def test_config1_preprocess_matches_fixture(dev):
    from metal_gauss_amd import backend as B

    z = G.load("config1")
    W, H = int(z["W"]), int(z["H"])
    K, vm = torch.from_numpy(z["K"]), torch.from_numpy(z["viewmat"])
    fx, fy, cx, cy, vm_h, cc = B._camera(K, vm)
    sh_in, rest_in = B._sh_inputs(_t(z["sh_dc"], dev), None)
    with torch.no_grad():
        uv, conic, depth, rxy, valid, color = B._PreprocessMetal.apply(
            _t(z["means"], dev), _t(z["quats"], dev), _t(z["scales"], dev), sh_in, rest_in,
            _t(z["opacities"], dev), vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
            float(max(W, H)), cc, 0)
    v = z["valid"].astype(bool)
    assert np.array_equal(valid.cpu().numpy().astype(bool), v)
    for name, got in (("uv", uv), ("conic", conic), ("rxy", rxy), ("depth", depth),
                      ("color", color)):
        g, w = got.cpu().numpy()[v], z[name][v]
        # Relative to each Gaussian's own magnitude (a conic's small
        # off-diagonal term carries the rounding of its large diagonal ones).
        mag = np.abs(w).max(axis=-1, keepdims=True) if w.ndim > 1 else np.abs(w)
        err = np.abs(g - w) / np.maximum(mag, 1e-3 * np.abs(w).max())
        assert err.max() < 2e-5, (name, float(err.max()))


def test_config1_tile_lists_equal_fixture(dev):
    from metal_gauss_amd.backend import build_tile_lists_metal

    z = G.load("config1")
    W, H = int(z["W"]), int(z["H"])
    ids, off, tx = build_tile_lists_metal(
        _t(z["uv"], dev), _t(z["rxy"], dev), _t(z["depth"], dev),
        _t(z["valid"], dev, torch.int32), _t(z["conic"], dev), _t(z["opacities"], dev), W, H, 16)
    assert tx == 16
    assert np.array_equal(off.cpu().numpy(), z["tile_offsets"])
    assert np.array_equal(ids.cpu().numpy(), z["gauss_ids"])


def test_config1_image_matches_fixture(dev):
    from metal_gauss_amd import render

    z = G.load("config1")
    W, H = int(z["W"]), int(z["H"])
    with torch.no_grad():
        rgb, alpha, info = render(
            _t(z["means"], dev), _t(z["quats"], dev), _t(z["scales"], dev),
            _t(z["opacities"], dev), _t(z["sh_dc"], dev), torch.from_numpy(z["K"]),
            torch.from_numpy(z["viewmat"]), W, H, sh_degree=0, min_transmittance=0.0)
    assert info["isect_total"] == z["gauss_ids"].size
    ok = z["ambiguous"] == 0
    assert (~ok).mean() < 1e-3
    assert float(np.abs(rgb.cpu().numpy() - z["rgb"])[ok].max()) < 1e-4
    assert float(np.abs(alpha.cpu().numpy() - z["alpha"])[ok].max()) < 1e-4


def test_fwd_bwd_small_matches_fixture(dev):
    from metal_gauss_amd import render

    z = G.load("fwd_bwd_small")
    W, H = int(z["W"]), int(z["H"])
    names = ("means", "quats", "scales", "opacities", "sh")
    leaves = {k: _t(z[k], dev).requires_grad_(True) for k in names}
    rgb, alpha, _ = render(leaves["means"], leaves["quats"], leaves["scales"],
                           leaves["opacities"], leaves["sh"], torch.from_numpy(z["K"]),
                           torch.from_numpy(z["viewmat"]), W, H, sh_degree=3,
                           min_transmittance=0.0)
    ((rgb * _t(z["w_rgb"], dev)).sum() + (alpha * _t(z["w_alpha"], dev)).sum()).backward()
    assert float(np.abs(rgb.detach().cpu().double().numpy() - z["rgb"]).max()) < 1e-4
    assert float(np.abs(alpha.detach().cpu().double().numpy() - z["alpha"]).max()) < 1e-4
    for k in names:
        e = rel_l2(leaves[k].grad.cpu(), torch.from_numpy(z[f"d_{k}"]))
        assert e < 1e-3, (k, e)


def test_adam_matches_fixture(dev):
    from metal_gauss_amd import FusedAdam

    z = G.load("adam_small")
    for tag, eps in (("e15", 1e-15), ("e8", 1e-8)):
        p = _t(z["p0"], dev).requires_grad_(True)
        opt = FusedAdam([p], lr=float(z["lr"]), betas=(float(z["b1"]), float(z["b2"])), eps=eps)
        for g in z["grads"]:
            p.grad = _t(g, dev)
            opt.step()
        scale = float(np.abs(z[f"p_{tag}"]).max())
        assert float(np.abs(p.detach().cpu().numpy() - z[f"p_{tag}"]).max()) / scale < 1e-6
        st = opt.state[p]
        for k, name in (("m", "exp_avg"), ("v", "exp_avg_sq")):
            want = z[f"{k}_{tag}"]
            got = st[name].cpu().numpy()
            assert float(np.abs(got - want).max()) / float(np.abs(want).max()) < 1e-6, (tag, k)


def test_selective_adam_matches_fixture(dev):
    from metal_gauss_amd import SelectiveAdam

    z = G.load("adam_small")
    p = _t(z["sel_p0"], dev).requires_grad_(True)
    opt = SelectiveAdam([{"params": [p], "lr": float(z["lr"])}],
                        betas=(float(z["b1"]), float(z["b2"])), eps=1e-15)
    for g, m in zip(z["sel_grads"], z["sel_masks"]):
        p.grad = _t(g, dev)
        opt.step(_t(m, dev, torch.bool))
    scale = float(np.abs(z["sel_p"]).max())
    assert float(np.abs(p.detach().cpu().numpy() - z["sel_p"]).max()) / scale < 1e-6
    steps = opt.state[p]["steps"].cpu().numpy().reshape(-1)
    assert np.array_equal(steps.astype(np.float32), z["sel_steps"])
