"""Mip-Splatting's filters folded into the projection kernel, and the 3D
filter's size kernel, against oracle/mip_ref.py (float64 on the CPU).

The reference applies the 3D filter in torch before render
(train.py:223-227, mipfilter.py:76-93) and the 2D antialias factor in torch
after preprocess (metal_backend.py:506-511). Here both run inside
preprocess_fwd/bwd; the bar is the one of every preprocess test: outputs
within rounding of the float64 restatement, gradients within 1e-4 relative
L2 at the preprocess level and 1e-3 through the whole render; images within
1e-4 max-abs."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import intrinsics, rel_l2, scene
from oracle import mip_ref, render_ref

pytestmark = pytest.mark.gpu


def make(n, seed, off_frac=0.1, small=True):
    # Small Gaussians so that a good share are sub-pixel and both filters bite.
    s = scene(n=n, seed=seed, spread=0.8, scale=(0.002, 0.03) if small else (0.01, 0.12))
    g = torch.Generator().manual_seed(100 + seed)
    s["filter_3d"] = torch.rand(n, generator=g) * 0.01
    k = int(n * off_frac)
    s["means"][:k, 0] += 25.0
    s["means"][k:2 * k, 2] = -3.0
    return s


def gpu_pre(s, W, H, dev, *, filt=True, aa=True, deg=3, split=False, grad=True):
    from metal_gauss_amd.backend import _PreprocessMip, _camera

    K = intrinsics(W, H)
    fx, fy, cx, cy, vm_h, cc = _camera(K, torch.eye(4))
    leaves = {k: s[k].clone().to(dev).requires_grad_(grad)
              for k in ("means", "quats", "scales", "opacities")}
    sh = s["sh"].clone().to(dev)
    if split:
        leaves["sh_dc"] = sh[:, :1].contiguous().requires_grad_(grad)
        leaves["sh_rest"] = sh[:, 1:].contiguous().requires_grad_(grad)
        sh_args = (leaves["sh_dc"], leaves["sh_rest"])
    else:
        leaves["sh"] = sh.requires_grad_(grad)
        sh_args = (leaves["sh"], None)
    f = s["filter_3d"].to(dev) if filt else None
    out = _PreprocessMip.apply(leaves["means"], leaves["quats"], leaves["scales"],
                               leaves["opacities"], *sh_args, f, aa, vm_h, fx, fy, cx, cy, W, H,
                               0.01, 100.0, 0.3, float(max(W, H)), cc, deg)
    return out, leaves


def ref_pre(s, W, H, *, filt=True, aa=True, deg=3):
    K = intrinsics(W, H).double()
    leaves = {k: s[k].clone().double().requires_grad_(True)
              for k in ("means", "quats", "scales", "opacities", "sh")}
    out = mip_ref.preprocess_mip(
        leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"], leaves["sh"],
        torch.eye(4, dtype=torch.float64), float(K[0, 0]), float(K[1, 1]), float(K[0, 2]),
        float(K[1, 2]), W, H, sh_degree=deg,
        filter_3d=s["filter_3d"].double() if filt else None, antialias=aa)
    return out, leaves


@pytest.mark.parametrize("filt,aa", [(True, True), (True, False), (False, True)])
def test_forward_matches_contract(dev, filt, aa):
    W, H = 160, 120
    s = make(3000, 1, off_frac=0.1)
    out, _ = gpu_pre(s, W, H, dev, filt=filt, aa=aa, grad=False)
    uv, conic, depth, rxy, valid, color, op = out
    rout, _ = ref_pre(s, W, H, filt=filt, aa=aa)
    ruv, rconic, _, rrxy, rvalid, rcolor, rop = rout
    agree = (valid.cpu() != 0) == rvalid
    assert float(agree.double().mean()) > 0.999, f"{int((~agree).sum())} validity flips"
    both = agree & rvalid

    def rel(a, b):
        b = b.detach()
        floor = 1e-3 * float(b.abs().max())
        return float(((a.cpu().double() - b).abs() / (b.abs() + floor)).max())

    assert rel(uv[both], ruv[both]) < 1e-5
    assert rel(conic[both], rconic[both]) < 1e-4
    assert rel(rxy[both], rrxy[both]) < 1e-4
    assert float((color[both].cpu().double() - rcolor[both].detach()).abs().max()) < 1e-5
    # The effective opacity: the determinant ratios of sub-pixel Gaussians
    # cancel, so compare against the float64 value with an absolute floor.
    err = (op[both].cpu().double() - rop[both].detach()).abs()
    assert float(err.max()) < 5e-5, float(err.max())
    assert bool((op.cpu() <= s["opacities"] + 1e-6).all())
    if aa or filt:
        assert float((s["opacities"][both] - op[both].cpu()).abs().max()) > 1e-2


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("filt,aa", [(True, True), (True, False), (False, True)])
def test_backward_matches_autograd(dev, filt, aa, split):
    W, H = 160, 120
    s = make(2000, 2, off_frac=0.1)
    out, leaves = gpu_pre(s, W, H, dev, filt=filt, aa=aa, split=split)
    uv, conic, _, _, valid, color, op = out
    rout, rleaves = ref_pre(s, W, H, filt=filt, aa=aa)
    ruv, rconic, _, _, rvalid, rcolor, rop = rout
    n = s["means"].shape[0]
    g = torch.Generator().manual_seed(3)
    mask = ((valid.cpu() != 0) & rvalid).double()
    cot = [torch.randn(n, 2, generator=g).double() * mask[:, None],
           torch.randn(n, 3, generator=g).double() * mask[:, None],
           torch.randn(n, 3, generator=g).double() * mask[:, None],
           torch.randn(n, generator=g).double() * mask]
    torch.autograd.backward([uv, conic, color, op], [c.float().to(dev) for c in cot])
    torch.autograd.backward([ruv, rconic, rcolor, rop], cot)
    for name in ("means", "quats", "scales", "opacities"):
        e = rel_l2(leaves[name].grad.cpu(), rleaves[name].grad)
        assert e < 1e-4, f"{name}: rel L2 {e:.2e}"
    gsh = (torch.cat([leaves["sh_dc"].grad, leaves["sh_rest"].grad], 1) if split
           else leaves["sh"].grad)
    assert rel_l2(gsh.cpu(), rleaves["sh"].grad) < 1e-4
    inval = valid.cpu() == 0
    assert float(leaves["opacities"].grad[inval].abs().max()) == 0.0


def _render_pair(s, W, H, dev, *, use_sh, filt, aa, t_min=0.0):
    from metal_gauss_amd import render

    names = ["means", "quats", "scales", "opacities"] + (["sh"] if use_sh else ["colors"])
    hip = {k: s[k].clone().to(dev).requires_grad_(True) for k in names}
    ref = {k: s[k].clone().double().requires_grad_(True) for k in names}
    K = intrinsics(W, H)
    vm = torch.eye(4)
    f = s["filter_3d"]
    rgb, alpha, _ = render(hip["means"], hip["quats"], hip["scales"], hip["opacities"],
                           hip.get("sh"), K, vm, W, H, colors=hip.get("colors"),
                           min_transmittance=t_min, antialias=aa,
                           filter_3d=f.to(dev) if filt else None)
    sc, op = ref["scales"], ref["opacities"]
    if filt:
        sc, op = mip_ref.apply_3d_filter(sc, op, f.double())
    rrgb, ralpha, _ = render_ref.render(ref["means"], ref["quats"], sc, op, ref.get("sh"),
                                        K.double(), vm.double(), W, H, colors=ref.get("colors"),
                                        min_transmittance=t_min, antialias=aa)
    (rgb.square().mean() + 0.1 * alpha.square().mean()).backward()
    (rrgb.square().mean() + 0.1 * ralpha.square().mean()).backward()
    return (rgb, alpha, hip), (rrgb, ralpha, ref)


@pytest.mark.parametrize("use_sh", [False, True])
@pytest.mark.parametrize("filt,aa", [(True, True), (True, False), (False, True)])
def test_render_matches_reference(dev, use_sh, filt, aa):
    """render(filter_3d=, antialias=) against the reference's route: torch
    apply_3d_filter, then torch_ref.render(antialias=...)."""
    W, H = 96, 64
    s = make(600, 4 + use_sh, off_frac=0.05)
    (rgb, alpha, hip), (rrgb, ralpha, ref) = _render_pair(s, W, H, dev, use_sh=use_sh,
                                                          filt=filt, aa=aa)
    assert float((rgb.detach().cpu().double() - rrgb.detach()).abs().max()) < 1e-4
    assert float((alpha.detach().cpu().double() - ralpha.detach()).abs().max()) < 1e-4
    for k in hip:
        e = rel_l2(hip[k].grad.cpu(), ref[k].grad)
        assert e < 1e-3, f"{k}: rel L2 {e:.2e}"


def test_fused_filter_equals_the_torch_reparameterisation(dev):
    """render(filter_3d=f) and render(*apply_3d_filter(...)) run the same
    kernels on inputs that differ only by the rounding of the filter."""
    from metal_gauss_amd import apply_3d_filter, render

    W, H = 128, 96
    s = make(2000, 6, off_frac=0.0)
    K = intrinsics(W, H)
    m, q, sc, op, sh = (s[k].to(dev) for k in ("means", "quats", "scales", "opacities", "sh"))
    f = s["filter_3d"].to(dev)
    a = render(m, q, sc, op, sh, K, torch.eye(4), W, H, filter_3d=f)[0]
    b = render(m, q, *apply_3d_filter(sc, op, f), sh, K, torch.eye(4), W, H)[0]
    assert float((a - b).abs().max()) < 1e-4
    c = render(m, q, sc, op, sh, K, torch.eye(4), W, H)[0]
    assert float((a - c).abs().max()) > 1e-3, "the filter changed nothing"


class _View:
    def __init__(self, K, vm, W, H):
        self.K, self.viewmat = K, vm
        self.image = torch.zeros(H, W, 3, dtype=torch.uint8)


def _look_at(eye, target=(0.0, 0.0, 0.0)):
    eye = np.asarray(eye, dtype=np.float64)
    fwd = np.asarray(target) - eye
    fwd /= np.linalg.norm(fwd)
    right = np.cross(fwd, [0.0, 1.0, 0.0])
    if np.linalg.norm(right) < 1e-9:
        right = np.array([1.0, 0.0, 0.0])
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    R = np.stack([right, down, fwd])
    vm = np.eye(4)
    vm[:3, :3] = R
    vm[:3, 3] = -R @ eye
    return vm


@pytest.mark.parametrize("n_views", [1, 7, 300])
def test_compute_3d_filter_matches_oracle(dev, n_views):
    from metal_gauss_amd import compute_3d_filter

    g = np.random.default_rng(n_views)
    n = 20000
    means = (g.standard_normal((n, 3)) * 1.5).astype(np.float32)
    views, tuples = [], []
    for i in range(n_views):
        W, H = int(g.integers(200, 900)), int(g.integers(200, 900))
        f = float(g.uniform(300, 1200))
        K = np.array([[f, 0, W / 2], [0, f, H / 2], [0, 0, 1.0]])
        eye = g.standard_normal(3)
        eye = eye / np.linalg.norm(eye) * g.uniform(3.0, 6.0)
        vm = _look_at(eye)
        # The views are float32 tensors, as a trainer holds them.
        K32, vm32 = K.astype(np.float32), vm.astype(np.float32)
        views.append(_View(torch.from_numpy(K32), torch.from_numpy(vm32), W, H))
        tuples.append((K32.astype(np.float64), vm32.astype(np.float64), W, H))
    got = compute_3d_filter(torch.from_numpy(means).to(dev), views).cpu().numpy()
    want = mip_ref.compute_3d_filter(means.astype(np.float64), tuples)
    rel = np.abs(got - want) / want
    # A Gaussian within rounding of a frame or near-plane bound may flip its
    # visibility in one view: allow a handful, all others to float rounding.
    bad = rel > 2e-6
    assert bad.sum() <= max(2, n // 2000), f"{bad.sum()} mismatches, worst {rel.max():.2e}"


def test_compute_3d_filter_reference_cases(dev):
    """tests/test_mipfilter.py:108-144 on the GPU kernel."""
    from metal_gauss_amd import compute_3d_filter

    def view(z, f=1000.0, hw=(400, 400)):
        K = torch.tensor([[f, 0, hw[1] / 2], [0, f, hw[0] / 2], [0, 0, 1.0]])
        vm = torch.eye(4)
        vm[2, 3] = z
        return _View(K, vm, hw[1], hw[0])

    m = torch.tensor([[0.0, 0.0, 0.0], [0.0, 0.0, 3.0]], device=dev)
    f = compute_3d_filter(m, [view(5.0)]).cpu()
    assert float(f[1]) > float(f[0]) > 0
    assert float(f[0]) == pytest.approx(5.0 / 1000.0 * math.sqrt(0.2), rel=1e-6)
    lo = compute_3d_filter(torch.zeros(1, 3, device=dev), [view(5.0, 500.0)])
    hi = compute_3d_filter(torch.zeros(1, 3, device=dev), [view(5.0, 2000.0)])
    assert float(hi) < float(lo)
    m = torch.tensor([[0.0, 0.0, 0.0], [0.0, 0.0, -100.0]], device=dev)
    f = compute_3d_filter(m, [view(5.0)]).cpu()
    assert bool(torch.isfinite(f).all()) and float(f[1]) == float(f[0])
    none = compute_3d_filter(torch.tensor([[0.0, 0.0, -50.0]], device=dev), [view(5.0, 400.0)])
    assert float(none) == pytest.approx(1.0 / 400.0 * math.sqrt(0.2), rel=1e-6)
    empty = compute_3d_filter(torch.zeros(0, 3, device=dev), [view(5.0)])
    assert empty.numel() == 0
