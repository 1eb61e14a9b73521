"""The fused preprocess kernels against the oracle's preprocess contract
(oracle/render_ref.preprocess, float64 on the CPU): projection, conic, depth,
SnugBox extents, validity and SH colour forward; the analytic backward against
torch autograd of the same restatement. Both SH layouts, degrees 0-3."""

from __future__ import annotations

import pytest
import torch

from conftest import intrinsics, rel_l2, scene
from oracle import render_ref

pytestmark = pytest.mark.gpu


def make(n, seed, W, H, off_frac=0.0):
    s = scene(n=n, seed=seed, spread=0.8, scale=(0.01, 0.12))
    if off_frac:
        k = int(n * off_frac)
        s["means"][:k, 0] += 25.0          # far outside the frustum
        s["means"][k:2 * k, 2] = -3.0      # behind the camera
    return s


def gpu_pre(s, W, H, dev, deg=3, split=False, grad=False, unaligned=False):
    """unaligned: the split rest rows handed over as a view one float into
    its storage (not 16-byte aligned), which the kernels must read as they
    are."""
    from metal_gauss_amd.backend import _PreprocessMetal, _camera

    K = intrinsics(W, H)
    fx, fy, cx, cy, vm_h, cc = _camera(K, torch.eye(4))
    leaves = [s[k].clone().to(dev).requires_grad_(grad) for k in ("means", "quats", "scales")]
    sh = s["sh"].clone().to(dev)
    if split:
        dc = sh[:, :1].contiguous().requires_grad_(grad)
        rest = sh[:, 1:].contiguous().requires_grad_(grad)
        shl = [dc, rest]
        rest_in = rest
        if unaligned:
            pad = torch.zeros(1, device=dev)
            rest_in = torch.cat([pad, rest.flatten()])[1:].view(rest.shape)
            assert rest_in.data_ptr() % 16 != 0
    else:
        shl = [sh.requires_grad_(grad), None]
        rest_in = None
    out = _PreprocessMetal.apply(*leaves, shl[0], rest_in, s["opacities"].to(dev), vm_h, fx,
                                 fy, cx, cy, W, H, 0.01, 100.0, 0.3, float(max(W, H)), cc, deg)
    return out, leaves, shl


def ref_pre(s, W, H, deg=3):
    K = intrinsics(W, H).double()
    leaves = [s[k].clone().double().requires_grad_(True) for k in ("means", "quats", "scales", "sh")]
    out = render_ref.preprocess(leaves[0], leaves[1], leaves[2], s["opacities"].double(),
                                leaves[3], torch.eye(4, dtype=torch.float64), float(K[0, 0]),
                                float(K[1, 1]), float(K[0, 2]), float(K[1, 2]), W, H,
                                sh_degree=deg)
    return out, leaves


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_forward_matches_contract(dev, deg):
    W, H = 160, 120
    s = make(3000, deg, W, H, off_frac=0.2)
    (uv, conic, depth, rxy, valid, color), _, _ = gpu_pre(s, W, H, dev, deg)
    (ruv, rconic, rdepth, rrxy, rvalid, rcolor), _ = ref_pre(s, W, H, deg)
    v = rvalid.numpy()
    agree = (valid.cpu().numpy() != 0) == v
    # A validity flip needs a screen-edge test within rounding: count them.
    assert agree.mean() > 0.999, f"{(~agree).sum()} validity flips"
    both = torch.from_numpy(agree & v)
    def tol(a, b):
        # Relative error per element, with the denominator floored at 1e-3 of
        # the tensor's largest magnitude (uv near 0 is not ill-conditioned).
        b = b.detach()
        floor = 1e-3 * float(b.abs().max())
        return float(((a.cpu().double() - b).abs() / (b.abs() + floor)).max())
    assert tol(uv[both], ruv[both]) < 1e-5
    assert tol(conic[both], rconic[both]) < 1e-4
    assert tol(depth[both], rdepth[both]) < 1e-6
    assert tol(rxy[both], rrxy[both]) < 1e-4
    assert float((color[both].cpu().double() - rcolor[both].detach()).abs().max()) < 1e-5
    # Invalid Gaussians carry no colour (preprocess.metal:207).
    inval = torch.from_numpy((valid.cpu().numpy() == 0))
    assert float(color[inval].abs().max()) == 0.0 if inval.any() else True


@pytest.mark.parametrize("split,n,unaligned", [(False, 2000, False), (True, 2000, False),
                                               (False, 2003, False), (True, 2011, False),
                                               (True, 2000, True)])
@pytest.mark.parametrize("deg", [0, 1, 3])
def test_backward_matches_autograd(dev, deg, split, n, unaligned):
    """Also: counts that end inside a 16-Gaussian round of the SH phase, and
    split rest rows that are not 16-byte aligned (the rows are then read and
    written without staging)."""
    W, H = 160, 120
    s = make(n, 10 + deg, W, H, off_frac=0.1)
    (uv, conic, depth, rxy, valid, color), leaves, shl = gpu_pre(s, W, H, dev, deg, split, True,
                                                                 unaligned)
    (ruv, rconic, _, _, rvalid, rcolor), rleaves = ref_pre(s, W, H, deg)
    g = torch.Generator().manual_seed(deg)
    n = s["means"].shape[0]
    # Upstream gradients only where both sides agree the Gaussian is valid:
    # the rasteriser never sends gradient to an invalid one.
    mask = ((valid.cpu() != 0) & rvalid).double()
    d_uv = torch.randn(n, 2, generator=g).double() * mask[:, None]
    d_conic = torch.randn(n, 3, generator=g).double() * mask[:, None]
    d_col = torch.randn(n, 3, generator=g).double() * mask[:, None]
    d_col[::7] = 0.0                      # rows that skip the SH branch
    torch.autograd.backward([uv, conic, color],
                            [d_uv.float().to(dev), d_conic.float().to(dev), d_col.float().to(dev)])
    torch.autograd.backward([ruv, rconic, rcolor], [d_uv, d_conic, d_col])
    for name, a, b in zip(("means", "quats", "scales"), leaves, rleaves):
        assert rel_l2(a.grad.cpu(), b.grad) < 1e-4, f"{name}: {rel_l2(a.grad.cpu(), b.grad):.2e}"
    nb = (deg + 1) ** 2
    gsh = torch.cat([shl[0].grad, shl[1].grad], 1) if split else shl[0].grad
    assert rel_l2(gsh[:, :nb].cpu(), rleaves[3].grad[:, :nb]) < 1e-4
    assert float(gsh[:, nb:].abs().max() if nb < 16 else 0.0) == 0.0
    # Invalid rows: exact zeros for quats and scales.
    inval = valid.cpu() == 0
    assert float(leaves[1].grad[inval].abs().max()) == 0.0
    assert float(leaves[2].grad[inval].abs().max()) == 0.0
