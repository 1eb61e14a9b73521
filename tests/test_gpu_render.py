"""End-to-end render on the GPU against the PyTorch-CPU restatement of
torch_ref (oracle/render_ref.py), in the reference's test style
(tests/test_metal.py, test_sh_split_layout.py, test_antialias.py,
test_absgrad.py, test_boundary_culling.py).

Bars: images within 1e-4 max-abs, parameter
gradients within 1e-3 relative L2. The oracle runs in float64 and composites
every listed Gaussian (min_transmittance = 0); so does the GPU in these
comparisons, which isolates arithmetic from the early-stop heuristic (the
reference's kernel stops per pixel at T < 1e-4, its torch renderer per slab).
With the default early stop the difference is bounded by 1e-4 x max colour."""

from __future__ import annotations

import pytest
import torch

from conftest import intrinsics, rel_l2, scene
from oracle import render_ref

pytestmark = pytest.mark.gpu


def run(backend, s, W, H, dev, *, sh_degree=3, use_sh=False, grad=True, t_min=0.0, tile=16,
        background=(0.0, 0.0, 0.0), antialias=False, split=False):
    names = ["means", "quats", "scales", "opacities"] + (["sh"] if use_sh else ["colors"])
    if backend == "hip":
        leaves = {k: s[k].clone().to(dev).requires_grad_(grad) for k in names}
    else:
        leaves = {k: s[k].clone().double().requires_grad_(grad) for k in names}
    K = intrinsics(W, H)
    vm = torch.eye(4)
    if backend == "hip":
        from metal_gauss_amd import render
        kw = dict(sh_degree=sh_degree, tile=tile, min_transmittance=t_min,
                  background=background, antialias=antialias)
        if use_sh and split:
            dc = leaves["sh"][:, :1].detach().clone().requires_grad_(grad)
            rest = leaves["sh"][:, 1:].detach().clone().requires_grad_(grad)
            rgb, alpha, info = render(leaves["means"], leaves["quats"], leaves["scales"],
                                      leaves["opacities"], dc, K, vm, W, H, sh_rest=rest, **kw)
            leaves["sh_dc"], leaves["sh_rest"] = dc, rest
        elif use_sh:
            rgb, alpha, info = render(leaves["means"], leaves["quats"], leaves["scales"],
                                      leaves["opacities"], leaves["sh"], K, vm, W, H, **kw)
        else:
            rgb, alpha, info = render(leaves["means"], leaves["quats"], leaves["scales"],
                                      leaves["opacities"], None, K, vm, W, H,
                                      colors=leaves["colors"], **kw)
    else:
        rgb, alpha, info = render_ref.render(
            leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"],
            leaves.get("sh"), K.double(), vm.double(), W, H, sh_degree=sh_degree, tile=tile,
            colors=leaves.get("colors"), min_transmittance=t_min, background=background,
            antialias=antialias)
    if grad:
        (rgb.square().mean() + 0.1 * alpha.square().mean()).backward()
    return rgb.detach().cpu().double(), alpha.detach().cpu().double(), leaves, info


def max_abs(a, b):
    return float((a - b).abs().max())


@pytest.mark.parametrize("tile", [8, 16])
def test_repeated_backward_gives_the_same_gradients(dev, tile):
    """Each backward accumulates into per-Gaussian gradient records that the
    forward of the same render clears; two renders and backwards of the same
    scene must give the same gradients (equal up to the order of the float
    atomics), not the second one carrying the first one's sums."""
    s = scene(n=600, seed=7, sh=True)
    runs = [run("hip", s, 96, 80, dev, use_sh=True, tile=tile)[2] for _ in range(3)]
    for k in ("means", "quats", "scales", "opacities", "sh"):
        g0 = runs[0][k].grad
        assert g0 is not None and float(g0.abs().sum()) > 0, k
        for r in runs[1:]:
            assert rel_l2(r[k].grad.cpu(), g0.cpu()) < 1e-5, k


def test_forward_matches_reference(dev):
    W, H = 96, 64
    s = scene(n=400, seed=0)
    a = run("hip", s, W, H, dev, grad=False)
    b = run("ref", s, W, H, dev, grad=False)
    assert max_abs(a[0], b[0]) < 1e-4 and max_abs(a[1], b[1]) < 1e-4


def test_forward_with_sh_matches_reference(dev):
    W, H = 64, 64
    s = scene(n=250, seed=3)
    a = run("hip", s, W, H, dev, use_sh=True, grad=False)
    b = run("ref", s, W, H, dev, use_sh=True, grad=False)
    assert max_abs(a[0], b[0]) < 1e-4


def test_default_early_stop_is_within_its_bound(dev):
    """The kernel's per-pixel stop at T < 1e-4 drops at most T * max colour."""
    W, H = 96, 64
    s = scene(n=1500, seed=4, spread=0.4)
    a = run("hip", s, W, H, dev, grad=False, t_min=1e-4)
    b = run("ref", s, W, H, dev, grad=False, t_min=0.0)
    assert max_abs(a[0], b[0]) < 1e-4 * float(s["colors"].max()) + 1e-5


@pytest.mark.parametrize("use_sh", [False, True])
def test_gradients_match_reference(dev, use_sh):
    W, H = 64, 48
    s = scene(n=300, seed=11)
    a = run("hip", s, W, H, dev, use_sh=use_sh)
    b = run("ref", s, W, H, dev, use_sh=use_sh)
    assert max_abs(a[0], b[0]) < 1e-4
    for k, t in a[2].items():
        g = t.grad.detach().cpu().double()
        assert torch.isfinite(g).all(), k
        assert rel_l2(g, b[2][k].grad) < 1e-3, f"{k}: rel L2 {rel_l2(g, b[2][k].grad):.2e}"


@pytest.mark.parametrize("tile", [8, 12, 16, 32])
def test_every_tile_size_matches_reference(dev, tile):
    """tests/test_metal.py:174-202 with long, thin, rotated splats."""
    W, H = 100, 63
    s = scene(n=300, seed=17)
    s["scales"] = s["scales"] * torch.tensor([4.0, 0.5, 1.0])
    a = run("hip", s, W, H, dev, tile=tile)
    b = run("ref", s, W, H, dev, tile=tile)
    assert max_abs(a[0], b[0]) < 1e-4 and max_abs(a[1], b[1]) < 1e-4
    for k, t in a[2].items():
        assert rel_l2(t.grad.cpu(), b[2][k].grad) < 1e-3, k


def test_offscreen_gaussians_get_exactly_zero_gradient(dev):
    """tests/test_metal.py:120-150: half the scene pushed out of frame."""
    W, H = 64, 48
    n = 300
    s = scene(n=n, seed=13)
    off = torch.arange(n) % 2 == 1
    s["means"][off, 0] += 20.0
    a = run("hip", s, W, H, dev, use_sh=True)
    b = run("ref", s, W, H, dev, use_sh=True)
    for k in ("means", "quats", "scales", "sh"):
        g = a[2][k].grad.cpu()
        assert float(g[off].abs().max()) == 0.0, f"{k}: off-screen gradient"
        assert rel_l2(g, b[2][k].grad) < 1e-3, k


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_split_sh_matches_fused(dev, deg):
    """tests/test_sh_split_layout.py:44-67: image identical, SH gradients equal
    up to the atomic-accumulation order."""
    W, H = 96, 128
    s = scene(n=4000, seed=0, z=3.0, spread=0.4, scale=(0.01, 0.06))
    a = run("hip", s, W, H, dev, use_sh=True, sh_degree=deg)
    b = run("hip", s, W, H, dev, use_sh=True, sh_degree=deg, split=True)
    assert torch.equal(a[0], b[0])
    gf = a[2]["sh"].grad
    assert rel_l2(gf[:, :1].cpu(), b[2]["sh_dc"].grad.cpu()) < 1e-5
    if deg > 0:
        assert rel_l2(gf[:, 1:].cpu(), b[2]["sh_rest"].grad.cpu()) < 1e-5


def test_sh_gradient_is_not_doubled(dev):
    W, H = 96, 128
    s = scene(n=2000, seed=1, z=3.0, spread=0.4)
    from metal_gauss_amd import render

    sh1 = s["sh"].clone().to(dev).requires_grad_(True)
    args = [s[k].to(dev) for k in ("means", "quats", "scales", "opacities")]
    rgb, _, _ = render(*args, sh1, intrinsics(W, H), torch.eye(4), W, H)
    rgb.square().mean().backward()
    sh2 = s["sh"].clone().to(dev).requires_grad_(True)
    rgb2, _, _ = render(*args, sh2, intrinsics(W, H), torch.eye(4), W, H)
    (2.0 * rgb2).square().mean().backward()
    assert torch.allclose(sh2.grad, 4.0 * sh1.grad, rtol=1e-4, atol=1e-7)


def test_full_sh_with_sh_rest_is_rejected(dev):
    from metal_gauss_amd import render

    s = scene(n=20)
    with pytest.raises(ValueError, match="DC band"):
        render(*[s[k].to(dev) for k in ("means", "quats", "scales", "opacities")],
               s["sh"].to(dev), intrinsics(32, 32), torch.eye(4), 32, 32,
               sh_rest=s["sh"][:, 1:].to(dev))


def test_empty_scene_renders_the_background(dev):
    from metal_gauss_amd import render

    W, H = 48, 32
    z = lambda *sh: torch.zeros(*sh, device=dev)  # noqa: E731
    rgb, alpha, info = render(z(0, 3), z(0, 4), z(0, 3), z(0), z(0, 16, 3), intrinsics(W, H),
                              torch.eye(4), W, H, background=(1.0, 0.0, 0.0))
    assert torch.equal(rgb, torch.tensor([1.0, 0.0, 0.0], device=dev).expand(H, W, 3))
    assert float(alpha.max()) == 0.0 and info["isect_total"] == 0


def test_info_contract(dev):
    W, H = 96, 64
    s = scene(n=800, seed=5)
    _, _, leaves, info = run("hip", s, W, H, dev)
    assert info["backend"] == "hip" and info["isect_dropped"] == 0 and info["isect_total"] > 0
    assert info["tiles"] == 6 * 4
    assert info["valid_mask"].dtype == torch.bool and info["valid_mask"].shape == (800,)
    assert info["uv"].grad is not None and info["uv"].grad.shape == (800, 2)


def test_uv_grad_is_retained_like_retain_grad(dev):
    """info["uv"].grad (metal_backend.py:548-549 retains it for the
    trainer's densification statistics) equals the gradient at uv, sums over
    repeated backwards as retain_grad does, starts again after a reset, and
    raises no non-leaf warning."""
    import warnings

    from metal_gauss_amd import render

    W, H, n = 96, 64, 500
    s = scene(n=n, seed=12)
    args = (s["quats"].to(dev), s["scales"].to(dev), s["opacities"].to(dev), None,
            intrinsics(W, H), torch.eye(4), W, H)
    m = s["means"].to(dev).requires_grad_(True)
    # The gradient at uv from a separate render, by torch.autograd.grad.
    rgb0, _, info0 = render(m, *args, colors=s["colors"].to(dev))
    (g_ref,) = torch.autograd.grad(rgb0.square().mean(), info0["uv"])
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        rgb, _, info = render(m, *args, colors=s["colors"].to(dev))
        uv = info["uv"]
        loss = rgb.square().mean()
        loss.backward(retain_graph=True)
        g1 = uv.grad.clone()
        assert torch.allclose(g1, g_ref, rtol=1e-4, atol=1e-9) and float(g1.abs().max()) > 0
        loss.backward(retain_graph=True)
        assert torch.allclose(uv.grad, 2 * g1, rtol=1e-4, atol=1e-9)
        uv.grad = None
        loss.backward()
        assert torch.allclose(uv.grad, g1, rtol=1e-4, atol=1e-9)


def test_background_blend_matches_reference(dev):
    W, H = 96, 64
    s = scene(n=400, seed=8)
    a = run("hip", s, W, H, dev, grad=False, background=(1.0, 1.0, 1.0))
    b = run("ref", s, W, H, dev, grad=False, background=(1.0, 1.0, 1.0))
    assert max_abs(a[0], b[0]) < 1e-4


def test_antialias_matches_reference_and_darkens(dev):
    """tests/test_antialias.py:128-163."""
    W, H = 96, 64
    s = scene(n=400, seed=0, scale=(0.004, 0.034))
    a = run("hip", s, W, H, dev, grad=False, antialias=True)
    b = run("ref", s, W, H, dev, grad=False, antialias=True)
    assert max_abs(a[0], b[0]) < 1e-4
    off = run("hip", s, W, H, dev, grad=False, antialias=False)
    assert max_abs(off[0], a[0]) > 1e-4
    assert float(a[0].sum()) <= float(off[0].sum()) + 1e-3


def test_absgrad_buffer(dev):
    """tests/test_absgrad.py: populated, non-negative, dominates |d uv|."""
    from metal_gauss_amd import render

    W, H, n = 96, 64, 300
    s = scene(n=n, seed=0, scale=(0.02, 0.10))
    m = s["means"].to(dev).requires_grad_(True)
    buf = torch.zeros(n, device=dev)
    rgb, _, info = render(m, s["quats"].to(dev), s["scales"].to(dev), s["opacities"].to(dev),
                          None, intrinsics(W, H), torch.eye(4), W, H,
                          colors=s["colors"].to(dev), absgrad_out=buf)
    rgb.square().mean().backward()
    assert torch.isfinite(buf).all() and (buf >= 0).all() and buf.sum() > 0
    slack = buf - info["uv"].grad.norm(dim=1)
    assert (slack >= -1e-4 * buf.max()).all() and (slack > 1e-6 * buf.max()).any()


@pytest.mark.parametrize("lo,hi", [(28.0, 36.0), (-8.0, 8.0), (120.0, 136.0)])
def test_no_discontinuity_across_boundaries(dev, lo, hi):
    """tests/test_boundary_culling.py:50-66: sweeping a splat across a tile or
    screen edge changes the rendered energy continuously."""
    import numpy as np

    from metal_gauss_amd import render

    W = H = 128
    F, Z = 100.0, 2.0
    K = torch.tensor([[F, 0, W / 2], [0, F, H / 2], [0, 0, 1.0]])
    q = torch.tensor([[1.0, 0, 0, 0]], device=dev)
    sc = torch.full((1, 3), 0.04, device=dev)
    sh = torch.zeros(1, 16, 3, device=dev)
    sh[:, 0] = 1.0
    op = torch.tensor([0.99], device=dev)
    es = []
    for u in np.arange(lo, hi, 0.05):
        m = torch.tensor([[(u - W / 2) * Z / F, 0.0, Z]], device=dev, dtype=torch.float32)
        rgb, _, _ = render(m, q, sc, op, sh, K, torch.eye(4), W, H, tile=32)
        es.append(float(rgb.sum()))
    steps = np.abs(np.diff(es))
    assert steps.max() <= 8 * max(np.median(steps), 1e-9)


def test_chunked_backward_matches_single_chain(dev):
    """render(chunked_backward=True) runs the raster backward as 512-entry
    units per tile from forward checkpoints; same image, same gradients up to
    rounding (both recover T by division, from different starting points)."""
    from metal_gauss_amd import render

    s = scene(n=5000, seed=12, sh=True)
    W, H = 64, 48
    grads = []
    for chunked in (False, True):
        leaves = {k: s[k].clone().to(dev).requires_grad_(True)
                  for k in ("means", "quats", "scales", "opacities", "sh")}
        rgb, alpha, info = render(leaves["means"], leaves["quats"], leaves["scales"],
                                  leaves["opacities"], leaves["sh"], intrinsics(W, H),
                                  torch.eye(4), W, H, sh_degree=3, background=(1.0, 1.0, 1.0),
                                  chunked_backward=chunked)
        (rgb.square().mean() + 0.1 * alpha.square().mean()).backward()
        grads.append((rgb.detach(), {k: v.grad.detach().clone() for k, v in leaves.items()}))
    assert torch.equal(grads[0][0], grads[1][0])
    for k in grads[0][1]:
        e = rel_l2(grads[1][1][k].cpu(), grads[0][1][k].cpu())
        assert e < 1e-4, (k, e)


@pytest.mark.parametrize("use_sh", [False, True])
def test_preview_renders_exactly_what_training_renders(dev, use_sh):
    """tests/test_trainer.py:410-439: a forward-only render (no autograd, as
    the viewer and the video renderer call it) gives the same pixels, bit for
    bit, as the training render, here with the Mip 3D filter, antialias and a
    white background all on."""
    from metal_gauss_amd import render

    W, H = 128, 96
    s = scene(n=3000, seed=5, scale=(0.004, 0.05))
    g = torch.Generator().manual_seed(6)
    f3d = (torch.rand(3000, generator=g) * 0.01).to(dev)
    K = intrinsics(W, H)
    vm = torch.eye(4)
    names = ["means", "quats", "scales", "opacities"] + (["sh"] if use_sh else ["colors"])
    leaves = {k: s[k].clone().to(dev).requires_grad_(True) for k in names}
    kw = dict(antialias=True, filter_3d=f3d, background=(1.0, 1.0, 1.0))
    trained, a_t, _ = render(leaves["means"], leaves["quats"], leaves["scales"],
                             leaves["opacities"], leaves.get("sh"), K, vm, W, H,
                             colors=leaves.get("colors"), **kw)
    with torch.no_grad():
        previewed, a_p, _ = render(*(leaves[k].detach() for k in names[:4]),
                                   leaves["sh"].detach() if use_sh else None, K, vm, W, H,
                                   colors=None if use_sh else leaves["colors"].detach(), **kw)
    assert torch.equal(trained.detach(), previewed)
    assert torch.equal(a_t.detach(), a_p)


@pytest.mark.parametrize("antialias,filt,split", [(False, False, False), (False, False, True),
                                                  (True, False, False), (True, True, True)])
def test_activations_in_the_kernel_match_torch_activations(dev, antialias, filt, split):
    """render(activations=True) on log scales and logits against render on
    torch.exp / torch.sigmoid of them (the trainer's train.py:221-222), with
    and without Mip's filters: the same lists and image, and through torch's
    exp and sigmoid backward the same gradients on every leaf."""
    from metal_gauss_amd import render

    W, H = 96, 80
    s = scene(n=500, seed=7)
    K, vm = intrinsics(W, H), torch.eye(4)
    g = torch.Generator().manual_seed(8)
    f3 = (torch.rand(500, generator=g) * 0.02 + 0.005).to(dev) if filt else None
    base = dict(means=s["means"], quats=s["quats"], log_scales=s["scales"].log(),
                logits=torch.logit(s["opacities"]), sh=s["sh"])
    outs = []
    for fused in (False, True):
        p = {k: t.clone().to(dev).requires_grad_(True) for k, t in base.items()}
        if fused:
            sc, op = p["log_scales"], p["logits"]
        else:
            sc, op = torch.exp(p["log_scales"]), torch.sigmoid(p["logits"])
        if split:
            dc = p["sh"][:, :1]
            kw = dict(sh_rest=p["sh"][:, 1:])
        else:
            dc, kw = p["sh"], {}
        rgb, alpha, info = render(p["means"], p["quats"], sc, op, dc, K, vm, W, H, sh_degree=3,
                                  min_transmittance=0.0, antialias=antialias, filter_3d=f3,
                                  activations=fused, **kw)
        (rgb.square().mean() + 0.1 * alpha.square().mean()).backward()
        outs.append((rgb.detach(), alpha.detach(), {k: v.grad for k, v in p.items()}, info))
    (r0, a0, g0, i0), (r1, a1, g1, i1) = outs
    assert i0["isect_total"] == i1["isect_total"] > 0
    assert torch.equal(i0["valid_mask"], i1["valid_mask"])
    assert (r0 - r1).abs().max() < 1e-6 and (a0 - a1).abs().max() < 1e-6
    for k in base:
        assert g1[k] is not None and rel_l2(g1[k].cpu(), g0[k].cpu()) < 1e-5, k
    # The logit gradient is the opacity gradient through sigmoid: nonzero
    # where a Gaussian is drawn, exactly zero where it is not.
    assert (g1["logits"][~i1["valid_mask"]] == 0).all()
    assert g1["logits"].abs().sum() > 0
