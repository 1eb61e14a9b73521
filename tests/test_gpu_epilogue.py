"""FusedAdam's update as the projection backward's epilogue
(render(optimizer=)) against the reference's order of work: the backward,
then FusedAdam.step() (train.py:389-400 with fused_adam.py:26-54).

With the same incoming gradients the epilogue computes the same parameter
gradients and applies the same update function (one shared device routine,
bias corrections formed in double on the host; the library compiles both
files with multiply-add fusion limited to single expressions, so the two
instantiations of the gradient arithmetic round alike), so parameters and
both moments must agree bit for bit. Through a whole render the rasteriser's
backward accumulates gradients with float atomics, whose order differs run
to run; there the bar is elementwise closeness of the update for all but a
1e-3 fraction of elements."""

from __future__ import annotations

import pytest
import torch

from conftest import intrinsics, rel_l2, scene

pytestmark = pytest.mark.gpu

NAMES = ("means", "quats", "log_scales", "logits", "sh_dc", "sh_rest")
LRS = {"means": 1.6e-4, "quats": 1e-3, "log_scales": 5e-3, "logits": 5e-2, "sh_dc": 2.5e-3,
       "sh_rest": 1.25e-4, "sh": 2.5e-3}


def _leaves(s, dev, split):
    base = dict(means=s["means"], quats=s["quats"], log_scales=s["scales"].log(),
                logits=torch.logit(s["opacities"]))
    if split:
        base["sh_dc"] = s["sh"][:, :1].contiguous()
        base["sh_rest"] = s["sh"][:, 1:].contiguous()
    else:
        base["sh"] = s["sh"]
    return {k: t.clone().to(dev).requires_grad_(True) for k, t in base.items()}


def _opt(p):
    from metal_gauss_amd import FusedAdam

    return FusedAdam([{"params": [t], "lr": LRS[k]} for k, t in p.items()], eps=1e-15)


@pytest.mark.parametrize("split,mip,reg", [(True, False, None), (False, False, None),
                                           (True, True, None), (True, False, (0.01, 0.01)),
                                           (False, True, (0.03, 0.002))])
def test_epilogue_equals_backward_then_step_bitwise(dev, split, mip, reg):
    """Two steps through the projection function with fixed seeded incoming
    gradients (second step on the updated parameters, with new gradients):
    epilogue path and backward + step() agree exactly on parameters,
    exp_avg and exp_avg_sq. N = 5007 leaves a partial last SH round; part of
    the Gaussians lie behind the camera (invalid rows get the update of a
    zero gradient, as FusedAdam gives them, plus the regularisers' gradient
    when ``reg`` is given)."""
    from metal_gauss_amd import backend

    n, W, H = 5007, 160, 120
    s = scene(n=n, seed=11)
    s["means"][: n // 5, 2] *= -1.0           # behind the camera
    K, vm = intrinsics(W, H), torch.eye(4)
    fx, fy, cx, cy, vm_h, cam = backend._camera(K, vm)
    g = torch.Generator().manual_seed(12)
    f3d = (torch.rand(n, generator=g) * 0.02).to(dev) if mip else None
    runs = []
    for fused in (True, False):
        p = _leaves(s, dev, split)
        opt = _opt(p)
        gg = torch.Generator().manual_seed(13)
        for _ in range(2):
            valid_b = torch.empty(n, dtype=torch.bool, device=dev)
            dc = p["sh_dc"] if split else p["sh"]
            rest = p["sh_rest"] if split else None
            outs = backend._PreprocessMip.apply(
                p["means"], p["quats"], p["log_scales"], p["logits"], dc, rest, f3d, mip, vm_h,
                fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3, float(max(W, H)), cam, 3, valid_b, 3,
                opt if fused else None, reg)
            uv, conic, _, _, _, color, op_eff = outs
            grads = [torch.randn(t.shape, generator=gg).to(dev) * 1e-2
                     for t in (uv, conic, color, op_eff)]
            opt.zero_grad(set_to_none=True)
            torch.autograd.backward([uv, conic, color, op_eff], grads)
            if fused:
                assert all(t.grad is None for t in p.values())
            else:
                assert all(t.grad is not None for t in p.values())
            opt.step()
        assert bool(valid_b.any()) and not bool(valid_b.all())
        runs.append({k: (t.detach().clone(), opt.state[t]["exp_avg"].clone(),
                         opt.state[t]["exp_avg_sq"].clone(), opt.state[t]["step"])
                     for k, t in p.items()})
    fused_run, plain_run = runs
    for k in fused_run:
        pf, mf, vf, sf = fused_run[k]
        pp, mp, vp, sp = plain_run[k]
        assert sf == sp == 2, k
        assert torch.equal(mf, mp), k
        assert torch.equal(vf, vp), k
        assert torch.equal(pf, pp), k


def test_render_with_optimizer_matches_backward_then_step(dev):
    """The config-4 step's shape (split SH, activations, photometric loss):
    one step with render(optimizer=) against render, backward, step(). The
    gradients differ only by the rasteriser's atomic summation order."""
    from metal_gauss_amd import gaussian_kernel, photometric_loss, render

    n, W, H = 4000, 128, 96
    s = scene(n=n, seed=21, scale=(0.01, 0.06))
    K, vm = intrinsics(W, H), torch.eye(4)
    gt = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(22)).to(dev)
    window = gaussian_kernel(device=dev, groups=15)
    start = _leaves(s, dev, True)
    res = []
    for fused in (True, False):
        p = {k: t.detach().clone().requires_grad_(True) for k, t in start.items()}
        opt = _opt(p)
        rgb, _, info = render(p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"],
                              K, vm, W, H, sh_degree=3, sh_rest=p["sh_rest"],
                              background=(0.0, 0.0, 0.0), activations=True,
                              optimizer=opt if fused else None)
        loss, _ = photometric_loss(rgb, gt, window, 0.2)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        assert all((t.grad is None) == fused for t in p.values())
        opt.step()
        assert info["uv"].grad is not None
        res.append({k: t.detach() - start[k].detach() for k, t in p.items()})
    # At step 1 every element with a nonzero gradient moves by about its lr;
    # a gradient that rounds to the other sign under another summation order
    # (a near-exact cancellation) flips its element's update, so the bar
    # allows a 1e-3 fraction of elements outside the tolerance.
    for k in NAMES:
        a, b = res[0][k].cpu(), res[1][k].cpu()
        assert a.abs().sum() > 0, k
        close = torch.isclose(a, b, rtol=1e-3, atol=1e-4 * LRS[k])
        assert float(close.double().mean()) > 0.999, k
        assert rel_l2(a, b) < 5e-2, k


def test_optimizer_falls_back_when_a_parameter_is_not_a_leaf(dev):
    """torch.exp / torch.sigmoid in front of render (train.py:221-222): the
    scales and opacities handed to render are not the optimizer's
    parameters, so the backward returns every gradient and step() makes the
    update; no step is counted early."""
    from metal_gauss_amd import render

    n, W, H = 1000, 96, 80
    s = scene(n=n, seed=31)
    K, vm = intrinsics(W, H), torch.eye(4)
    p = _leaves(s, dev, True)
    opt = _opt(p)
    rgb, alpha, _ = render(p["means"], p["quats"], torch.exp(p["log_scales"]),
                           torch.sigmoid(p["logits"]), p["sh_dc"], K, vm, W, H, sh_degree=3,
                           sh_rest=p["sh_rest"], antialias=True, optimizer=opt)
    (rgb.square().mean() + 0.1 * alpha.square().mean()).backward()
    assert all(t.grad is not None for t in p.values())
    assert all(not opt.state[t] or opt.state[t]["step"] == 0 for t in p.values())
    before = {k: t.detach().clone() for k, t in p.items()}
    opt.step()
    assert all(opt.state[t]["step"] == 1 for t in p.values())
    assert any(not torch.equal(before[k], p[k].detach()) for k in p)


def _trainer_reg(p, w_o=0.01, w_s=0.01):
    """The reference trainer's regularisers in torch (train.py:396-398)."""
    return w_o * torch.sigmoid(p["logits"]).mean() + w_s * torch.exp(p["log_scales"]).mean()


def test_regularisers_in_the_kernel_equal_torch_autograd(dev):
    """render's opacity_reg / scale_reg: the projection backward adds the
    gradient of w_o mean(sigmoid(logit)) + w_s mean(exp(log_scale)) to every
    row, visible or not. Against the same regularisers written in torch and
    differentiated by autograd (train.py:396-398) on the same incoming
    gradients: equal up to float rounding of the sum."""
    from metal_gauss_amd import backend

    n, W, H = 3001, 128, 96
    s = scene(n=n, seed=41)
    s["means"][: n // 4, 2] *= -1.0           # a quarter behind the camera: reg only
    K, vm = intrinsics(W, H), torch.eye(4)
    fx, fy, cx, cy, vm_h, cam = backend._camera(K, vm)
    got = []
    for in_kernel in (True, False):
        p = _leaves(s, dev, True)
        valid_b = torch.empty(n, dtype=torch.bool, device=dev)
        outs = backend._PreprocessMip.apply(
            p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"], p["sh_rest"],
            None, False, vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3, float(max(W, H)), cam, 3,
            valid_b, 3, None, (0.01, 0.02) if in_kernel else None)
        uv, conic, _, _, _, color, op_eff = outs
        gg = torch.Generator().manual_seed(42)
        grads = [torch.randn(t.shape, generator=gg).to(dev) * 1e-2
                 for t in (uv, conic, color, op_eff)]
        tensors = [uv, conic, color, op_eff]
        if not in_kernel:
            tensors.append(_trainer_reg(p, 0.01, 0.02))
            grads.append(torch.ones((), device=dev))
        torch.autograd.backward(tensors, grads)
        got.append({k: t.grad.detach().cpu().double() for k, t in p.items()})
    assert not bool(valid_b.all())
    for k in got[0]:
        a, b = got[0][k], got[1][k]
        tol = 1e-6 * float(b.abs().max()) + 1e-12
        assert float((a - b).abs().max()) <= tol, k
    # The invisible rows' log-scale and logit gradients are the
    # regularisers' alone, and nonzero.
    inv = ~valid_b.cpu()
    assert float(got[0]["logits"][inv].abs().min()) > 0
    assert float(got[0]["log_scales"][inv].abs().min()) > 0


def test_trainer_loss_with_regularisers_through_the_epilogue(dev):
    """The reference trainer's default loss (photometric + 0.01 mean
    sigmoid(logit) + 0.01 mean exp(log scale), train.py:389-398 with the
    defaults at 733-734): render(optimizer=, opacity_reg=, scale_reg=) and
    step() against render, the regularisers in torch, backward and step();
    the same bar as the photometric-only comparison above. The loss value
    with info["regularizer"]() equals the torch loss."""
    from metal_gauss_amd import gaussian_kernel, photometric_loss, render

    n, W, H = 4000, 128, 96
    s = scene(n=n, seed=51, scale=(0.01, 0.06))
    K, vm = intrinsics(W, H), torch.eye(4)
    gt = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(52)).to(dev)
    window = gaussian_kernel(device=dev, groups=15)
    start = _leaves(s, dev, True)
    res, losses = [], []
    for fused in (True, False):
        p = {k: t.detach().clone().requires_grad_(True) for k, t in start.items()}
        opt = _opt(p)
        for it in range(2):
            kw = dict(optimizer=opt, opacity_reg=0.01, scale_reg=0.01) if fused else {}
            rgb, _, info = render(p["means"], p["quats"], p["log_scales"], p["logits"],
                                  p["sh_dc"], K, vm, W, H, sh_degree=3, sh_rest=p["sh_rest"],
                                  activations=True, **kw)
            loss, _ = photometric_loss(rgb, gt, window, 0.2)
            if fused:
                total = loss.detach() + info["regularizer"]()
            else:
                loss = loss + _trainer_reg(p)
                total = loss.detach()
            opt.zero_grad(set_to_none=True)
            loss.backward()
            assert all((t.grad is None) == fused for t in p.values())
            opt.step()
            if it == 0:
                losses.append(float(total))
        res.append({k: t.detach() - start[k].detach() for k, t in p.items()})
        assert all(opt.state[t]["step"] == 2 for t in p.values())
    assert abs(losses[0] - losses[1]) <= 1e-6 * abs(losses[1])
    for k in NAMES:
        a, b = res[0][k].cpu(), res[1][k].cpu()
        assert a.abs().sum() > 0, k
        close = torch.isclose(a, b, rtol=1e-3, atol=1e-4 * LRS[k])
        assert float(close.double().mean()) > 0.999, k
        assert rel_l2(a, b) < 5e-2, k


def test_step_refuses_a_second_update_after_the_epilogue(dev):
    """A loss that uses the parameters outside render(optimizer=) (the
    trainer's regularisers written in torch) reaches them as .grad after the
    epilogue has updated them: step() raises instead of taking a second Adam
    step, and leaves every parameter and step count as the epilogue left
    them, also when it is called again; once the gradients are cleared,
    step() closes the step without an update. A second render(optimizer=)
    before step() raises too."""
    from metal_gauss_amd import render

    n, W, H = 1000, 96, 80
    s = scene(n=n, seed=61)
    K, vm = intrinsics(W, H), torch.eye(4)
    p = _leaves(s, dev, True)
    opt = _opt(p)
    rgb, alpha, _ = render(p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"], K,
                           vm, W, H, sh_degree=3, sh_rest=p["sh_rest"], activations=True,
                           optimizer=opt)
    opt.zero_grad(set_to_none=True)
    (rgb.square().mean() + _trainer_reg(p)).backward()
    assert p["logits"].grad is not None and p["means"].grad is None
    after = {k: t.detach().clone() for k, t in p.items()}
    for _ in range(2):     # a retried step() is refused again, not applied twice
        with pytest.raises(RuntimeError, match="already applied this step's update"):
            opt.step()
    assert all(torch.equal(after[k], p[k].detach()) for k in p)
    assert all(opt.state[t]["step"] == 1 for t in p.values())
    # Without the stray gradients step() closes the step and changes nothing.
    opt.zero_grad(set_to_none=True)
    opt.step()
    assert all(torch.equal(after[k], p[k].detach()) for k in p)
    assert all(opt.state[t]["step"] == 1 for t in p.values())

    for it in range(2):
        rgb, _, _ = render(p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"], K,
                           vm, W, H, sh_degree=3, sh_rest=p["sh_rest"], activations=True,
                           optimizer=opt)
        if it == 0:
            rgb.square().mean().backward()
        else:
            with pytest.raises(RuntimeError, match="already applied this step's update"):
                rgb.square().mean().backward()
