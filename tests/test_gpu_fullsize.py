"""Parity at BASELINE.json's full configuration sizes, through the product's
own entry points, against the CPU oracle.

* Config 4 (1M Gaussians, SH 3, 800x800, two of its seeded views): the
  projection with the trainer's activations, the tile lists (bit-exact
  against oracle/binning_ref.py), the raster forward (1e-4 max-abs) and
  backward (1e-3 relative L2) against oracle/raster_seq.c on the real lists
  with the photometric-loss gradient, the projection forward and backward
  against float64 autograd of oracle/render_ref.py on a seeded 20k-row
  subsample, and the optimizer epilogue against backward then step() on all
  1M rows, bit for bit, with the trainer's regularisers.
* Config 5 (3M, 1920x1080, 8160 tiles: the radix route past 4096 tiles) and
  its crowded variant (tile lists over 10k entries, over 30M intersections):
  the same binning, raster and projection checks.
* At each of these, the capacity-sized lists (no host read; capacity equal
  to the total and 25% above it) equal the host-read lists bit for bit.
* Config 3 (1M x 59 floats): SelectiveAdam with Bernoulli(0.6) masks and
  FusedAdam, 1 and 101 steps, against oracle/adam_ref.py on a seeded
  subsample of rows (every row's update is independent of the others), the
  per-row step counts exactly on every row.

The intersection counts and the longest tile list reached are printed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import rel_l2
from oracle import adam_ref, binning_ref, raster_ref, render_ref
from test_gpu_lists_capped import _host_block_work
from test_gpu_raster import gpu_backward, gpu_forward

pytestmark = pytest.mark.gpu

SUB = 20_000


def _leaves(sc, dev):
    return {k: t.to(dev).clone().requires_grad_(True) for k, t in
            (("means", sc.means), ("quats", sc.quats), ("log_scales", sc.log_scales),
             ("logits", sc.logit_opac), ("sh_dc", sc.sh_dc), ("sh_rest", sc.sh_rest))}


def _project(p, cam, opt=None, reg=None):
    """The product's projection (render's activations path)."""
    from metal_gauss_amd import backend

    fx, fy, cx, cy, vm_h, cc = backend._camera(cam.K, cam.viewmat)
    n = p["means"].shape[0]
    valid_b = torch.empty(n, dtype=torch.bool, device=p["means"].device)
    outs = backend._PreprocessMip.apply(
        p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"], p["sh_rest"], None,
        False, vm_h, fx, fy, cx, cy, cam.W, cam.H, 0.01, 100.0, 0.3, float(max(cam.W, cam.H)),
        cc, 3, valid_b, 3, opt, reg)
    return outs, valid_b


def _np(t):
    return t.detach().cpu().numpy()


def _binning_bit_exact(uv, rxy, conic, op, valid, depth, W, H, label):
    from metal_gauss_amd import backend

    gids, offs, tx = backend._bin(uv.detach(), rxy, depth, valid, conic.detach(), op.detach(),
                                  W, H, 16)
    cpu = [_np(t) for t in (uv, rxy, conic, op, valid, depth)]
    rids, roffs, _, rkeys = binning_ref.build_tile_lists(*cpu, W, H, 16)
    g, o = _np(gids), _np(offs)
    longest = int(np.diff(o).max()) if o.size > 1 else 0
    print(f"{label}: {int(_np(valid).sum())} visible, {rids.size} intersections, "
          f"{o.size - 1} tiles, longest list {longest}", flush=True)
    assert np.array_equal(o, roffs), "tile offsets differ"
    assert np.array_equal(g, rids), "gauss_ids (sorted order incl. ties) differ"
    tiles = np.repeat(np.arange(o.size - 1, dtype=np.uint64), np.diff(o))
    dbits = cpu[5].astype(np.float32).view(np.uint32).astype(np.uint64)[g]
    assert np.array_equal((tiles << np.uint64(32)) | dbits, rkeys), "sorted keys differ"
    # The same lists sized by a capacity instead of the host read (exact, and
    # with the 25% headroom ListCapacity keeps): past 4096 tiles the radix
    # passes and the tile ranges then take the kept count from the device.
    # The second build also orders the binning's blocks heaviest first, from
    # the projection's work estimate (recomputed here), as render does.
    total = int(rids.size)
    bw = torch.from_numpy(_host_block_work(cpu[0], cpu[1], cpu[4], W, H, 16)).to(
        device=uv.device, dtype=torch.int32)
    for cap, work in ((total, None), (total + total // 4, bw)):
        cids, coffs, _, status = backend._bin_capped(uv.detach(), rxy, depth, valid,
                                                      conic.detach(), op.detach(), W, H, 16,
                                                      cap, block_work=work)
        assert status.tolist() == [total, 0], (status.tolist(), total, cap)
        assert np.array_equal(_np(coffs), roffs), f"capacity {cap}: tile offsets differ"
        assert np.array_equal(_np(cids)[:total], rids), f"capacity {cap}: gauss_ids differ"
    return gids, offs, tx, rids.size, longest


def _raster_parity(args, W, H, grad_rgb, grad_alpha):
    """Forward within 1e-4 max-abs and backward within 1e-3 relative L2 of
    raster_seq.c on the same lists; returns the GPU forward and records."""
    fwd = gpu_forward(args, W, H, 16, 1e-4, chunked=False)
    r = raster_ref.forward(*[_np(a) for a in args[:6]], W, H, 16, 1e-4)
    ok = ~r[4]
    assert r[4].mean() < 1e-3, f"{r[4].sum()} ill-conditioned pixels"
    for a, b in zip(fwd[:3], r[:3]):
        assert np.abs(_np(a) - b)[ok].max() < 1e-4
    assert (_np(fwd[3]) == r[3])[ok].all(), "stop indices differ"
    ga = torch.zeros(H, W, device=grad_rgb.device) if grad_alpha is None else grad_alpha
    outs = gpu_backward(args, fwd, grad_rgb, ga, W, H, 16, absgrad=True)
    ref = raster_ref.backward(*[_np(a) for a in args[:6]], _np(fwd[2]), _np(fwd[3]),
                              _np(grad_rgb), _np(ga), W, H, 16)
    for name, a, b in zip(("d_uv", "d_conic", "d_opacity", "d_color", "d_absuv"), outs, ref):
        assert torch.isfinite(a).all(), name
        assert rel_l2(_np(a), b) < 1e-3, f"{name} rel L2 {rel_l2(_np(a), b):.2e}"
    return fwd, outs


def _subsample(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(n, generator=g)[:SUB].sort().values


def _reference_rows(sc, idx, cam, dtype=torch.float64):
    """Leaves of the subsample in ``dtype`` and render_ref.preprocess on them,
    with the trainer's exp / sigmoid in front (train.py:221-222)."""
    leaves = {k: t[idx].to(dtype).clone().requires_grad_(True) for k, t in
              (("means", sc.means), ("quats", sc.quats), ("log_scales", sc.log_scales),
               ("logits", sc.logit_opac), ("sh_dc", sc.sh_dc), ("sh_rest", sc.sh_rest))}
    K = cam.K.to(dtype)
    op = torch.sigmoid(leaves["logits"])
    sh = torch.cat([leaves["sh_dc"], leaves["sh_rest"]], dim=1)
    out = render_ref.preprocess(leaves["means"], leaves["quats"], torch.exp(leaves["log_scales"]),
                                op, sh, cam.viewmat.to(dtype), float(K[0, 0]), float(K[1, 1]),
                                float(K[0, 2]), float(K[1, 2]), cam.W, cam.H)
    return leaves, out, op


def _tol(a, b):
    """Largest relative error, the denominator floored at 1% of the tensor's
    largest magnitude: u = fx px / z + cx near 0 cancels two terms of ~W/2,
    so float32 holds it only to about one ulp of W/2."""
    b = b.detach()
    floor = 1e-2 * float(b.abs().max())
    return float(((a.detach().cpu().double() - b).abs() / (b.abs() + floor)).max())


def _projection_parity(sc, cam, outs, idx, rec, label):
    """Forward outputs of the subsample rows against float64 render_ref, and
    the backward's gradients with the rasteriser's gradients of those rows
    (rows visible on both sides) against float64 autograd.

    Each bar is the larger of a fixed tolerance and twice the error of the
    same restatement evaluated in float32 on the CPU: heavy-tailed scales
    (config 5) give near rank-1 covariances whose conic loses digits to the
    a c - b^2 cancellation in any float32 evaluation; the kernel must be as
    accurate as float32 arithmetic of the reference's formulas allows."""
    uv, conic, depth, rxy, valid, color, op_eff = outs
    leaves, (ruv, rconic, rdepth, rrxy, rvalid, rcolor), rop = _reference_rows(sc, idx, cam)
    l32, (fuv, fconic, fdepth, frxy, _, fcolor), fop = _reference_rows(sc, idx, cam,
                                                                        torch.float32)
    dev = uv.device
    gi = idx.to(dev)
    gv = _np(valid[gi]) != 0
    agree = gv == rvalid.numpy()
    assert agree.mean() > 0.999, f"{(~agree).sum()} validity flips of {SUB}"
    both = torch.from_numpy(agree & gv)
    for name, a, f, b, bar in (("uv", uv, fuv, ruv, 1e-5), ("conic", conic, fconic, rconic, 1e-4),
                               ("depth", depth, fdepth, rdepth, 1e-6),
                               ("rxy", rxy, frxy, rrxy, 1e-4)):
        got, f32 = _tol(a[gi][both], b[both]), _tol(f[both], b[both])
        print(f"{label} {name}: GPU {got:.2e}, CPU float32 {f32:.2e}", flush=True)
        assert got < max(bar, 2.0 * f32), f"{name}: {got:.2e} (float32 CPU {f32:.2e})"
    assert float((color[gi][both].cpu().double() - rcolor[both].detach()).abs().max()) < 1e-5
    assert float((op_eff[gi].cpu().double() - rop.detach()).abs().max()) < 1e-6

    # Backward: the rasteriser's gradient record rows of the subsample.
    m = both.double()
    g_uv = rec[0][gi].cpu().double() * m[:, None]
    g_conic = rec[1][gi].cpu().double() * m[:, None]
    g_op = rec[2][gi].cpu().double() * m
    g_col = rec[3][gi].cpu().double() * m[:, None]
    grads = (g_uv, g_conic, g_col, g_op)
    torch.autograd.backward([ruv, rconic, rcolor, rop], list(grads))
    torch.autograd.backward([fuv, fconic, fcolor, fop], [g.float() for g in grads])
    return leaves, l32, grads, both


def _gpu_projection_grads(sc, cam, idx, grads, dev):
    """The product's projection backward on the subsample rows with the same
    incoming gradients (the kernel treats every row on its own)."""
    p = {k: t[idx].to(dev).clone().requires_grad_(True) for k, t in
         (("means", sc.means), ("quats", sc.quats), ("log_scales", sc.log_scales),
          ("logits", sc.logit_opac), ("sh_dc", sc.sh_dc), ("sh_rest", sc.sh_rest))}
    (uv, conic, _, _, _, color, op_eff), _ = _project(p, cam)
    g_uv, g_conic, g_col, g_op = (t.float().to(dev) for t in grads)
    torch.autograd.backward([uv, conic, color, op_eff], [g_uv, g_conic, g_col, g_op])
    return p


def _check_projection_grads(p, leaves, l32, both, label):
    """Relative L2 of every parameter gradient against float64 autograd:
    below 1e-4, or twice the float32 restatement's own error."""
    # Rows visible on both sides (the others get no incoming gradient; the
    # float32 restatement's overflowing covariances of huge invisible splats
    # give 0 * inf = nan there).
    for k in ("means", "quats", "log_scales", "logits", "sh_dc", "sh_rest"):
        a = p[k].grad.detach().cpu().double()[both]
        b = leaves[k].grad[both]
        got, f32 = rel_l2(a, b), rel_l2(l32[k].grad[both], b)
        print(f"{label} d_{k}: GPU {got:.2e}, CPU float32 {f32:.2e}", flush=True)
        assert got < max(1e-4, 2.0 * f32), f"{k}: rel L2 {got:.2e} (float32 CPU {f32:.2e})"
    inv = ~both
    if inv.any():
        assert float(p["quats"].grad[inv.to(p["quats"].device)].abs().max()) == 0.0


def _projection_check(sc, cam, outs, idx, rec, dev, label):
    leaves, l32, grads, both = _projection_parity(sc, cam, outs, idx, rec, label)
    _check_projection_grads(_gpu_projection_grads(sc, cam, idx, grads, dev), leaves, l32, both,
                            label)


# ------------------------------------------------------------------ config 2

def test_config2_parameter_gradients_through_render(dev):
    """BASELINE configs[1] end to end through render(): 300k Gaussians, SH 3,
    800x800, white background, L1 against the 5x5 box-blurred target. The
    gradients of the activated inputs render takes (means, quats, scales,
    opacities, SH) on a seeded 20k-row subsample, against float64 autograd
    of render_ref.preprocess driven by raster_seq.c's forward and backward
    on the same lists with the same image gradient (the reference's own
    gradient check, tests/test_metal.py:95-117, at the configuration's
    size). Bar: 1e-3 relative L2 per parameter."""
    from metal_gauss_amd import render, scenes
    from metal_gauss_amd.backend import _PreprocessMetal, _camera, build_tile_lists_metal

    sc, cam, bg = scenes.config2()
    W, H = cam.W, cam.H
    act = [t.to(dev) for t in sc.activated()]     # means, quats, scales, opacities, sh (N,16,3)
    leaves = [t.clone().requires_grad_(True) for t in act]
    rgb, alpha, info = render(*leaves, cam.K, cam.viewmat, W, H, sh_degree=3, background=bg)
    target = scenes.config2_target().to(dev)
    # L1's gradient, formed once from the GPU image and given to both sides
    # (sign() at |rgb - target| < 1e-4 would otherwise differ between them).
    grad_rgb = (torch.sign(rgb.detach() - target) / rgb.numel()).contiguous()
    rgb.backward(grad_rgb)
    torch.cuda.synchronize()

    # The C contract on the same projection and lists.
    fx, fy, cx, cy, vm_h, cc = _camera(cam.K, cam.viewmat)
    with torch.no_grad():
        uv, conic, depth, rxy, valid, col = _PreprocessMetal.apply(
            act[0], act[1], act[2], act[4], None, act[3], vm_h, fx, fy, cx, cy, W, H, 0.01,
            100.0, 0.3, float(max(W, H)), cc, 3)
        gids, offs, _ = build_tile_lists_metal(uv, rxy, depth, valid, conic, act[3], W, H, 16)
    assert gids.numel() == int(info["isect_total"])
    c_in = [_np(t) for t in (uv, conic, act[3], col, gids, offs)]
    r = raster_ref.forward(*c_in, W, H, 16, 1e-4)
    ok = ~r[4]
    img = r[0] + (1.0 - r[1])[..., None]
    assert np.abs(_np(rgb) - img)[ok].max() < 1e-4
    g_rgb = _np(grad_rgb)
    g_alpha = -(g_rgb.sum(axis=-1))                         # through the white blend
    d_uv, d_conic, d_op, d_col, _ = raster_ref.backward(*c_in, r[2], r[3], g_rgb, g_alpha,
                                                         W, H, 16)

    # float64 (and float32) autograd of the projection on the subsample.
    idx = _subsample(sc.n, 200)
    gi = idx.to(dev)
    K = cam.K.double()
    ref = {}
    for dt in (torch.float64, torch.float32):
        lv = [t[idx].to(dt).clone().requires_grad_(True) for t in sc.activated()]
        ruv, rconic, _, _, rvalid, rcol = render_ref.preprocess(
            lv[0], lv[1], lv[2], lv[3], lv[4], cam.viewmat.to(dt), float(K[0, 0]),
            float(K[1, 1]), float(K[0, 2]), float(K[1, 2]), W, H)
        grads = [torch.from_numpy(a[idx.numpy()]).to(dt) for a in (d_uv, d_conic, d_col)]
        torch.autograd.backward([ruv, rconic, rcol], grads)
        lv[3].grad = torch.from_numpy(d_op[idx.numpy()]).to(dt)   # op enters only the raster
        ref[dt] = (lv, rvalid)
    (r64, rvalid), (r32, _) = ref[torch.float64], ref[torch.float32]
    gv = _np(valid[gi]) != 0
    agree = gv == rvalid.numpy()
    assert agree.mean() > 0.999, f"{(~agree).sum()} validity flips of {SUB}"
    both = torch.from_numpy(agree & gv)
    print(f"config 2: {gids.numel()} intersections, {int(gv.sum())} of {SUB} rows visible",
          flush=True)
    for name, a, b, f in zip(("means", "quats", "scales", "opacities", "sh"), leaves, r64, r32):
        got = rel_l2(a.grad[gi].cpu().double()[both], b.grad[both])
        f32 = rel_l2(f.grad[both].double(), b.grad[both])
        print(f"config 2 d_{name}: GPU {got:.2e}, CPU float32 {f32:.2e}", flush=True)
        assert got < 1e-3, f"d_{name}: relative L2 {got:.2e} (float32 CPU {f32:.2e})"
    # Rows the projection marked invalid: exact zeros.
    hidden = torch.from_numpy(~gv).to(dev)
    if bool(hidden.any()):
        for a in leaves:
            assert float(a.grad[gi][hidden].abs().max()) == 0.0


# ------------------------------------------------------------------ config 4

@pytest.mark.parametrize("view", [0, 57])
def test_config4_step_parity(dev, view):
    """1M Gaussians, SH 3, 800x800, the photometric loss
    0.8 L1 + 0.2 (1 - SSIM) of the view's smooth target."""
    from metal_gauss_amd import gaussian_kernel, photometric_loss, scenes

    sc, cams, _ = scenes.config4()
    cam = cams[view]
    W, H = cam.W, cam.H
    p = _leaves(sc, dev)
    with torch.no_grad():
        outs, valid_b = _project(p, cam)
    uv, conic, depth, rxy, valid, color, op_eff = outs
    gids, offs, tx, n_isect, _ = _binning_bit_exact(uv, rxy, conic, op_eff, valid, depth, W, H,
                                                    f"config 4 view {view}")
    assert n_isect > 3_000_000
    args = (uv, conic, op_eff, color, gids, offs, tx)
    # The loss gradient at the rendered image (black background).
    rgb0 = gpu_forward(args, W, H, 16, 1e-4, chunked=False)[0].clone().requires_grad_(True)
    gt = scenes.config4_target(view).to(dev)
    loss, _ = photometric_loss(rgb0, gt, gaussian_kernel(device=dev, groups=15), 0.2)
    loss.backward()
    grad_rgb = rgb0.grad.contiguous()
    _, rec = _raster_parity(args, W, H, grad_rgb, None)

    _projection_check(sc, cam, outs, _subsample(sc.n, 400 + view), rec, dev,
                      f"config 4 view {view}")


def test_config4_epilogue_equals_backward_then_step_at_full_size(dev):
    """The optimizer epilogue over all 1M rows with the rasteriser's
    gradients of a seeded image gradient and the trainer's regularisers
    (0.01, 0.01): parameters, exp_avg and exp_avg_sq bit-identical to the
    backward followed by FusedAdam.step(), two steps."""
    from metal_gauss_amd import FusedAdam, scenes

    sc, cams, _ = scenes.config4()
    cam = cams[3]
    W, H = cam.W, cam.H
    lrs = {"means": 1.6e-4, "quats": 1e-3, "log_scales": 5e-3, "logits": 5e-2,
           "sh_dc": 2.5e-3, "sh_rest": 1.25e-4}
    # Fixed incoming gradients: the raster backward of a seeded image gradient.
    p0 = _leaves(sc, dev)
    with torch.no_grad():
        outs, _ = _project(p0, cam)
        uv, conic, depth, rxy, valid, color, op_eff = outs
        from metal_gauss_amd import backend
        gids, offs, tx = backend._bin(uv, rxy, depth, valid, conic, op_eff, W, H, 16)
    args = (uv, conic, op_eff, color, gids, offs, tx)
    fwd = gpu_forward(args, W, H, 16, 1e-4, chunked=False)
    g = torch.Generator(device=dev).manual_seed(77)
    grad_rgb = torch.randn(H, W, 3, device=dev, generator=g) * 1e-6
    rec = [t.clone() for t in gpu_backward(args, fwd, grad_rgb, torch.zeros(H, W, device=dev),
                                           W, H, 16, absgrad=False)[:4]]
    del p0, outs, args, fwd
    runs = []
    for fused in (True, False):
        p = _leaves(sc, dev)
        opt = FusedAdam([{"params": [t], "lr": lrs[k]} for k, t in p.items()], eps=1e-15)
        for _ in range(2):
            (uv, conic, _, _, _, color, op_eff), _ = _project(p, cam, opt if fused else None,
                                                              (0.01, 0.01))
            opt.zero_grad(set_to_none=True)
            torch.autograd.backward([uv, conic, color, op_eff], [rec[0], rec[1], rec[3], rec[2]])
            assert all((t.grad is None) == fused for t in p.values())
            opt.step()
        runs.append({k: (t.detach(), opt.state[t]["exp_avg"], opt.state[t]["exp_avg_sq"])
                     for k, t in p.items()})
        del opt
    for k in runs[0]:
        for a, b, what in zip(runs[0][k], runs[1][k], ("param", "exp_avg", "exp_avg_sq")):
            assert torch.equal(a, b), f"{k} {what}"


def test_config4_render_step_with_optimizer_matches_unfused(dev):
    """The timed step of bench.py at full size: render(activations=True,
    optimizer=, opacity_reg=0.01, scale_reg=0.01) + the fused photometric
    loss + step(), against render + loss + the trainer's regularisers in
    torch + backward + step(). The rasteriser's atomics reorder sums run to
    run, so the bar is elementwise closeness for all but 1e-3 of the 59M
    updated elements."""
    from metal_gauss_amd import FusedAdam, gaussian_kernel, photometric_loss, render, scenes

    sc, cams, _ = scenes.config4()
    cam = cams[11]
    lrs = {"means": 1.6e-4, "quats": 1e-3, "log_scales": 5e-3, "logits": 5e-2,
           "sh_dc": 2.5e-3, "sh_rest": 1.25e-4}
    gt = scenes.config4_target(11).to(dev)
    window = gaussian_kernel(device=dev, groups=15)
    start = _leaves(sc, dev)
    res = []
    for fused in (True, False):
        p = {k: t.detach().clone().requires_grad_(True) for k, t in start.items()}
        opt = FusedAdam([{"params": [t], "lr": lrs[k]} for k, t in p.items()], eps=1e-15)
        kw = dict(optimizer=opt, opacity_reg=0.01, scale_reg=0.01) if fused else {}
        rgb, _, info = render(p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"],
                              cam.K, cam.viewmat, cam.W, cam.H, sh_degree=3,
                              sh_rest=p["sh_rest"], activations=True, **kw)
        loss, _ = photometric_loss(rgb, gt, window, 0.2)
        if not fused:
            loss = loss + 0.01 * torch.sigmoid(p["logits"]).mean() \
                + 0.01 * torch.exp(p["log_scales"]).mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        res.append({k: (t.detach() - start[k].detach()).cpu() for k, t in p.items()})
        del opt, p
    for k in res[0]:
        a, b = res[0][k], res[1][k]
        close = torch.isclose(a, b, rtol=1e-3, atol=1e-4 * lrs[k])
        assert float(close.double().mean()) > 0.999, k
        assert rel_l2(a, b) < 5e-2, k


# ------------------------------------------------------------------ config 5

@pytest.mark.parametrize("crowded", [False, True])
def test_config5_parity(dev, crowded):
    """BASELINE configs[4] (3M Gaussians, 1920x1080 from inside the cloud,
    8160 tiles) and the crowded variant that reaches the configuration's
    stated stress: tile lists of more than 10k entries and more than 30M
    intersections. Binning bit-exact, raster forward and backward against
    the C contract with a seeded image gradient (colour and coverage), the
    projection on a 20k-row subsample."""
    from metal_gauss_amd import scenes

    sc, cam, _ = scenes.config5_crowded() if crowded else scenes.config5()
    W, H = cam.W, cam.H
    p = _leaves(sc, dev)
    with torch.no_grad():
        outs, _ = _project(p, cam)
    uv, conic, depth, rxy, valid, color, op_eff = outs
    label = "config 5 crowded" if crowded else "config 5"
    gids, offs, tx, n_isect, longest = _binning_bit_exact(uv, rxy, conic, op_eff, valid, depth,
                                                          W, H, label)
    assert offs.numel() - 1 == 8160
    if crowded:
        assert n_isect > 30_000_000 and longest > 10_000
    args = (uv, conic, op_eff, color, gids, offs, tx)
    g = torch.Generator(device=dev).manual_seed(5)
    grad_rgb = torch.randn(H, W, 3, device=dev, generator=g) / (H * W)
    grad_alpha = torch.randn(H, W, device=dev, generator=g) / (H * W)
    _, rec = _raster_parity(args, W, H, grad_rgb, grad_alpha)
    _projection_check(sc, cam, outs, _subsample(sc.n, 500 + int(crowded)), rec, dev, label)


# ------------------------------------------------------------------ config 3

# Config-3 groups: (name, floats per Gaussian, lr).
GROUPS = [("means", 3, 1.6e-4), ("log_scales", 3, 5e-3), ("quats", 4, 1e-3),
          ("opacity", 1, 5e-2), ("sh_dc", 3, 2.5e-3), ("sh_rest", 45, 1.25e-4)]


def _config3_params(dev):
    g = torch.Generator().manual_seed(2)
    return [torch.randn(1_000_000, w, generator=g).to(dev).requires_grad_(True)
            for _, w, _ in GROUPS]


@pytest.mark.parametrize("selective", [True, False])
def test_config3_adam_at_full_size(dev, selective):
    """1M Gaussians x 59 floats in six groups, gradients
    N(0, 1e-3) drawn fresh each step, beta (0.9, 0.999), eps 1e-15; the
    selective variant with a fresh Bernoulli(0.6) visibility mask per step.
    After step 1 and step 101 the parameters of a seeded 20k-row subsample
    are within 1e-6 (relative to the largest parameter) of the numpy
    restatement run on those rows; SelectiveAdam's per-row step counts match
    exactly on all 1M rows, and rows not visible at step 1 are untouched by
    it."""
    from metal_gauss_amd import FusedAdam, SelectiveAdam

    n = 1_000_000
    P = _config3_params(dev)
    idx = _subsample(n, 3)
    gi = idx.to(dev)
    ref = [[_np(t[gi]).copy(), np.zeros((SUB, w), np.float32), np.zeros((SUB, w), np.float32),
            np.zeros(SUB, np.float32)] for t, (_, w, _) in zip(P, GROUPS)]
    start = [t.detach().clone() for t in P]
    groups = [{"params": [t], "lr": lr} for t, (_, _, lr) in zip(P, GROUPS)]
    opt = SelectiveAdam(groups, eps=1e-15) if selective else FusedAdam(groups, eps=1e-15)
    gen = torch.Generator(device=dev).manual_seed(303)
    counts = torch.zeros(n, dtype=torch.float32, device=dev)
    for k in range(1, 102):
        vis = (torch.rand(n, device=dev, generator=gen) < 0.6) if selective else None
        for t in P:
            t.grad = torch.randn(t.shape, device=dev, generator=gen) * 1e-3
        if selective:
            opt.step(vis)
            counts += vis.float()
        else:
            opt.step()
        vsub = _np(vis[gi]) if selective else None
        for (pr, mr, vr, sr), t, (_, _, lr) in zip(ref, P, GROUPS):
            gsub = _np(t.grad[gi])
            if selective:
                adam_ref.selective_adam_step(pr, gsub, mr, vr, sr, vsub, lr, 0.9, 0.999, 1e-15)
            else:
                adam_ref.adam_step(pr.reshape(-1), gsub.reshape(-1), mr.reshape(-1),
                                   vr.reshape(-1), lr, 0.9, 0.999, 1e-15, k)
        if k == 1 and selective:
            hidden = ~vis
            for t, s in zip(P, start):
                assert torch.equal(t.detach()[hidden], s[hidden])
        if k in (1, 101):
            for (pr, _, _, _), t, (name, _, _) in zip(ref, P, GROUPS):
                got = _np(t[gi])
                err = np.abs(got - pr).max() / max(np.abs(pr).max(), 1e-30)
                assert err < 1e-6, f"step {k} {name}: {err:.2e}"
    if selective:
        for t in P:
            assert torch.equal(opt.state[t]["steps"], counts)
