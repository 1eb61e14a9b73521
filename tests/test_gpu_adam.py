"""FusedAdam and SelectiveAdam on the GPU against the numpy restatement
(oracle/adam_ref.py) and torch.optim.Adam. Mirrors tests/test_fused_adam.py
and the SelectiveAdam tests of tests/test_trainer.py:80-315. Bar: updates
within 1e-6 relative to the largest parameter change."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import adam_ref

pytestmark = pytest.mark.gpu

# Config-3 groups: (floats per Gaussian, lr) for means, log-scales, quats,
# opacity, SH DC, SH rest.
GROUPS = [(3, 1.6e-4), (3, 5e-3), (4, 1e-3), (1, 5e-2), (3, 2.5e-3), (45, 1.25e-4)]


def _params(n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, w, generator=g).to(dev).requires_grad_(True) for w, _ in GROUPS]


def _max_rel_step(got, want, start):
    """max |got - want| relative to the largest parameter magnitude, the
    reference's metric (tests/test_fused_adam.py:37). A last-bit difference in
    an fp32 parameter is ~1e-7 of its magnitude; measured against the step
    size (~1e-4 of it) the same bit would read as ~1e-3."""
    return np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)


@pytest.mark.parametrize("steps", [1, 30, 101])
def test_fused_adam_matches_the_restatement(dev, steps):
    from metal_gauss_amd import FusedAdam

    n = 2000
    P = _params(n, 2, dev)
    start = [p.detach().cpu().numpy().copy() for p in P]
    ref = [(s.copy(), np.zeros_like(s), np.zeros_like(s)) for s in start]
    opt = FusedAdam([{"params": [p], "lr": lr} for p, (_, lr) in zip(P, GROUPS)], eps=1e-15)
    g = torch.Generator().manual_seed(5)
    for k in range(1, steps + 1):
        grads = [torch.randn(p.shape, generator=g) * 1e-3 for p in P]
        for p, gr in zip(P, grads):
            p.grad = gr.to(dev)
        opt.step()
        for (pr, mr, vr), gr, (_, lr) in zip(ref, grads, GROUPS):
            adam_ref.adam_step(pr.reshape(-1), gr.numpy().reshape(-1), mr.reshape(-1),
                               vr.reshape(-1), lr, 0.9, 0.999, 1e-15, k)
    for p, (pr, _, _), s in zip(P, ref, start):
        assert _max_rel_step(p.detach().cpu().numpy(), pr, s) < 1e-6


def test_fused_adam_matches_torch_adam_over_many_steps(dev):
    """tests/test_fused_adam.py:21-38 (rel < 1e-5 there; tighter here)."""
    from metal_gauss_amd import FusedAdam

    shapes = [(5000, 3), (5000, 4), (5000, 1, 3), (5000, 15, 3), (5000,)]
    lrs = [1.6e-4, 1e-3, 2.5e-3, 1.25e-4, 1e-2]
    g = torch.Generator().manual_seed(7)
    init = [torch.randn(*s, generator=g) for s in shapes]
    A = [t.clone().to(dev).requires_grad_(True) for t in init]
    B = [t.clone().to(dev).requires_grad_(True) for t in init]
    oa = torch.optim.Adam([{"params": [t], "lr": l} for t, l in zip(A, lrs)], eps=1e-15)
    ob = FusedAdam([{"params": [t], "lr": l} for t, l in zip(B, lrs)], eps=1e-15)
    for _ in range(30):
        gs = [torch.randn(t.shape, generator=g).to(dev) for t in A]
        for t, gr in zip(A, gs):
            t.grad = gr.clone()
        for t, gr in zip(B, gs):
            t.grad = gr.clone()
        oa.step()
        ob.step()
    for a, b in zip(A, B):
        rel = ((a - b).abs().max() / a.abs().max()).item()
        assert rel < 1e-6, f"diverged from torch Adam: rel {rel:.2e}"


def test_first_step_closed_form_at_config3_size(dev):
    """Step 1 of Adam: m = (1-b1) g, v = (1-b2) g^2 and the bias corrections
    cancel, so dp = -lr g / (|g| + eps). Checked on all 59 floats of 1M
    Gaussians."""
    from metal_gauss_amd import FusedAdam

    n = 1_000_000
    P = _params(n, 2, dev)
    start = [p.detach().clone() for p in P]
    opt = FusedAdam([{"params": [p], "lr": lr} for p, (_, lr) in zip(P, GROUPS)], eps=1e-15)
    gen = torch.Generator(device=dev).manual_seed(3)
    for p in P:
        p.grad = torch.randn(p.shape, device=dev, generator=gen) * 1e-3
    opt.step()
    for p, s, (_, lr) in zip(P, start, GROUPS):
        g = p.grad.double()
        want = -lr * g / (g.abs() + 1e-15)
        got = (p.detach() - s).double()
        # The stored parameter is rounded to fp32: allow one ulp of it.
        ulp = torch.finfo(torch.float32).eps * p.detach().abs().double()
        err = ((got - want).abs() - ulp).clamp_min(0).max().item() / lr
        assert err < 1e-6, f"step-1 closed form off by {err:.2e} of lr"


def test_state_layout_matches_torch(dev):
    from metal_gauss_amd import FusedAdam

    p = torch.randn(100, 3, device=dev, requires_grad=True)
    o = FusedAdam([{"params": [p], "lr": 1e-3}], eps=1e-15)
    p.grad = torch.randn_like(p)
    o.step()
    st = o.state[p]
    assert {"step", "exp_avg", "exp_avg_sq"} <= set(st)
    assert st["exp_avg"].shape == p.shape and st["step"] == 1
    # mcmc.reset_adam_state (mcmc.py:107-121) zeroes moments in place.
    idx = torch.arange(10, device=dev)
    st["exp_avg"][idx] = 0.0
    assert st["exp_avg"][idx].abs().sum() == 0


# ------------------------------------------------------------ selective Adam

def test_selective_adam_matches_the_restatement_with_bernoulli_masks(dev):
    from metal_gauss_amd import SelectiveAdam

    n = 3000
    P = _params(n, 4, dev)
    start = [p.detach().cpu().numpy().copy() for p in P]
    ref = [(s.copy(), np.zeros((n, w), np.float32), np.zeros((n, w), np.float32),
            np.zeros(n, np.float32)) for s, (w, _) in zip(start, GROUPS)]
    opt = SelectiveAdam([{"params": [p], "lr": lr} for p, (_, lr) in zip(P, GROUPS)], eps=1e-15)
    g = torch.Generator().manual_seed(9)
    for _ in range(12):
        vis = torch.rand(n, generator=g) < 0.6
        grads = [torch.randn(p.shape, generator=g) * 1e-3 for p in P]
        for p, gr in zip(P, grads):
            p.grad = gr.to(dev)
        opt.step(vis.to(dev))
        for (pr, mr, vr, sr), gr, (_, lr) in zip(ref, grads, GROUPS):
            adam_ref.selective_adam_step(pr, gr.numpy(), mr, vr, sr, vis.numpy(), lr, 0.9,
                                         0.999, 1e-15)
    for p, (pr, _, _, sr), s0 in zip(P, ref, start):
        assert _max_rel_step(p.detach().cpu().numpy(), pr, s0) < 1e-6
        assert np.array_equal(opt.state[p]["steps"].cpu().numpy(), sr)


def test_selective_adam_leaves_invisible_rows_and_padding_untouched(dev):
    from metal_gauss_amd import SelectiveAdam

    t = torch.randn(40, 3, device=dev, requires_grad=True)
    before = t.detach().clone()
    opt = SelectiveAdam([{"params": [t], "lr": 1e-2}])
    vis = torch.zeros(30, dtype=torch.bool, device=dev)   # 10 rows of padding
    vis[:10] = True
    t.grad = torch.randn_like(t)
    opt.step(vis)
    assert not torch.allclose(t[:10], before[:10])
    assert torch.equal(t[10:], before[10:])
    st = opt.state[t]["steps"].cpu()
    assert torch.equal(st, torch.cat([torch.ones(10), torch.zeros(30)]))


def test_selective_adam_fully_visible_equals_adam(dev):
    """tests/test_trainer.py:80-98: atol 1e-6 against torch Adam."""
    from metal_gauss_amd import SelectiveAdam

    g = torch.Generator().manual_seed(0)
    a0 = torch.randn(50, 3, generator=g)
    a = a0.clone().to(dev).requires_grad_(True)
    b = a0.clone().to(dev).requires_grad_(True)
    dense = torch.optim.Adam([b], lr=1e-2, eps=1e-15)
    sel = SelectiveAdam([{"params": [a], "lr": 1e-2}], eps=1e-15)
    vis = torch.ones(50, dtype=torch.bool, device=dev)
    for _ in range(5):
        for t in (a, b):
            t.grad = None
        a.square().sum().backward()
        b.square().sum().backward()
        sel.step(vis)
        dense.step()
    assert torch.allclose(a, b, atol=1e-6)


def test_selective_adam_dense_auxiliary_group(dev):
    """Appearance-style groups use plain Adam with a scalar step
    (tests/test_trainer.py:118-145)."""
    from metal_gauss_amd import SelectiveAdam

    g = torch.Generator().manual_seed(2)
    gauss = torch.randn(12, 3, generator=g).to(dev).requires_grad_(True)
    app0 = torch.randn(4, 3, generator=g)
    app = app0.clone().to(dev).requires_grad_(True)
    ref = app0.clone().to(dev).requires_grad_(True)
    opt = SelectiveAdam([{"params": [gauss], "lr": 1e-2}])
    opt.add_param_group({"params": [app], "lr": 3e-3, "rowwise": False})
    dense = torch.optim.Adam([ref], lr=3e-3, eps=1e-15)
    vis = torch.zeros(12, dtype=torch.bool, device=dev)
    vis[:3] = True
    for _ in range(3):
        gauss.grad = torch.randn(gauss.shape, generator=g).to(dev)
        app.grad = torch.randn(app.shape, generator=g).to(dev)
        ref.grad = app.grad.clone()
        opt.step(vis)
        dense.step()
    assert torch.allclose(app, ref, atol=1e-6)
    assert "step" in opt.state[app] and "steps" not in opt.state[app]


# Widths on each of the kernel's paths: narrow tensors moved whole (1-15
# floats per row), wide tensors skipped per 64-byte chunk (16-255), and the
# element-by-element path (256 and up, or any tensor not 16-byte aligned).
@pytest.mark.parametrize("width", [1, 2, 3, 4, 5, 8, 15, 16, 17, 31, 32, 45, 64, 255, 300])
@pytest.mark.parametrize("aligned", [True, False])
def test_selective_adam_every_path_through_the_c_abi(dev, width, aligned):
    """mg_selective_adam_step on ragged row counts (one, a partial block, a
    block boundary and past it) and masks shorter than the tensor, dense to
    empty: visible rows within 1e-6 of the restatement with exact step
    counts, every other row (parameters, moments and step count) bit-for-bit
    as it was."""
    from metal_gauss_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(width * 2 + aligned)
    for rows, n_vis, dens in ((1, 1, 1.0), (63, 50, 0.6), (64, 64, 0.05), (1025, 1000, 0.6),
                              (2111, 2111, 1.0), (700, 700, 0.0)):
        host = {k: rng.standard_normal((rows, width)).astype(np.float32) for k in "pg"}
        host["g"] *= np.float32(1e-3)
        host["m"] = (rng.random((rows, width)) * 1e-3).astype(np.float32)
        host["v"] = (rng.random((rows, width)) * 1e-6).astype(np.float32)
        steps0 = rng.integers(0, 5, rows).astype(np.float32)
        vis = rng.random(n_vis) < dens
        off = 0 if aligned else 1
        dev_t = {}
        for k, a in host.items():
            buf = torch.zeros(a.size + off, device=dev)
            buf[off:] = torch.from_numpy(a.ravel()).to(dev)
            dev_t[k] = buf
        st_buf = torch.zeros(rows + off, device=dev)
        st_buf[off:] = torch.from_numpy(steps0).to(dev)
        vis_d = torch.from_numpy(vis).to(dev)

        def ptr(t):
            return t.data_ptr() + 4 * off

        _lib.check(lib.mg_selective_adam_step(
            1, _lib.ptr_array([ptr(dev_t["p"])]), _lib.ptr_array([ptr(dev_t["g"])]),
            _lib.ptr_array([ptr(dev_t["m"])]), _lib.ptr_array([ptr(dev_t["v"])]),
            _lib.ptr_array([ptr(st_buf)]), _lib.i64_array([rows]), _lib.i32_array([width]),
            _lib.f32_array([1e-2]), vis_d.data_ptr(), n_vis, 0.9, 0.999, 1e-15,
            _lib.stream(vis_d)))
        torch.cuda.synchronize()
        got = {k: t[off:].cpu().numpy().reshape(rows, width) for k, t in dev_t.items()}
        got_steps = st_buf[off:].cpu().numpy()
        want = {k: a.copy() for k, a in host.items()}
        want_steps = steps0.copy()
        adam_ref.selective_adam_step(want["p"], want["g"], want["m"], want["v"], want_steps,
                                     vis, 1e-2, 0.9, 0.999, 1e-15)
        case = f"rows={rows} n_vis={n_vis} dens={dens}"
        assert np.array_equal(got_steps, want_steps), case
        assert np.array_equal(got["g"], host["g"]), case
        seen = np.zeros(rows, bool)
        seen[:n_vis] = vis
        for k in "pmv":
            assert np.array_equal(got[k][~seen], host[k][~seen]), (case, k)
        if seen.any():
            assert _max_rel_step(got["p"], want["p"], host["p"]) < 1e-6, case
            for k in "mv":
                # A one-ulp difference of a multiply-add at the moment's
                # magnitude is the only slack.
                np.testing.assert_allclose(got[k][seen], want[k][seen], rtol=1e-6,
                                           atol=1e-6 * np.abs(want[k]).max(), err_msg=case)
