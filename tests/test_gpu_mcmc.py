"""MCMC densification kernels (relocate, grow, add_noise, Adam-state reset)
against oracle/mcmc_ref.py, plus the reference's own MCMC tests
(tests/test_trainer.py:44-79, 213-335) on the GPU path.

The kernels draw from Philox4x64-10 keyed by a seed; the oracle is given the
same seed, so it makes the same draws: copies must then be bit-identical
(a copy is a copy), the split opacity and scale corrections within float32
rounding (1e-5), untouched rows and optimizer state bit-identical, and the
touched rows' optimizer state exactly zero."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mcmc_ref as M

pytestmark = pytest.mark.gpu


def make_params(n, dead_frac=0.3, seed=0, sh_split=True):
    g = torch.Generator().manual_seed(seed)
    logit = torch.randn(n, generator=g) * 1.5 + 1.0
    dead = torch.randperm(n, generator=g)[: int(n * dead_frac)]
    logit[dead] = -8.0 + torch.rand(dead.numel(), generator=g)
    p = {"means": torch.randn(n, 3, generator=g),
         "log_scales": torch.randn(n, 3, generator=g) * 0.3 - 4.0,
         "quats": torch.randn(n, 4, generator=g),
         "logit_opac": logit}
    if sh_split:
        p["sh_dc"] = torch.randn(n, 1, 3, generator=g)
        p["sh_rest"] = torch.randn(n, 15, 3, generator=g) * 0.1
    else:
        p["sh"] = torch.randn(n, 16, 3, generator=g)
    return p


def to_dev(p, dev, grad=False):
    return {k: v.clone().to(dev).requires_grad_(grad) for k, v in p.items()}


def to_np(p):
    return {k: v.detach().double().cpu().numpy().copy() for k, v in p.items()}


def check_against(gp, rp, before, touched, atol=1e-5):
    """Copies exact, corrected columns within atol, untouched rows unchanged.

    The split opacity is compared as an opacity: its logit log(o / (1 - o))
    amplifies float32 rounding of o by 1 / (1 - o) for opaque sources, in the
    reference's float32 arithmetic as here."""
    n = gp["logit_opac"].shape[0]
    untouched = np.ones(n, dtype=bool)
    untouched[touched] = False
    for k, t in gp.items():
        got = t.detach().double().cpu().numpy()
        if k == "logit_opac":
            err = np.abs(M.sigmoid(got) - M.sigmoid(rp[k])).max()
            assert err < 2e-6, (k, err)
        elif k == "log_scales":
            assert np.abs(got - rp[k]).max() < atol, (k, np.abs(got - rp[k]).max())
        else:
            assert np.array_equal(got, rp[k]), k
        assert np.array_equal(got[untouched], before[k][untouched]), f"{k}: untouched rows moved"


@pytest.mark.parametrize("n,dead_frac", [(20000, 0.3), (5000, 0.9), (3000, 0.01)])
def test_relocate_matches_oracle(dev, n, dead_frac):
    from metal_gauss_amd import mcmc

    p = make_params(n, dead_frac, seed=n)
    gp = to_dev(p, dev)
    rp, before = to_np(p), to_np(p)
    moved = mcmc.relocate(gp, seed=1234)
    want, touched = M.relocate(rp, u=M.uniforms(n, 1234))
    assert moved == want
    check_against(gp, rp, before, touched)


def test_relocate_with_weights_active_and_fallback(dev):
    from metal_gauss_amd import mcmc

    n, act = 8000, 6000
    p = make_params(n, 0.2, seed=5)
    g = torch.Generator().manual_seed(9)
    weights = torch.rand(n, generator=g) ** 4                 # gradient-aware style weights
    for w in (weights, torch.full((n,), float("nan")), torch.zeros(n)):
        gp = to_dev(p, dev)
        rp, before = to_np(p), to_np(p)
        moved = mcmc.relocate(gp, active=act, weights=w.to(dev), seed=77)
        want, touched = M.relocate(rp, active=act, weights=w.double().numpy(),
                                   u=M.uniforms(act, 77))
        assert moved == want
        check_against(gp, rp, before, touched)
        # Rows past `active` are never touched.
        for k in gp:
            assert torch.equal(gp[k][act:].cpu(), p[k][act:])


@pytest.mark.parametrize("opt_kind", ["fused", "selective"])
def test_relocate_zeroes_touched_optimizer_rows(dev, opt_kind):
    """tests/test_trainer.py:272-292, and the per-row step counts of
    SelectiveAdam (selective_adam.py state 'steps', mcmc.py:115-120)."""
    from metal_gauss_amd import FusedAdam, SelectiveAdam, mcmc

    n = 4000
    p = make_params(n, 0.25, seed=3)
    gp = to_dev(p, dev, grad=True)
    if opt_kind == "fused":
        opt = FusedAdam([{"params": [t], "lr": 1e-3} for t in gp.values()], eps=1e-15)
        for t in gp.values():
            t.grad = torch.randn_like(t)
        opt.step()
    else:
        opt = SelectiveAdam([{"params": [t], "lr": 1e-3} for t in gp.values()], eps=1e-15)
        for t in gp.values():
            t.grad = torch.randn_like(t)
        opt.step(torch.ones(n, dtype=torch.bool, device=dev))
    states = {k: {s: v.clone() for s, v in opt.state[t].items() if torch.is_tensor(v) and
                  v.dim() > 0} for k, t in gp.items()}
    rp = to_np({k: t.detach() for k, t in gp.items()})
    mcmc.relocate(gp, opt=opt, seed=5)
    _, touched = M.relocate(rp, u=M.uniforms(n, 5))
    mask = np.zeros(n, dtype=bool)
    mask[touched] = True
    mask_t = torch.from_numpy(mask).to(dev)
    for k, t in gp.items():
        for s, old in states[k].items():
            new = opt.state[t][s]
            assert float(new[mask_t].abs().max()) == 0.0, (k, s)
            assert torch.equal(new[~mask_t], old[~mask_t]), (k, s)
    if opt_kind == "selective":
        assert "steps" in opt.state[gp["means"]]


def test_grow_matches_oracle(dev):
    from metal_gauss_amd import FusedAdam, mcmc

    n = 10000
    p = make_params(n, 0.0, seed=11)
    gp = to_dev(p, dev, grad=True)
    opt = FusedAdam([{"params": [t], "lr": 1e-3} for t in gp.values()], eps=1e-15)
    for t in gp.values():
        t.grad = torch.randn_like(t)
    opt.step()
    rp, before = to_np(p), to_np(p)
    for k, t in gp.items():
        rp[k] = before[k] = t.detach().double().cpu().numpy().copy()
    new = mcmc.grow(gp, target=7500, active=4000, opt=opt, seed=99)
    want, touched = M.grow(rp, target=7500, active=4000, u=M.uniforms(3500, 99))
    assert new == want == 7500
    check_against(gp, rp, before, touched)
    touched_t = torch.from_numpy(np.unique(touched)).to(dev)
    for t in gp.values():
        assert float(opt.state[t]["exp_avg"][touched_t].abs().max()) == 0.0
    # Capped at the preallocated size; no-op when already there.
    assert mcmc.grow(gp, target=10 ** 6, active=7500, seed=1) == n
    assert mcmc.grow(gp, target=100, active=n) == n


def test_add_noise_matches_oracle(dev):
    from metal_gauss_amd import mcmc

    n = 50000
    p = make_params(n, 0.5, seed=21)
    g = torch.Generator().manual_seed(1)
    z = torch.randn(n, 3, generator=g)
    gp = to_dev(p, dev)
    rp = to_np(p)
    mcmc.add_noise(gp, lr_means=2e-4, eps=z.to(dev))
    M.add_noise(rp, 2e-4, z=z.double().numpy())
    got = gp["means"].double().cpu().numpy()
    delta_want = rp["means"] - p["means"].double().numpy()
    delta_got = got - p["means"].double().numpy()
    # float32 means: compare the displacement, to float32 rounding of the mean.
    err = np.abs(delta_got - delta_want).max()
    assert err < 2e-6 + 1e-5 * np.abs(delta_want).max(), err
    # The kernel's own normals: the oracle's Philox + Box-Muller with the seed.
    gp = to_dev(p, dev)
    rp = to_np(p)
    mcmc.add_noise(gp, lr_means=2e-4, seed=31337, active=40000)
    M.add_noise(rp, 2e-4, active=40000, z=M.normals(40000, 31337))
    d_got = gp["means"].double().cpu().numpy() - p["means"].double().numpy()
    d_want = rp["means"] - p["means"].double().numpy()
    assert np.abs(d_got - d_want).max() < 2e-6 + 1e-4 * np.abs(d_want).max()
    assert np.array_equal(d_got[40000:], np.zeros((n - 40000, 3)))


def test_add_noise_is_seeded_by_torch(dev):
    from metal_gauss_amd import mcmc

    p = make_params(2000, 1.0, seed=2)
    outs = []
    for _ in range(2):
        gp = to_dev(p, dev)
        torch.manual_seed(123)
        mcmc.add_noise(gp, lr_means=2e-4)
        outs.append(gp["means"].cpu())
    assert torch.equal(outs[0], outs[1])
    gp = to_dev(p, dev)
    torch.manual_seed(124)
    mcmc.add_noise(gp, lr_means=2e-4)
    assert not torch.equal(gp["means"].cpu(), outs[0])


def test_reference_mcmc_invariants(dev):
    """tests/test_trainer.py:44-79 and 226-335 on the GPU path."""
    from metal_gauss_amd import mcmc

    # Budget kept, dead revived.
    p = make_params(500, 0.3, seed=0)
    dead = (torch.sigmoid(p["logit_opac"]) < 0.005)
    gp = to_dev(p, dev)
    assert mcmc.relocate(gp) == int(dead.sum())
    assert bool((torch.sigmoid(gp["logit_opac"][dead.to(dev)]) > 0.005).all())
    # No-op when all alive.
    p0 = make_params(300, 0.0, seed=1)
    p0["logit_opac"] = p0["logit_opac"].abs() + 1.0
    gp = to_dev(p0, dev)
    assert mcmc.relocate(gp) == 0
    for k in p0:
        assert torch.equal(gp[k].cpu(), p0[k])
    # Duplicate picks: 32 dead onto one live -> a 32-way split.
    n = 33
    q = {"means": torch.zeros(n, 3), "quats": torch.zeros(n, 4),
         "log_scales": torch.full((n, 3), -3.0), "sh": torch.zeros(n, 16, 3),
         "logit_opac": torch.full((n,), -8.0)}
    q["logit_opac"][0] = 4.0
    gq = to_dev(q, dev)
    mcmc.relocate(gq)
    o = torch.sigmoid(gq["logit_opac"]).double().cpu()
    o_src = torch.sigmoid(torch.tensor(4.0)).double()
    assert bool((o > 0.005).all()) and float(o.max()) < 0.5 * float(o_src)
    assert torch.allclose((1 - o) ** 32, (1 - o_src).expand(n), rtol=1e-5)
    # Stack never more opaque than its source.
    r = {"means": torch.randn(200, 3), "quats": torch.randn(200, 4),
         "log_scales": torch.full((200, 3), -3.0), "sh": torch.randn(200, 16, 3),
         "logit_opac": torch.full((200,), 2.0)}
    r["logit_opac"][:120] = -8.0
    gr = to_dev(r, dev)
    mcmc.relocate(gr)
    o = torch.sigmoid(gr["logit_opac"])
    assert bool((o > 0.005).all()) and float(o.max()) <= float(torch.sigmoid(torch.tensor(2.0))) + 1e-5
    # Noise moves transparent Gaussians and anneals with the learning rate.
    p = make_params(500, 0.3, seed=0)
    transparent = (torch.sigmoid(p["logit_opac"]) < 0.005).to(dev)
    gp = to_dev(p, dev)
    before = gp["means"].clone()
    mcmc.add_noise(gp, lr_means=2e-4)
    d = (gp["means"] - before).norm(dim=1)
    assert float(d[transparent].mean()) > 50 * max(float(d[~transparent].mean()), 1e-12)
    hot, cold = to_dev(p, dev), to_dev(p, dev)
    mcmc.add_noise(hot, lr_means=2e-4, seed=3)
    mcmc.add_noise(cold, lr_means=2e-6, seed=3)
    m0 = p["means"].to(dev)
    assert float((hot["means"] - m0).norm()) > 50 * float((cold["means"] - m0).norm())


def test_draws_follow_the_weights(dev):
    """Chi-square of which live row each of 200k dead rows copied."""
    from scipy.stats import chisquare

    from metal_gauss_amd import mcmc

    live = 10
    n = 200_000 + live
    w = torch.tensor([0.5, 2.0, 0.0, 1.0, 3.0, 0.25, 1.5, 0.75, 4.0, 1.0])
    p = {"means": torch.zeros(n, 3), "quats": torch.zeros(n, 4),
         "log_scales": torch.full((n, 3), -3.0), "logit_opac": torch.full((n,), -9.0)}
    p["logit_opac"][:live] = 3.0
    p["means"][:live, 0] = torch.arange(live, dtype=torch.float32)
    weights = torch.zeros(n)
    weights[:live] = w
    gp = to_dev(p, dev)
    assert mcmc.relocate(gp, weights=weights.to(dev), seed=8) == n - live
    src = gp["means"][live:, 0].round().long().cpu()
    freq = torch.bincount(src, minlength=live).numpy()
    assert freq[2] == 0
    wd = w.double().numpy()
    keep = wd > 0
    pv = chisquare(freq[keep], wd[keep] / wd.sum() * (n - live)).pvalue
    assert pv > 1e-3, pv


def test_cpu_tensors_are_refused():
    from metal_gauss_amd import mcmc

    p = make_params(10, 0.5)
    with pytest.raises(RuntimeError, match="ROCm"):
        mcmc.relocate(p)
