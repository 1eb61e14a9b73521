"""Pins of oracle/mcmc_ref.py (CPU): the Philox restatement against numpy's own
Philox4x64-10, the Box-Muller identities, the inverse-CDF sampler's
distribution, and the reference's MCMC invariant tests
(tests/test_trainer.py:44-79, 213-315) applied to the restatement."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import mcmc_ref as M
from oracle import render_ref as R


@pytest.mark.parametrize("key", [(0, 0), (7, 11), (2 ** 62 - 1, M.NOISE_TAG),
                                 (0x243F6A8885A308D3, 0x13198A2E03707344)])
def test_philox_matches_numpy(key):
    """numpy.random.Philox is Philox4x64-10; its k-th block of four words is
    the function at counter k + 1 (numpy advances the counter first)."""
    bg = np.random.Philox(key=list(key), counter=[0, 0, 0, 0])
    raw = bg.random_raw(4 * 64).reshape(64, 4)
    ctr = np.zeros((64, 4), dtype=np.uint64)
    ctr[:, 0] = np.arange(1, 65, dtype=np.uint64)
    assert np.array_equal(M.philox4x64(ctr, key), raw)
    # A counter that carries into the higher words.
    bg = np.random.Philox(key=list(key), counter=(2 ** 64 - 1) + (5 << 64))
    got = M.philox4x64(np.array([[0, 6, 0, 0]], dtype=np.uint64), key)
    assert np.array_equal(got[0], bg.random_raw(4))


def test_box_muller_identities_and_moments():
    n = 200_000
    b = M._rows_block(n, 12345, M.NOISE_TAG)
    z = M.normals(n, 12345)
    u1, u2 = M._u24(b[:, 0]), M._u24(b[:, 1])
    assert np.allclose(z[:, 0] ** 2 + z[:, 1] ** 2, -2.0 * np.log(u1), rtol=1e-12)
    ang = np.mod(np.arctan2(z[:, 1], z[:, 0]), 2 * np.pi)
    d = np.abs(ang - 2 * np.pi * u2)
    assert np.minimum(d, 2 * np.pi - d).max() < 1e-9
    assert np.abs(z.mean(0)).max() < 0.01
    assert np.abs(z.var(0) - 1.0).max() < 0.01
    # Fourth moment of a normal is 3.
    assert np.abs((z ** 4).mean(0) - 3.0).max() < 0.05
    u = M.uniforms(n, 99)
    assert u.min() > 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.003


def test_inverse_cdf_draws_follow_the_weights():
    """Chi-square goodness of fit of 200k draws over 10 weights (one zero)."""
    from scipy.stats import chisquare

    w = np.array([0.5, 2.0, 0.0, 1.0, 3.0, 0.25, 1.5, 0.75, 4.0, 1.0])
    u = M.uniforms(200_000, 4)
    idx = M.inverse_cdf(w, u)
    freq = np.bincount(idx, minlength=w.size)
    assert freq[2] == 0
    keep = w > 0
    p = chisquare(freq[keep], w[keep] / w.sum() * u.size).pvalue
    assert p > 1e-3, p


def _params(n=500, dead_frac=0.3, seed=0):
    """tests/test_trainer.py:29-41 in float64 numpy."""
    g = torch.Generator().manual_seed(seed)
    logit = torch.full((n,), 2.0)
    dead = torch.randperm(n, generator=g)[: int(n * dead_frac)]
    logit[dead] = -8.0
    p = {"means": torch.randn(n, 3, generator=g), "log_scales": torch.randn(n, 3, generator=g) * 0.1 - 3,
         "quats": torch.randn(n, 4, generator=g), "logit_opac": logit,
         "sh": torch.randn(n, 16, 3, generator=g)}
    return {k: v.double().numpy().copy() for k, v in p.items()}, dead.numpy()


def test_relocate_keeps_budget_and_revives_dead():
    p, dead = _params()
    moved, touched = M.relocate(p, u=M.uniforms(500, 1))
    assert moved == dead.size
    assert (M.sigmoid(p["logit_opac"][dead]) > 0.005).all()
    assert set(dead) <= set(touched)


def test_relocate_noop_when_all_alive():
    p, _ = _params(dead_frac=0.0)
    before = {k: v.copy() for k, v in p.items()}
    assert M.relocate(p, u=M.uniforms(500, 1))[0] == 0
    for k in p:
        assert np.array_equal(p[k], before[k])


def test_split_composites_back():
    """N copies at o' composite to the source: (1 - o')^N = 1 - o; and the
    scale ratio is sqrt(clamp(1/N, 0.05, 1)) (o'/(N o') = 1/N)."""
    o = np.array([0.02, 0.3, 0.7, 0.95])
    for n in (1, 2, 3, 7, 33, 51):
        lg, lr = M.split(o, float(n))
        on = M.sigmoid(lg)
        assert np.allclose((1 - on) ** n, 1 - o, rtol=1e-12)
        assert np.allclose(np.exp(lr), math.sqrt(min(max(1.0 / n, 0.05), 1.0)), rtol=1e-12)


def test_relocation_splits_duplicate_picks():
    """tests/test_trainer.py:247-269: 32 dead onto the single live one."""
    n = 33
    p = {"means": np.zeros((n, 3)), "quats": np.zeros((n, 4)), "log_scales": np.full((n, 3), -3.0),
         "sh": np.zeros((n, 16, 3)), "logit_opac": np.full(n, -8.0)}
    p["logit_opac"][0] = 4.0
    o_src = M.sigmoid(4.0)
    M.relocate(p, u=M.uniforms(n, 2))
    o = M.sigmoid(p["logit_opac"])
    assert (o > 0.005).all()
    assert o.max() < o_src * 0.5
    # 32 draws of one source: clamp(32, 1, 51) = 32-way split everywhere.
    assert np.allclose((1 - o) ** 32, 1 - o_src, rtol=1e-9)


def test_relocation_stack_is_not_more_opaque():
    """tests/test_trainer.py:226-244."""
    n = 200
    g = np.random.default_rng(0)
    p = {"means": g.standard_normal((n, 3)), "quats": g.standard_normal((n, 4)),
         "log_scales": np.full((n, 3), -3.0), "sh": g.standard_normal((n, 16, 3)),
         "logit_opac": np.full(n, 2.0)}
    p["logit_opac"][:120] = -8.0
    o_before = M.sigmoid(p["logit_opac"][120:]).copy()
    M.relocate(p, u=M.uniforms(n, 3))
    o_after = M.sigmoid(p["logit_opac"])
    assert (o_after > 0.005).all()
    assert o_after.max() <= o_before.max() + 1e-5


def test_grow_ramps_and_caps():
    """tests/test_trainer.py:295-315."""
    n = 1000
    g = np.random.default_rng(1)
    p = {"means": g.standard_normal((n, 3)), "quats": g.standard_normal((n, 4)),
         "log_scales": np.full((n, 3), -3.0), "sh": g.standard_normal((n, 16, 3)),
         "logit_opac": np.full(n, 2.0)}
    new, touched = M.grow(p, target=400, active=200, u=M.uniforms(200, 5))
    assert new == 400
    assert (M.sigmoid(p["logit_opac"][200:400]) > 0.005).all()
    assert set(range(200, 400)) <= set(touched)
    assert M.grow(p, target=5000, active=400, u=M.uniforms(600, 6))[0] == n


def test_add_noise_rotation_gate_and_annealing():
    """The rotation formula against the rotation matrix of render_ref (a
    different formula), the opacity gate, and annealing with the learning
    rate (tests/test_trainer.py:64-79, 318-335)."""
    n = 400
    g = np.random.default_rng(2)
    q = g.standard_normal((n, 4))
    ls = g.standard_normal((n, 3)) * 0.2 - 3.0
    z = g.standard_normal((n, 3))
    logit = np.where(np.arange(n) % 2 == 0, -8.0, 3.0)
    p = {"means": np.zeros((n, 3)), "log_scales": ls, "quats": q, "logit_opac": logit}
    M.add_noise(p, lr_means=2e-4, z=z)
    Rm = R.quat_to_rotmat(torch.from_numpy(q)).numpy()
    eps = z * np.exp(ls)
    gate = M.sigmoid(-100.0 * (M.sigmoid(logit) - 0.005))
    want = np.einsum("nij,nj->ni", Rm, eps) * gate[:, None] * 2e-4 * 4e4
    assert np.allclose(p["means"], want, rtol=1e-10, atol=1e-15)
    moved = np.linalg.norm(p["means"], axis=1)
    assert moved[0::2].mean() > 50 * max(moved[1::2].mean(), 1e-12)
    cold = {"means": np.zeros((n, 3)), "log_scales": ls, "quats": q, "logit_opac": logit}
    M.add_noise(cold, lr_means=2e-6, z=z)
    assert np.linalg.norm(p["means"]) > 50 * np.linalg.norm(cold["means"])
