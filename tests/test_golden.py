"""The committed golden fixtures (tests/golden/*.npz) against the CPU oracle.

The fixtures were written by tests/golden/make_golden.py from the oracle; these
tests regenerate each case and require the same arrays. Any change to the
oracle's arithmetic, to the seeded scenes or to the binning order therefore
fails here before it reaches the GPU comparisons. They also check that each
fixture is self-consistent and not trivial (a blank image or an empty tile
list would pin nothing)."""

from __future__ import annotations

import numpy as np
import pytest

from golden import make_golden as G


@pytest.fixture(scope="module", params=sorted(G.CASES))
def case(request):
    return request.param, G.load(request.param), G.CASES[request.param]()


def test_fixture_regenerates_from_the_oracle(case):
    name, stored, fresh = case
    assert sorted(stored) == sorted(fresh), name
    for k, want in stored.items():
        got = np.asarray(fresh[k])
        assert got.shape == want.shape and got.dtype == want.dtype, (name, k)
        if np.issubdtype(want.dtype, np.integer) or want.dtype == np.bool_:
            assert np.array_equal(got, want), (name, k)
        else:
            np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7, err_msg=f"{name}.{k}")


def test_config1_fixture_is_consistent():
    z = G.load("config1")
    N = z["means"].shape[0]
    ids, off = z["gauss_ids"], z["tile_offsets"]
    assert off.shape == (16 * 16 + 1,)
    assert off[0] == 0 and off[-1] == ids.size and np.all(np.diff(off) >= 0)
    assert ids.size > N                       # about two tiles per visible Gaussian
    assert np.all(z["valid"][ids] == 1) and ids.min() >= 0 and ids.max() < N
    # Inside every tile the list is sorted by depth, ties by Gaussian id.
    for t in range(off.size - 1):
        seg = ids[off[t]:off[t + 1]]
        d = z["depth"][seg].view(np.uint32).astype(np.int64)
        key = d * (N + 1) + seg
        assert np.all(np.diff(key) > 0), t
    assert 0.05 < float(z["alpha"].mean()) < 0.99
    assert z["rgb"].shape == (256, 256, 3) and float(z["rgb"].max()) > 0.1
    assert np.all(z["color"][z["valid"] == 0] == 0)


def test_fwd_bwd_fixture_is_not_trivial():
    z = G.load("fwd_bwd_small")
    assert 0.05 < float(z["alpha"].mean()) < 0.99
    for k in ("d_means", "d_quats", "d_scales", "d_opacities", "d_sh"):
        assert np.isfinite(z[k]).all() and np.abs(z[k]).max() > 0, k


def test_adam_fixture_moves_the_parameters():
    z = G.load("adam_small")
    for tag in ("e15", "e8"):
        step = np.abs(z[f"p_{tag}"] - z["p0"])
        # 20 steps of at most lr each (Adam's step is bounded by lr per step).
        assert 0 < step.max() <= 20 * 1e-3 * (1 + 1e-5)
    assert np.array_equal(z["sel_steps"], z["sel_masks"].sum(axis=0).astype(np.float32))
