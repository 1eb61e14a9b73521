"""Host-side behaviour that needs no GPU: backend selection, device refusal,
the build-lock message, the antialias algebra and optimizer argument checks.
Mirrors the reference's CPU tests (tests/test_metal_build.py,
tests/test_antialias.py:30-97, tests/test_torch_ref.py:198-215,
tests/test_trainer.py selective-Adam type checks)."""

from __future__ import annotations

import os

import pytest
import torch

from conftest import intrinsics, scene


# ------------------------------------------------------------ backend choice

def test_unknown_backend_is_rejected():
    from metal_gauss_amd import render

    with pytest.raises(ValueError, match="unknown backend"):
        render(None, None, None, None, None, None, None, 8, 8, backend="cuda")


def test_torch_ref_backend_is_not_shipped():
    from metal_gauss_amd import render

    with pytest.raises(ValueError, match="test oracle"):
        render(None, None, None, None, None, None, None, 8, 8, backend="torch_ref")


@pytest.mark.parametrize("backend", ["hip", "metal"])
def test_native_backend_never_silently_falls_back(backend):
    """CPU tensors are an error, never a silent copy or a torch render
    (tests/test_torch_ref.py:203-215, tests/test_metal.py:153-159)."""
    from metal_gauss_amd import render

    s = scene(n=10)
    with pytest.raises(RuntimeError, match="requires ROCm"):
        render(s["means"], s["quats"], s["scales"], s["opacities"], None, intrinsics(16, 16),
               torch.eye(4), 16, 16, colors=s["colors"], backend=backend)


def test_tile_lists_refuse_cpu_tensors():
    from metal_gauss_amd.backend import build_tile_lists_metal

    z = torch.zeros(4, 2)
    with pytest.raises(RuntimeError, match="requires ROCm"):
        build_tile_lists_metal(z, z, torch.ones(4), torch.ones(4, dtype=torch.bool),
                               torch.zeros(4, 3), torch.ones(4), 16, 16, 16)


def test_full_sh_with_sh_rest_is_rejected_before_any_launch():
    from metal_gauss_amd.backend import _sh_inputs

    with pytest.raises(ValueError, match="DC band"):
        _sh_inputs(torch.zeros(5, 16, 3), torch.zeros(5, 15, 3))


def test_narrow_sh_is_zero_padded():
    from metal_gauss_amd.backend import _sh_inputs

    sh, rest = _sh_inputs(torch.ones(5, 4, 3), None)
    assert rest is None and sh.shape == (5, 16, 3)
    assert torch.equal(sh[:, 4:], torch.zeros(5, 12, 3))
    dc, rest = _sh_inputs(torch.ones(5, 1, 3), torch.ones(5, 3, 3))
    assert rest.shape == (5, 15, 3) and float(rest[:, 3:].abs().sum()) == 0.0


# --------------------------------------------------------------- build lock

def _lock(d, age_s, now=1_000_000.0):
    lock = d / "lock"
    lock.touch()
    os.utime(lock, (now - age_s, now - age_s))
    return lock


def test_no_lock_means_nothing_to_say(tmp_path):
    from metal_gauss_amd.backend import stale_lock_message

    assert stale_lock_message(tmp_path, now=1_000_000.0) is None
    assert stale_lock_message(tmp_path / "never-built", now=1_000_000.0) is None


def test_fresh_and_old_locks(tmp_path):
    from metal_gauss_amd.backend import stale_lock_message

    lock = _lock(tmp_path, 5.0)
    msg = stale_lock_message(tmp_path, now=1_000_000.0)
    assert str(lock) in msg and "5s" in msg and "stale" not in msg.lower()
    _lock(tmp_path, 3600.0)
    msg = stale_lock_message(tmp_path, now=1_000_000.0)
    assert "stale" in msg.lower() and "delete" in msg.lower()


# ----------------------------------------------------------- antialias math

BLUR = 0.3


def _conic_from_cov(a, b, c):
    det = a * c - b * b
    return torch.stack([c / det, -b / det, a / det], dim=-1)


def test_antialias_scale_is_the_determinant_ratio():
    from metal_gauss_amd.backend import antialias_scale

    g = torch.Generator().manual_seed(0)
    n = 512
    sx = torch.rand(n, generator=g).double() * 5.0 + 0.01
    sy = torch.rand(n, generator=g).double() * 5.0 + 0.01
    rho = (torch.rand(n, generator=g).double() - 0.5) * 1.2
    a0, c0, b0 = sx * sx, sy * sy, rho * sx * sy
    a1, c1 = a0 + BLUR, c0 + BLUR
    want = ((a0 * c0 - b0 * b0) / (a1 * c1 - b0 * b0)).clamp(0.0, 1.0).sqrt()
    got = antialias_scale(_conic_from_cov(a1, b0, c1), BLUR)
    assert torch.allclose(got, want, atol=1e-9)


def test_antialias_scale_bounds_and_limits():
    from metal_gauss_amd.backend import antialias_scale

    s = torch.rand(4096, generator=torch.Generator().manual_seed(1)).double() * 8.0 + 1e-3
    sc = antialias_scale(_conic_from_cov(s * s + BLUR, torch.zeros_like(s), s * s + BLUR), BLUR)
    assert (sc <= 1.0 + 1e-12).all() and (sc >= 0.0).all()
    wide = torch.tensor([100.0], dtype=torch.float64)
    assert antialias_scale(_conic_from_cov(wide + BLUR, torch.zeros(1).double(), wide + BLUR),
                           BLUR).item() > 0.99
    tiny = torch.tensor([0.01], dtype=torch.float64)
    assert antialias_scale(_conic_from_cov(tiny + BLUR, torch.zeros(1).double(), tiny + BLUR),
                           BLUR).item() < 0.1


def test_antialias_gradient_reaches_the_conic():
    from metal_gauss_amd.backend import antialias_scale

    s = torch.tensor([0.5, 2.0], dtype=torch.float64)
    conic = _conic_from_cov(s + BLUR, torch.zeros(2).double(), s + BLUR).requires_grad_(True)
    antialias_scale(conic, BLUR).sum().backward()
    assert torch.isfinite(conic.grad).all() and conic.grad.abs().sum() > 0


# ------------------------------------------------------- optimizer contracts

def test_selective_adam_rejects_a_non_boolean_mask():
    from metal_gauss_amd import SelectiveAdam

    t = torch.ones(4, 2, requires_grad=True)
    opt = SelectiveAdam([{"params": [t], "lr": 1e-2}])
    with pytest.raises(TypeError, match="boolean"):
        opt.step(torch.ones(4))


def test_selective_adam_rejects_a_mask_longer_than_the_rows():
    from metal_gauss_amd import SelectiveAdam

    t = torch.ones(4, 2, requires_grad=True)
    t.grad = torch.ones_like(t)
    opt = SelectiveAdam([{"params": [t], "lr": 1e-2}])
    with pytest.raises(ValueError, match="one row per visibility-mask entry"):
        opt.step(torch.ones(6, dtype=torch.bool))


def test_fused_adam_refuses_cpu_parameters():
    from metal_gauss_amd import FusedAdam

    t = torch.ones(4, requires_grad=True)
    t.grad = torch.ones_like(t)
    with pytest.raises(RuntimeError, match="ROCm"):
        FusedAdam([t]).step()


def test_fused_adam_epilogue_refusals_count_no_step():
    """FusedAdam.epilogue (the projection backward's optimizer epilogue)
    declines, without advancing any step count, for a tensor that is not one
    of its parameters, a parameter that already holds a gradient, and
    parameters off the GPU."""
    from metal_gauss_amd import FusedAdam

    a = torch.zeros(8, 3, requires_grad=True)
    b = torch.zeros(8, 4, requires_grad=True)
    opt = FusedAdam([{"params": [a], "lr": 1e-3}, {"params": [b], "lr": 1e-2}])
    assert opt.epilogue([a, torch.zeros(8, 4), None]) is None     # not a parameter
    assert opt.epilogue([a, b, None]) is None                     # CPU parameters
    b.grad = torch.zeros_like(b)
    assert opt.epilogue([b, a]) is None                           # gradient already there
    assert all(not opt.state[t] or opt.state[t]["step"] == 0 for t in (a, b))


def test_fused_adam_refused_step_keeps_the_epilogue_bookkeeping():
    """A step() refused because a parameter the epilogue already updated has
    a gradient must leave that parameter recognised: calling step() again
    refuses again instead of applying Adam to it a second time."""
    from metal_gauss_amd import FusedAdam

    p = torch.zeros(8, 3, requires_grad=True)
    opt = FusedAdam([p], lr=1e-3)
    opt._epilogue_applied = {id(p): p}       # as render(optimizer=opt)'s epilogue leaves it
    p.grad = torch.ones_like(p)
    for _ in range(2):
        with pytest.raises(RuntimeError, match="already applied"):
            opt.step()
    assert opt._epilogue_applied == {id(p): p}
