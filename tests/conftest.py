"""Shared test setup.

Markers: ``gpu`` for tests that need the MI355X (run with ``-m gpu`` on the GPU
box); everything else runs on the CPU. A gpu-marked test on a machine without a
visible GPU fails loudly instead of skipping, so a GPU run can never pass on a
silent fallback.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X); run with -m gpu")


@pytest.fixture
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible HIP GPU")
    return torch.device("cuda:0")


def intrinsics(W, H, f=None):
    import torch

    f = f or 0.8 * max(W, H)
    K = torch.eye(3)
    K[0, 0], K[1, 1], K[0, 2], K[1, 2] = f, f, W / 2, H / 2
    return K


def scene(n=400, seed=0, z=4.0, spread=0.6, scale=(0.03, 0.13), opac=(0.15, 0.85), sh=False):
    """Seeded CPU scene in the style of the reference's tests (test_metal.py:27-37)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    means = torch.randn(n, 3, generator=g) * spread + torch.tensor([0.0, 0.0, z])
    quats = torch.randn(n, 4, generator=g)
    scales = torch.rand(n, 3, generator=g) * (scale[1] - scale[0]) + scale[0]
    op = torch.rand(n, generator=g) * (opac[1] - opac[0]) + opac[0]
    cols = torch.rand(n, 3, generator=g)
    shc = torch.randn(n, 16, 3, generator=g) * 0.25
    return dict(means=means, quats=quats, scales=scales, opacities=op, colors=cols, sh=shc)


def rel_l2(a, b):
    import torch

    a, b = torch.as_tensor(a).double(), torch.as_tensor(b).double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))
