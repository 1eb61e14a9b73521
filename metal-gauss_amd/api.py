"""Single render entry point with an explicit backend (metal_gauss/api.py:11-27).

The reference offers ``"torch_ref"`` (its pure-PyTorch oracle) and ``"metal"``.
This package ships one backend, ``"hip"``; ``"metal"`` is accepted as the name
callers of the reference already pass and selects the same native kernels.
There is no silent substitution: an unknown backend is a ValueError and the
native backend either runs on the GPU or raises.
"""

from __future__ import annotations

BACKENDS = ("hip", "metal")


def render(*args, backend: str = "hip", **kwargs):
    if backend in BACKENDS:
        from . import backend as hip_backend
        return hip_backend.render(*args, **kwargs)
    if backend == "torch_ref":
        raise ValueError(
            "backend 'torch_ref' (the pure-PyTorch reference renderer) is not shipped in "
            "metal_gauss_amd; it is the test oracle. Use backend='hip'.")
    raise ValueError(f"unknown backend {backend!r}; expected one of {BACKENDS}")
