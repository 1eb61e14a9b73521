"""Selective Adam: row-masked updates with a per-row step count, one launch.

Same optimizer contract as metal_gauss/selective_adam.py:22-206:

* groups are ``rowwise`` by default: ``step(visible)`` updates only rows r
  with ``visible[r]``; each such row's float step count ``steps[r]`` goes up by
  one and its bias correction uses that count,
  ``p -= lr * sqrt(1-b2^k)/(1-b1^k) * m / (sqrt(v) + eps)`` (eps inside the
  root, unlike FusedAdam; selective_adam.py:144-148);
* rows past the end of the mask are padding and stay untouched (52-64);
* groups with ``rowwise=False`` (per-image appearance parameters) get ordinary
  Adam with a scalar step and the same eps placement (189-206);
* state names are torch's (``exp_avg``, ``exp_avg_sq``) plus ``steps`` for
  rowwise tensors, so the reference's reset_adam_state keeps working.

The reference picks between an index-gather path and a masked-dense path with
a host sync on the visible count (selective_adam.py:108-112) and runs ~15
torch launches per tensor. Here one kernel covers every rowwise tensor: a
workgroup owns 256 rows, reads the mask once per row, and invisible rows
issue no parameter loads at all. No host sync.
"""

from __future__ import annotations

import torch

from . import _lib
from .fused_adam import _skip_ptr

_MAX_PER_LAUNCH = 32


class SelectiveAdam(torch.optim.Optimizer):
    """Row-masked Adam: each Gaussian row steps only when visible, with its own
    step count; groups marked ``rowwise=False`` take ordinary dense Adam."""

    def __init__(self, groups: list[dict], eps: float = 1e-15,
                 betas: tuple[float, float] = (0.9, 0.999)):
        defaults = {"lr": 1e-3, "eps": eps, "betas": betas, "rowwise": True}
        super().__init__(groups, defaults)
        self.groups = self.param_groups

    def _state_for(self, p: torch.Tensor, rowwise: bool) -> dict:
        st = self.state[p]
        if "exp_avg" not in st:
            st["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
            st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
            if rowwise:
                st["steps"] = torch.zeros(p.shape[0], device=p.device)
            else:
                st["step"] = 0
        return st

    @staticmethod
    def _check_gradient(p: torch.Tensor) -> torch.Tensor:
        grad = p.grad
        if grad.is_sparse:
            raise RuntimeError("SelectiveAdam does not support sparse gradients")
        if grad.shape != p.shape:
            raise ValueError(
                f"gradient shape {tuple(grad.shape)} does not match parameter "
                f"shape {tuple(p.shape)}")
        if p.device.type != "cuda":
            raise RuntimeError(
                f"SelectiveAdam requires ROCm (cuda) parameters, got device '{p.device}'")
        if not p.is_contiguous():
            raise RuntimeError("SelectiveAdam parameters must be contiguous")
        return grad.contiguous()

    @torch.no_grad()
    def step(self, visible: torch.Tensor, closure=None, skip=None):
        """One step: rows with ``visible`` set in the row-wise groups (one
        launch for all of them), every element of the dense groups.

        ``skip`` (the device status of capacity-bounded tile lists,
        ``render(list_capacity=)``'s ``info["lists_status"]``) makes every
        launch do nothing when the lists overflowed, the per-row step counts
        included; ``rewind()`` then takes back the dense groups' step
        counts before the step is run again."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if visible.ndim != 1 or visible.dtype is not torch.bool:
            raise TypeError("visible must be a one-dimensional boolean tensor")

        rows_by_key: dict[tuple, list] = {}
        dense_by_key: dict[tuple, list] = {}
        vis_dev = None
        skip_ptr = None if skip is None else _skip_ptr(skip)
        self._last_dense_stepped = []
        for group in self.param_groups:
            b1, b2 = group["betas"]
            key = (float(b1), float(b2), float(group["eps"]))
            for p in group["params"]:
                if p.grad is None:
                    continue
                if not group["rowwise"]:
                    g = self._check_gradient(p)
                    st = self._state_for(p, rowwise=False)
                    st["step"] += 1
                    self._last_dense_stepped.append(p)
                    dense_by_key.setdefault(key, []).append(
                        (p, g, st["exp_avg"], st["exp_avg_sq"], float(group["lr"]), st["step"]))
                    continue
                if p.dim() == 0 or p.shape[0] < visible.numel():
                    raise ValueError(
                        "rowwise SelectiveAdam parameters must have at least "
                        "one row per visibility-mask entry")
                g = self._check_gradient(p)
                st = self._state_for(p, rowwise=True)
                if vis_dev is None:
                    vis_dev = visible.to(device=p.device).contiguous()
                rows_by_key.setdefault(key, []).append(
                    (p, g, st["exp_avg"], st["exp_avg_sq"], st["steps"], float(group["lr"])))

        if not rows_by_key and not dense_by_key:
            return loss
        lib = _lib.load()
        for (b1, b2, eps), items in rows_by_key.items():
            for i in range(0, len(items), _MAX_PER_LAUNCH):
                chunk = items[i:i + _MAX_PER_LAUNCH]
                p0 = chunk[0][0]
                _lib.check(lib.mg_selective_adam_step_guarded(
                    len(chunk),
                    _lib.ptr_array([it[0].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[1].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[2].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[3].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[4].data_ptr() for it in chunk]),
                    _lib.i64_array([it[0].shape[0] for it in chunk]),
                    _lib.i32_array([it[0].numel() // max(1, it[0].shape[0]) for it in chunk]),
                    _lib.f32_array([it[5] for it in chunk]),
                    vis_dev.data_ptr() if vis_dev.numel() else None, vis_dev.numel(),
                    b1, b2, eps, skip_ptr, _lib.stream(p0)))
        for (b1, b2, eps), items in dense_by_key.items():
            for i in range(0, len(items), _MAX_PER_LAUNCH):
                chunk = items[i:i + _MAX_PER_LAUNCH]
                _lib.check(lib.mg_adam_step_multi_guarded(
                    len(chunk),
                    _lib.ptr_array([it[0].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[1].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[2].data_ptr() for it in chunk]),
                    _lib.ptr_array([it[3].data_ptr() for it in chunk]),
                    _lib.i64_array([it[0].numel() for it in chunk]),
                    _lib.f64_array([it[4] for it in chunk]),
                    _lib.i64_array([it[5] for it in chunk]),
                    b1, b2, eps, 1, skip_ptr, _lib.stream(chunk[0][0])))
        return loss

    def rewind(self):
        """Take back the dense groups' step counts of the last ``step()``,
        whose launches a ``skip`` status turned off (the per-row counts of
        the row-wise groups live on the device and were not advanced)."""
        for p in getattr(self, "_last_dense_stepped", ()):
            self.state[p]["step"] -= 1
        self._last_dense_stepped = []
