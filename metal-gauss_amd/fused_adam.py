"""Adam as one HIP launch for every parameter group of a step.

Same optimizer contract as metal_gauss/fused_adam.py:26-54: a
``torch.optim.Optimizer`` whose per-parameter state is torch Adam's
(``step``, ``exp_avg``, ``exp_avg_sq``), so code that edits the moments of
relocated rows (the reference's mcmc.reset_adam_state, mcmc.py:107-121) works
unchanged. The update is torch's formula with eps added after the
sqrt(bias_correction2) divide (adam.metal:34-41).

The reference issues one kernel per parameter tensor; here all tensors that
share (betas, eps) go into a single launch (mg_adam_step_multi), up to 32 per
launch. Each element is read and written once: 28 bytes of HBM traffic.
"""

from __future__ import annotations

import torch

from . import _lib

_MAX_PER_LAUNCH = 32


class FusedAdam(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-15):
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        batches: dict[tuple, list] = {}
        for group in self.param_groups:
            b1, b2 = group["betas"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                g = p.grad
                if g.is_sparse:
                    raise RuntimeError("FusedAdam does not support sparse gradients")
                if p.device.type != "cuda":
                    raise RuntimeError(
                        f"FusedAdam requires ROCm (cuda) parameters, got device '{p.device}'")
                if not p.is_contiguous():
                    raise RuntimeError("FusedAdam parameters must be contiguous")
                st = self.state[p]
                if not st:
                    st["step"] = 0
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                st["step"] += 1
                g = g.contiguous()
                key = (float(b1), float(b2), float(group["eps"]), p.device)
                batches.setdefault(key, []).append(
                    (p, g, st["exp_avg"], st["exp_avg_sq"], float(group["lr"]), int(st["step"])))
        if batches:
            lib = _lib.load()
            for (b1, b2, eps, _dev), items in batches.items():
                for i in range(0, len(items), _MAX_PER_LAUNCH):
                    chunk = items[i:i + _MAX_PER_LAUNCH]
                    s = _lib.stream(chunk[0][0])
                    _lib.check(lib.mg_adam_step_multi(
                        len(chunk),
                        _lib.ptr_array([it[0].data_ptr() for it in chunk]),
                        _lib.ptr_array([it[1].data_ptr() for it in chunk]),
                        _lib.ptr_array([it[2].data_ptr() for it in chunk]),
                        _lib.ptr_array([it[3].data_ptr() for it in chunk]),
                        _lib.i64_array([it[0].numel() for it in chunk]),
                        _lib.f64_array([it[4] for it in chunk]),
                        _lib.i64_array([it[5] for it in chunk]),
                        b1, b2, eps, 0, s))
                    # Gradients made contiguous above must outlive the launch.
                    del chunk
        return loss
