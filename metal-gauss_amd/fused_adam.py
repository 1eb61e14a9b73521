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
        # Parameters whose update a render(optimizer=) backward has applied
        # since the last step(), by id.
        self._epilogue_applied: dict[int, torch.Tensor] = {}
        # Parameters whose step count the last step() advanced (rewind()).
        self._last_stepped: list[torch.Tensor] = []

    def _state_of(self, p):
        st = self.state[p]
        if not st:
            st["step"] = 0
            st["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
            st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
        return st

    def epilogue(self, tensors, skip=None):
        """This step's Adam for the given tensors as the preprocess backward's
        optimizer epilogue (``_lib.AdamEpilogue``), or None when it does not
        apply: a tensor that is not one of this optimizer's parameters (by
        storage), has a gradient already, is not a contiguous ROCm float32
        tensor, or groups that differ in betas or eps. On success each
        parameter's step count is advanced now, as ``step()`` would, and the
        backward leaves its ``.grad`` unset, so ``step()`` skips it. Moments
        that are not contiguous and 16-byte aligned (the kernel moves the SH
        rows as float4) also refuse.

        ``tensors``: means, quats, scales, opacities, sh, sh_rest (None when
        the SH is one fused tensor).

        A parameter this step has already updated (a second render with
        ``optimizer=`` before ``step()``) raises: a second epilogue would be
        a second Adam step.

        ``skip``: the device status of the render's capacity-bounded tile
        lists; the kernel leaves everything as it was if they overflowed
        (``rewind()`` after ``step()`` then takes back the step counts)."""
        owner = {}
        for group in self.param_groups:
            for p in group["params"]:
                owner[(p.data_ptr(), tuple(p.shape))] = (p, group)
        found = []
        for t in tensors:
            if t is None:
                found.append(None)
                continue
            hit = owner.get((t.data_ptr(), tuple(t.shape)))
            if hit is None:
                return None
            p, group = hit
            if id(p) in self._epilogue_applied:
                raise RuntimeError(
                    "FusedAdam: render(optimizer=) already applied this step's update to a "
                    f"parameter of shape {tuple(p.shape)}; call step() after each such render's "
                    "backward, or render without optimizer= and call step() once")
            if (p.grad is not None or p.device.type != "cuda" or p.dtype != torch.float32
                    or not p.is_contiguous()):
                return None
            found.append(hit)
        groups = [g for _, g in filter(None, found)]
        keys = {(tuple(g["betas"]), float(g["eps"])) for g in groups}
        if len(keys) != 1:
            return None
        (b1, b2), eps = next(iter(keys))
        for hit in filter(None, found):
            st = self._state_of(hit[0])
            for mom in (st["exp_avg"], st["exp_avg_sq"]):
                if (not mom.is_contiguous() or mom.data_ptr() % 16 or
                        mom.shape != hit[0].shape):
                    return None
        epi = _lib.AdamEpilogue()
        keep = []
        for i, hit in enumerate(found):
            if hit is None:
                continue
            p, group = hit
            st = self._state_of(p)
            st["step"] += 1
            self._epilogue_applied[id(p)] = p
            epi.p[i], epi.m[i], epi.v[i] = (p.data_ptr(), st["exp_avg"].data_ptr(),
                                             st["exp_avg_sq"].data_ptr())
            epi.lr[i] = float(group["lr"])
            epi.step[i] = int(st["step"])
            keep += [st["exp_avg"], st["exp_avg_sq"]]
        epi.beta1, epi.beta2, epi.eps = float(b1), float(b2), float(eps)
        if skip is not None:
            epi.skip = _skip_ptr(skip)
            keep.append(skip)
        epi._keep = keep
        return epi

    @torch.no_grad()
    def step(self, closure=None, skip=None):
        """One Adam step. ``skip`` (the device status of capacity-bounded
        tile lists, ``render(list_capacity=)``'s ``info["lists_status"]``)
        makes the launch do nothing when the lists overflowed; after such a
        step, ``rewind()`` takes back the step counts before it is run
        again."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        # Checked before the bookkeeping is reset, so a caller that catches
        # the error and steps again still skips these parameters.
        for p in self._epilogue_applied.values():
            if p.grad is not None:
                raise RuntimeError(
                    f"FusedAdam.step(): a parameter of shape {tuple(p.shape)} has a gradient, "
                    "but render(optimizer=) already applied this step's update to it: the "
                    "loss uses it outside the render (a regulariser, for instance). Pass "
                    "the trainer's regularisers to render (opacity_reg=, scale_reg=), or "
                    "render without optimizer=; zero_grad() then step() closes this step "
                    "without a second update.")
        applied, self._epilogue_applied = self._epilogue_applied, {}
        self._last_stepped = list(applied.values())
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
                st = self._state_of(p)
                st["step"] += 1
                self._last_stepped.append(p)
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
                    _lib.check(lib.mg_adam_step_multi_guarded(
                        len(chunk),
                        _lib.ptr_array([it[0].data_ptr() for it in chunk]),
                        _lib.ptr_array([it[1].data_ptr() for it in chunk]),
                        _lib.ptr_array([it[2].data_ptr() for it in chunk]),
                        _lib.ptr_array([it[3].data_ptr() for it in chunk]),
                        _lib.i64_array([it[0].numel() for it in chunk]),
                        _lib.f64_array([it[4] for it in chunk]),
                        _lib.i64_array([it[5] for it in chunk]),
                        b1, b2, eps, 0, None if skip is None else _skip_ptr(skip), s))
                    # Gradients made contiguous above must outlive the launch.
                    del chunk
        return loss

    def rewind(self):
        """Take back the step counts of the last ``step()`` (and of the
        epilogues it closed), whose device update a ``skip`` status turned
        off: parameters and moments are as before that step, and running it
        again advances the counts once more."""
        for p in getattr(self, "_last_stepped", ()):
            self.state[p]["step"] -= 1
        self._last_stepped = []


def _skip_ptr(skip):
    if (not isinstance(skip, torch.Tensor) or skip.dtype != torch.int64 or skip.numel() != 2
            or skip.device.type != "cuda" or not skip.is_contiguous()):
        raise TypeError("skip must be the device int64 (2,) status of render(list_capacity=)")
    return skip.data_ptr()
