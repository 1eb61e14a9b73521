"""MCMC densification (3DGS-MCMC) on the GPU: the surface of metal_gauss/mcmc.py.

Same functions, arguments and results:

* ``relocate(params, dead_thresh=0.005, opt=None, active=None, weights=None)``
  moves Gaussians whose opacity fell below the threshold onto live ones drawn
  in proportion to ``weights`` (default: opacity), splitting each source's
  opacity N ways and shrinking its scales (mcmc.py:52-104); returns how many
  moved;
* ``grow(params, target, active, opt=None, weights=None)`` clones drawn
  sources into rows active..target (mcmc.py:124-161); returns the new count;
* ``add_noise(params, lr_means, weight=4e4, active=None, opacity_gate=0.005)``
  random-walks the means of near-transparent Gaussians along their own axes
  (mcmc.py:164-192);
* ``reset_adam_state(opt, params, idx)`` zeroes the moments (and
  SelectiveAdam's per-row step counts) of rows (mcmc.py:107-121).

Underneath, each call is HIP kernels (libmgauss ``mg_add_noise``,
``mg_mcmc_weights`` + ``mg_mcmc_apply``): one fused pass for the noise, and
for relocate / grow a weight scan, inverse-CDF draws and two multi-tensor row
passes that also zero the touched rows' optimizer state, where the reference
runs some fifteen torch gather/scatter ops per parameter tensor. Random draws
come from Philox4x64-10 keyed by a seed taken from torch's default CPU
generator, so ``torch.manual_seed`` fixes them, as it fixes the reference's
``multinomial`` and ``randn`` (train.py:253). One host sync per
relocate / grow (the dead count), as in the reference.

``params`` is the trainer's dict: ``logit_opac`` (N,) and ``log_scales``
(N,3) get the split corrections, every other entry is copied row for row
(mcmc.py:36-41). All tensors are float32 ROCm tensors, contiguous, with the
same leading dimension.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

MAX_MULTIPLICITY = 51          # mcmc.py:33, also the kernels' clamp

_CORRECTED = ("logit_opac", "log_scales")

# Row kinds of mg_mcmc_apply.
_COPY, _LOG_SCALES, _LOGIT, _STATE = 0, 1, 2, 3


def _seed() -> int:
    """64 bits from torch's default generator (seeded by torch.manual_seed)."""
    return int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64).item())


def _check_params(params: dict) -> int:
    for k in _CORRECTED:
        if k not in params:
            raise KeyError(f"params needs '{k}'")
    n = params["logit_opac"].shape[0]
    for k, t in params.items():
        if t.device.type != "cuda":
            raise RuntimeError(
                f"hip backend requires ROCm (cuda) tensors, got '{k}' on '{t.device}'. "
                "Refusing to silently move data or fall back to another backend.")
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise RuntimeError(f"params['{k}'] must be a contiguous float32 tensor")
        if t.shape[0] != n:
            raise ValueError(f"params['{k}'] has {t.shape[0]} rows, logit_opac has {n}")
    return n


def _row_table(params: dict, opt):
    """(pointers, widths, kinds) of every parameter and optimizer-state tensor."""
    ptrs, widths, kinds = [], [], []

    def add(t, kind):
        ptrs.append(t.data_ptr())
        widths.append(t[0].numel() if t.dim() > 1 else 1)
        kinds.append(kind)

    for k, t in params.items():
        add(t, _LOGIT if k == "logit_opac" else _LOG_SCALES if k == "log_scales" else _COPY)
    if opt is not None:
        for t in params.values():
            st = opt.state.get(t)
            if not st:
                continue
            for key in ("exp_avg", "exp_avg_sq", "steps"):
                if key in st:
                    s = st[key]
                    if s.dtype != torch.float32 or not s.is_contiguous() or \
                            s.shape[0] != t.shape[0]:
                        raise RuntimeError(f"optimizer state '{key}' must be a contiguous "
                                           "float32 tensor with the parameter's rows")
                    add(s, _STATE)
    return ptrs, widths, kinds


def _run(params, opt, weights, n_rows, thresh, grow, n_draw, dst0, seed):
    """mg_mcmc_weights then, unless nothing is to be done, mg_mcmc_apply.
    Returns the number of copies made (None when there are no candidates)."""
    lib = _lib.load()
    logit = params["logit_opac"]
    dev = logit.device
    w = None
    if weights is not None:
        w = weights[:n_rows].detach().to(torch.float32).contiguous()
        if w.device != dev:
            raise RuntimeError("weights must be on the parameters' device")
    slots = n_draw if grow else n_rows
    ws = torch.empty(lib.mg_mcmc_workspace_bytes(n_rows, slots), dtype=torch.uint8, device=dev)
    tot = (ctypes.c_double * 5)()
    s = _lib.stream(logit)
    _lib.check(lib.mg_mcmc_weights(n_rows, logit.data_ptr(), None if w is None else w.data_ptr(),
                                   float(thresh), int(grow), ws.data_ptr(), ws.numel(), slots,
                                   tot, s))
    n_dead = int(tot[2])
    if grow:
        n_dest = n_draw
    else:
        n_dest = n_dead
        if n_dead == 0 or n_dead == n_rows:
            return 0
    # The reference falls back to opacity when the weights are not finite or
    # sum to nothing (mcmc.py:76-77, 145-146).
    use_opac = w is None or tot[3] != 0.0 or tot[4] == 0.0
    ptrs, widths, kinds = _row_table(params, opt)
    _lib.check(lib.mg_mcmc_apply(
        n_rows, logit.data_ptr(), None if w is None else w.data_ptr(), float(thresh), int(grow),
        int(use_opac), ws.data_ptr(), ws.numel(), slots, n_dest, dst0,
        _seed() if seed is None else int(seed), len(ptrs),
        _lib.ptr_array(ptrs), _lib.i32_array(widths), _lib.i32_array(kinds), s))
    return n_dest


@torch.no_grad()
def relocate(params: dict, dead_thresh: float = 0.005, opt=None, active: int | None = None,
             weights: torch.Tensor | None = None, seed: int | None = None) -> int:
    """Move dead Gaussians onto live ones drawn in proportion to ``weights``
    (default opacity). Returns how many moved (mcmc.py:52-104). ``seed``
    (default: drawn from torch's generator) keys the draws."""
    n_total = _check_params(params)
    n_act = n_total if active is None else int(active)
    if n_act <= 0:
        return 0
    return _run(params, opt, weights, n_act, dead_thresh, False, n_act, 0, seed)


@torch.no_grad()
def grow(params: dict, target: int, active: int, opt=None,
         weights: torch.Tensor | None = None, seed: int | None = None) -> int:
    """Activate rows active..target as clones of drawn live ones; returns the
    new active count, capped at the preallocated size (mcmc.py:124-161)."""
    n_total = _check_params(params)
    target = min(int(target), n_total)
    add = target - int(active)
    if add <= 0:
        return int(active)
    _run(params, opt, weights, int(active), 0.0, True, add, int(active), seed)
    return target


@torch.no_grad()
def add_noise(params: dict, lr_means: float, weight: float = 4e4, active: int | None = None,
              opacity_gate: float = 0.005, eps: torch.Tensor | None = None,
              seed: int | None = None) -> None:
    """SGLD-style exploration of near-transparent Gaussians (mcmc.py:164-192).

    ``eps`` (n,3) supplies the standard normals instead of the kernel's own
    draw (tests use it to compare with the reference's formula); ``seed``
    (default: drawn from torch's generator) keys the kernel's draw.
    """
    lib = _lib.load()
    n = params["means"].shape[0] if active is None else int(active)
    if n <= 0:
        return
    m = params["means"]
    for k in ("means", "log_scales", "quats", "logit_opac"):
        t = params[k]
        if t.device.type != "cuda" or t.dtype != torch.float32 or not t.is_contiguous():
            raise RuntimeError(f"params['{k}'] must be a contiguous float32 ROCm tensor")
        if t.shape[0] < n:
            raise ValueError(f"params['{k}'] has {t.shape[0]} rows, need {n}")
    e = None
    if eps is not None:
        e = eps.detach().to(torch.float32).contiguous()
        if tuple(e.shape) != (n, 3):
            raise ValueError(f"eps must be ({n}, 3)")
    _lib.check(lib.mg_add_noise(n, m.data_ptr(), params["log_scales"].data_ptr(),
                                params["quats"].data_ptr(), params["logit_opac"].data_ptr(),
                                None if e is None else e.data_ptr(), float(lr_means),
                                float(weight), float(opacity_gate),
                                _seed() if seed is None else int(seed), _lib.stream(m)))


@torch.no_grad()
def reset_adam_state(opt, params: dict, idx: torch.Tensor) -> None:
    """Zero Adam moments (and per-row step counts) for rows whose meaning just
    changed (mcmc.py:107-121). relocate and grow already do this in their
    kernels; this is for callers that move rows themselves."""
    for t in params.values():
        st = opt.state.get(t)
        if not st:
            continue
        for key in ("exp_avg", "exp_avg_sq"):
            if key in st:
                st[key][idx] = 0.0
        if "steps" in st:
            st["steps"][idx] = 0.0
