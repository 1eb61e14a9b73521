"""numpy restatement of the two Adam updates. TEST INFRASTRUCTURE ONLY.

adam_step: torch.optim.Adam's update, the oracle of the reference's own
FusedAdam test (tests/test_fused_adam.py:21-38), in the arrangement of
metal_gauss/csrc/adam.metal:34-41 (eps added after the sqrt(bias_correction2)
divide, bias corrections formed in double on the host, rasterize.mm:338-342).
One rounding follows torch rather than that kernel, deliberately: the moment
weights are (1 - beta) rounded from double, as torch's lerp weight and
addcmul value, where adam.metal takes 1 - fp32(beta) in fp32. For beta2 =
0.999 the two weights differ by 1.3e-5 relative (beta1 = 0.9: 2.4e-7), so
exp_avg_sq settles about 1.3e-5 above the reference kernel's and each update
differs by about 6.5e-6 of its own size (far below the parameters' 1e-6
relative bar); the reference's test holds its kernel to torch at 1e-5.

selective_adam_step: metal_gauss/selective_adam.py:116-149 (_step_indexed):
rows with visible[r] get steps[r] += 1 and
p -= lr * sqrt(1 - b2^k)/(1 - b1^k) * m / (sqrt(v) + eps); other rows and
rows past the mask are untouched.

dense_eps_inside_step: selective_adam.py:189-206, ordinary Adam with a scalar
step and eps inside the root (the auxiliary, non-rowwise groups).

Pinned by tests/test_oracle_adam_ssim_raster.py: the closed form of step 1
(dp = -lr g / (|g| + eps)), torch.optim.Adam over 30 and 101 steps, and a
float64 per-row brute force (each row runs plain Adam on exactly the steps
where it was visible, with its own step count).
"""

from __future__ import annotations

import math

import numpy as np

f32 = np.float32


def adam_step(p, g, m, v, lr, b1, b2, eps, step):
    """One in-place fp32 Adam step on flat arrays."""
    bc1 = 1.0 - math.pow(b1, step)
    bc2 = 1.0 - math.pow(b2, step)
    step_size = f32(lr / bc1)
    inv_sqrt_bc2 = f32(1.0 / math.sqrt(bc2))
    b1f, b2f = f32(b1), f32(b2)
    # torch scales the gradient by (1 - beta) formed in double (lerp weight,
    # addcmul value), not by 1 - fp32(beta).
    m[:] = b1f * m + f32(1.0 - b1) * g
    v[:] = b2f * v + f32(1.0 - b2) * g * g
    p[:] = p - step_size * m / (np.sqrt(v) * inv_sqrt_bc2 + f32(eps))


def dense_eps_inside_step(p, g, m, v, lr, b1, b2, eps, step):
    bc1 = 1.0 - math.pow(b1, step)
    bc2 = 1.0 - math.pow(b2, step)
    step_size = f32(lr * math.sqrt(bc2) / bc1)
    b1f, b2f = f32(b1), f32(b2)
    m[:] = b1f * m + f32(1.0 - b1) * g
    v[:] = b2f * v + f32(1.0 - b2) * g * g
    p[:] = p - step_size * m / (np.sqrt(v) + f32(eps))


def selective_adam_step(p, g, m, v, steps, visible, lr, b1, b2, eps):
    """In place on (rows, width) arrays; ``steps`` (rows,) fp32; ``visible``
    (n_visible,) bool with n_visible <= rows."""
    rows = p.shape[0]
    vis = np.zeros(rows, dtype=bool)
    vis[:visible.shape[0]] = visible
    idx = np.nonzero(vis)[0]
    if idx.size == 0:
        return
    k = steps[idx] + f32(1.0)
    steps[idx] = k
    b1f, b2f = f32(b1), f32(b2)
    pw1 = np.power(np.float64(b1f), k.astype(np.float64)).astype(f32)
    pw2 = np.power(np.float64(b2f), k.astype(np.float64)).astype(f32)
    step_size = f32(lr) * (np.sqrt(f32(1.0) - pw2) / (f32(1.0) - pw1))
    shape = (-1,) + (1,) * (p.ndim - 1)
    gs = g[idx]
    mm = m[idx] * b1f + gs * f32(1.0 - b1)
    vv = v[idx] * b2f + gs * gs * f32(1.0 - b2)
    m[idx] = mm
    v[idx] = vv
    p[idx] = p[idx] - step_size.reshape(shape) * mm / (np.sqrt(vv) + f32(eps))
