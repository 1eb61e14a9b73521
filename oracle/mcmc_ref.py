"""Restatement of the MCMC densification step. TEST INFRASTRUCTURE ONLY.

Follows metal_gauss/mcmc.py: relocate 52-104, reset_adam_state 107-121,
grow 124-161, add_noise 164-192, the split constants 33 and 43-49. Every
random draw of the reference (torch.multinomial with replacement, randn) is an
explicit input here:

* ``philox4x64`` restates Philox4x64-10 (Salmon, Moraes, Dror, Shaw, SC'11):
  the random source the HIP kernels draw from (counter = row, key = (seed,
  stream tag));
* ``uniforms`` / ``normals`` turn its output into the kernels' uniforms
  (53- or 24-bit, never 0) and Box-Muller normals;
* ``relocate`` / ``grow`` take one uniform per draw and sample by inverse CDF
  over the candidate rows: the first row whose running weight sum exceeds
  u * total (what torch.multinomial with replacement computes in
  distribution);
* ``add_noise`` takes the normals.

All arithmetic is float64 numpy.

Pinned by tests/test_oracle_mcmc.py:
  * philox4x64 against numpy.random.Philox (an independent implementation of
    Philox4x64-10), bit for bit, for several keys and counters;
  * Box-Muller: z0^2 + z1^2 = -2 ln u1 and atan2(z1, z0) = 2 pi u2 (mod 2 pi)
    per pair, and moments of 200k draws;
  * the sampler: a chi-square test of draw frequencies against the weights;
  * relocate / grow against the reference's invariant tests
    (tests/test_trainer.py:44-79, 213-315): budget kept, dead revived,
    copies and sources split so that N copies composite back to the source
    (1 - o')^N = 1 - o, duplicate picks split N ways, grow ramps and caps;
  * add_noise: the quaternion rotation against render_ref.quat_to_rotmat(q)
    @ eps, the gate, and annealing with the learning rate.
"""

from __future__ import annotations

import numpy as np

MAX_MULTIPLICITY = 51
NOISE_TAG = 0x6E6F697365
DRAW_TAG = 0x7069636B

_M0, _M1 = np.uint64(0xD2E7470EE14C6C93), np.uint64(0xCA5A826395121157)
_W0, _W1 = np.uint64(0x9E3779B97F4A7C15), np.uint64(0xBB67AE8584CAA73B)
_LO = np.uint64(0xFFFFFFFF)
_S32 = np.uint64(32)


def _mulhilo(a, b):
    """(hi, lo) 64-bit halves of the 128-bit product of uint64 arrays."""
    a_lo, a_hi = a & _LO, a >> _S32
    b_lo, b_hi = b & _LO, b >> _S32
    ll = a_lo * b_lo
    lh = a_lo * b_hi
    hl = a_hi * b_lo
    hh = a_hi * b_hi
    mid = (ll >> _S32) + (lh & _LO) + (hl & _LO)
    hi = hh + (lh >> _S32) + (hl >> _S32) + (mid >> _S32)
    lo = a * b
    return hi, lo


def philox4x64(ctr, key):
    """Philox4x64-10. ctr: (n, 4) uint64, key: (2,) or (n, 2) uint64 -> (n, 4)."""
    with np.errstate(over="ignore"):
        c = np.array(ctr, dtype=np.uint64).reshape(-1, 4).copy()
        k = np.broadcast_to(np.array(key, dtype=np.uint64), (c.shape[0], 2)).copy()
        for r in range(10):
            if r:
                k[:, 0] += _W0
                k[:, 1] += _W1
            hi0, lo0 = _mulhilo(np.full(c.shape[0], _M0), c[:, 0])
            hi1, lo1 = _mulhilo(np.full(c.shape[0], _M1), c[:, 2])
            c = np.stack([hi1 ^ c[:, 1] ^ k[:, 0], lo1, hi0 ^ c[:, 3] ^ k[:, 1], lo0], axis=1)
    return c


def _rows_block(n, seed, tag):
    ctr = np.zeros((n, 4), dtype=np.uint64)
    ctr[:, 0] = np.arange(n, dtype=np.uint64)
    return philox4x64(ctr, [seed, tag])


def uniforms(n, seed, tag=DRAW_TAG):
    """u_j in (0,1) from the first word of block j: ((x >> 11) + 1/2) / 2^53."""
    x = _rows_block(n, seed, tag)[:, 0]
    return ((x >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53


def _u24(x):
    return ((x >> np.uint64(40)).astype(np.float64) + 0.5) * 2.0 ** -24


def normals(n, seed, tag=NOISE_TAG):
    """(n,3) Box-Muller normals from block j's four 24-bit uniforms."""
    b = _rows_block(n, seed, tag)
    r0 = np.sqrt(-2.0 * np.log(_u24(b[:, 0])))
    t0 = 2.0 * np.pi * _u24(b[:, 1])
    r1 = np.sqrt(-2.0 * np.log(_u24(b[:, 2])))
    t1 = 2.0 * np.pi * _u24(b[:, 3])
    return np.stack([r0 * np.cos(t0), r0 * np.sin(t0), r1 * np.cos(t1)], axis=1)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, dtype=np.float64)))


def inverse_cdf(weights, u):
    """Row drawn by each uniform: first index whose running sum exceeds u * total."""
    cdf = np.cumsum(np.asarray(weights, dtype=np.float64))
    return np.searchsorted(cdf, u * cdf[-1], side="right")


def split(o, n):
    """(logit of the split opacity, log of the scale ratio) for an N-way split
    of opacity o (mcmc.py:43-49, 80-87)."""
    o_new = 1.0 - np.maximum(1.0 - o, 1e-6) ** (1.0 / n)
    logit_new = np.log(np.clip(o_new, 1e-6, 1 - 1e-6) / np.maximum(1.0 - o_new, 1e-6))
    denom = np.maximum(np.maximum(n, 1) * np.maximum(o_new, 1e-6), 1e-6)
    ratio = np.sqrt(np.clip(o_new / denom, 0.05, 1.0))
    return logit_new, np.log(ratio)


def _weights(opac, weights, n):
    w = opac if weights is None else np.maximum(np.asarray(weights[:n], dtype=np.float64), 0.0)
    if weights is not None:
        raw = np.asarray(weights[:n], dtype=np.float64)
        w = np.where(np.isnan(raw), np.nan, w)
    return w


def relocate(params, dead_thresh=0.005, active=None, weights=None, u=None):
    """mcmc.py:52-104 on a dict of float64 arrays, in place. ``u`` holds one
    uniform per row; dead row d draws with u[d]. Returns (moved, touched rows)."""
    n_total = params["logit_opac"].shape[0]
    n = n_total if active is None else active
    opac = sigmoid(params["logit_opac"][:n])
    dead = np.nonzero(opac < dead_thresh)[0]
    alive = np.nonzero(opac >= dead_thresh)[0]
    if dead.size == 0 or alive.size == 0:
        return 0, np.zeros(0, dtype=np.int64)
    w = _weights(opac, weights, n)
    w_alive = w[alive]
    if not np.isfinite(w_alive).all() or w_alive.sum() <= 0:
        w_alive = opac[alive]
    pick = alive[inverse_cdf(w_alive, u[dead])]
    counts = np.clip(np.bincount(pick, minlength=n), 1, MAX_MULTIPLICITY)
    logit_new, log_ratio = split(opac[pick], counts[pick].astype(np.float64))
    for k in params:
        if k not in ("logit_opac", "log_scales"):
            params[k][dead] = params[k][pick]
    params["log_scales"][dead] = params["log_scales"][pick] + log_ratio[:, None]
    params["logit_opac"][dead] = logit_new
    uniq = np.unique(pick)
    lu, lr = split(opac[uniq], counts[uniq].astype(np.float64))
    params["logit_opac"][uniq] = lu
    params["log_scales"][uniq] += lr[:, None]
    return int(dead.size), np.concatenate([dead, uniq])


def grow(params, target, active, weights=None, u=None):
    """mcmc.py:124-161 on a dict of float64 arrays, in place. ``u`` holds one
    uniform per draw. Returns (new active count, touched rows)."""
    n_total = params["logit_opac"].shape[0]
    target = min(target, n_total)
    add = target - active
    if add <= 0:
        return active, np.zeros(0, dtype=np.int64)
    opac = sigmoid(params["logit_opac"][:active])
    w = _weights(opac, weights, active)
    if not np.isfinite(w).all() or w.sum() <= 0:
        w = opac
    pick = inverse_cdf(np.maximum(w, 1e-8), u[:add])
    dst = np.arange(active, target)
    counts = np.clip(np.bincount(pick, minlength=active), 1, MAX_MULTIPLICITY) + 1
    logit_new, log_ratio = split(opac[pick], counts[pick].astype(np.float64))
    for k in params:
        if k not in ("logit_opac", "log_scales"):
            params[k][dst] = params[k][pick]
    params["log_scales"][dst] = params["log_scales"][pick] + log_ratio[:, None]
    params["logit_opac"][dst] = logit_new
    params["logit_opac"][pick] = logit_new
    params["log_scales"][pick] += log_ratio[:, None]
    return target, np.concatenate([dst, pick])


def add_noise(params, lr_means, weight=4e4, active=None, opacity_gate=0.005, z=None):
    """mcmc.py:164-192 on float64 arrays, in place; ``z`` (n,3) normals."""
    n = params["means"].shape[0] if active is None else active
    opac = sigmoid(params["logit_opac"][:n])
    gate = sigmoid(-100.0 * (opac - opacity_gate))
    eps = z * np.exp(params["log_scales"][:n])
    q = params["quats"][:n]
    q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-12)
    w_, u = q[:, 0:1], q[:, 1:4]
    t = 2.0 * np.cross(u, eps)
    world = eps + w_ * t + np.cross(u, t)
    params["means"][:n] += world * gate[:, None] * lr_means * weight
