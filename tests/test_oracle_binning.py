"""Pins oracle/binning_ref.py (the bit-exact binning restatement).

  * min_q_over_rect is the minimum of the quadratic form over the rectangle:
    checked against dense float64 sampling (no sample below it, the best
    sample close to it), including centres inside, outside and rotated forms;
  * the ellipse test drops only pairs that cannot blend: for every dropped
    (Gaussian, tile) pair, alpha < 1/255 at every pixel centre of the tile in
    float64 (the reference's exactness argument, metal_backend.py:149-165);
  * without the ellipse test the pairs are exactly the rectangle's tiles, the
    same set torch_ref's own binning assigns (torch_ref.py:160-175);
  * a hand-computed known answer for key layout and emission order;
  * sort invariants: keys ascending, ties in emission order, offsets
    monotone with offsets[0] = 0 and offsets[-1] = total.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from conftest import intrinsics, scene
from oracle import binning_ref as B
from oracle import render_ref as R


def test_min_q_over_rect_is_the_rectangle_minimum():
    g = np.random.default_rng(0)
    for _ in range(200):
        mu = g.uniform(-20, 40, 2)
        L = g.normal(size=(2, 2))
        C = L @ L.T + 0.05 * np.eye(2)                    # positive-definite conic
        x0, y0 = g.uniform(0, 16, 2)
        x1, y1 = x0 + g.uniform(1, 16), y0 + g.uniform(1, 16)
        got = float(B.min_q_over_rect(mu[0], mu[1], C[0, 0], C[0, 1], C[1, 1], x0, x1, y0, y1))
        xs, ys = np.meshgrid(np.linspace(x0, x1, 301), np.linspace(y0, y1, 301))
        ex, ey = xs - mu[0], ys - mu[1]
        q = C[0, 0] * ex * ex + 2 * C[0, 1] * ex * ey + C[1, 1] * ey * ey
        assert q.min() >= got - 1e-4 * max(1.0, abs(got)), "a sample lies below the minimum"
        assert q.min() <= got + 0.05 * max(1.0, abs(got)) + 0.2, "minimum not attained"


def _preprocessed(n, seed, W, H):
    s = scene(n=n, seed=seed, z=3.0, spread=0.5, scale=(0.005, 0.08))
    K = intrinsics(W, H, f=200.0)
    uv, conic, depth, rxy, valid, _ = R.preprocess(
        s["means"], s["quats"], s["scales"], s["opacities"], None, torch.eye(4), float(K[0, 0]),
        float(K[1, 1]), float(K[0, 2]), float(K[1, 2]), W, H)
    return [t.detach().numpy().astype(np.float32) for t in (uv, rxy, conic)] + \
        [s["opacities"].numpy(), valid.numpy(), depth.detach().numpy().astype(np.float32)]


def test_dropped_pairs_cannot_blend_anywhere_in_their_tile():
    W, H, tile = 96, 80, 16
    uv, rxy, conic, op, valid, depth = _preprocessed(1500, 1, W, H)
    kr, ir, _ = B.emit_pairs(uv, rxy, conic, op, valid, depth, W, H, tile, ellipse=False)
    ke, ie, _ = B.emit_pairs(uv, rxy, conic, op, valid, depth, W, H, tile, ellipse=True)
    kept = set(zip((ke >> np.uint64(32)).tolist(), ie.tolist()))
    rect = list(zip((kr >> np.uint64(32)).tolist(), ir.tolist()))
    assert len(kept) < len(rect), "the ellipse test removed nothing"
    assert kept <= set(rect)
    tx_n = math.ceil(W / tile)
    dropped = [p for p in rect if p not in kept]
    for t, gi in dropped:
        tx, ty = t % tx_n, t // tx_n
        px = np.arange(tx * tile, min((tx + 1) * tile, W)) + 0.5
        py = np.arange(ty * tile, min((ty + 1) * tile, H)) + 0.5
        X, Y = np.meshgrid(px, py)
        dx, dy = X - float(uv[gi, 0]), Y - float(uv[gi, 1])
        a, b, c = (float(v) for v in conic[gi])
        alpha = float(op[gi]) * np.exp(-0.5 * (a * dx * dx + 2 * b * dx * dy + c * dy * dy))
        assert alpha.max() < 1.0 / 255.0, f"dropped pair (tile {t}, g {gi}) blends"


def test_rectangle_mode_matches_torch_ref_assignment():
    W, H, tile = 96, 80, 16
    s = scene(n=800, seed=2, z=3.0, spread=0.5, scale=(0.01, 0.08))
    K = intrinsics(W, H, f=200.0)
    cov = R.build_cov3d(s["quats"], s["scales"])
    uv, conic, depth, radius, valid, _ = R.project(s["means"], cov, torch.eye(4), float(K[0, 0]),
                                                   float(K[1, 1]), float(K[0, 2]), float(K[1, 2]),
                                                   W, H, 0.01, 100.0)
    tx, ty, buf, total = R.tile_lists(uv, radius, valid, depth, W, H, tile)
    want = {(t, int(g)) for t in range(tx * ty) for g in buf[t].tolist() if g >= 0}
    rxy = torch.stack([radius, radius], -1).numpy().astype(np.float32)
    keys, ids, _ = B.emit_pairs(uv.numpy().astype(np.float32), rxy, None, None, valid.numpy(),
                                depth.numpy().astype(np.float32), W, H, tile, ellipse=False)
    got = set(zip((keys >> np.uint64(32)).tolist(), ids.tolist()))
    assert got == want and len(keys) == total


def test_key_layout_and_emission_order_known_answer():
    """One round Gaussian covering tiles (1..2, 0..1) of a 4x3 grid at tile 16;
    a second, invalid, claims nothing."""
    W, H, tile = 64, 48, 16
    uv = np.array([[32.0, 16.0], [5.0, 5.0]], np.float32)
    rxy = np.array([[9.0, 9.0], [3.0, 3.0]], np.float32)
    conic = np.array([[0.1, 0.0, 0.1], [1.0, 0.0, 1.0]], np.float32)
    op = np.array([0.9, 0.9], np.float32)
    valid = np.array([1, 0], np.int32)
    depth = np.array([2.5, 1.0], np.float32)
    keys, ids, counts = B.emit_pairs(uv, rxy, conic, op, valid, depth, W, H, tile)
    dbits = int(np.float32(2.5).view(np.uint32))
    # tiles x 1..2, y 0..1 in row-major emission: (1,0) (2,0) (1,1) (2,1)
    want = [((ty * 4 + tx) << 32) | dbits for ty in (0, 1) for tx in (1, 2)]
    assert keys.tolist() == want and ids.tolist() == [0, 0, 0, 0]
    assert counts.tolist() == [4, 0]


def test_sort_invariants_and_ties():
    W, H, tile = 96, 80, 16
    uv, rxy, conic, op, valid, depth = _preprocessed(2000, 3, W, H)
    depth[:50] = depth[0]                            # force equal depth bits
    gids, offs, tx, skeys = B.build_tile_lists(uv, rxy, conic, op, valid, depth, W, H, tile)
    assert (skeys[1:] >= skeys[:-1]).all()
    assert offs[0] == 0 and offs[-1] == gids.size and (offs[1:] >= offs[:-1]).all()
    same = skeys[1:] == skeys[:-1]
    assert same.any(), "no ties to check"
    assert (gids[1:][same] > gids[:-1][same]).all(), "ties not in Gaussian order"
    tiles = (skeys >> np.uint64(32)).astype(np.int64)
    for t in range(len(offs) - 1):
        assert (tiles[offs[t]:offs[t + 1]] == t).all()


def test_threshold_is_the_correctly_rounded_log():
    op = np.array([0.004, 0.5, 0.99, 1.0, 0.0039], np.float32)
    thr, live = B.level_threshold(op)
    oa = (np.float32(255.0) * op)
    for o, t, l in zip(oa, thr, live):
        assert l == (o > 1.0)
        if l:
            exact = 2.0 * math.log(float(o))
            assert np.float32(exact) == t
