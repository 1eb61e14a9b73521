"""Bit-exact numpy restatement of the tile binning. TEST INFRASTRUCTURE ONLY.

Restates metal_gauss/csrc/binning.metal:25-120 (tile rectangle, exact
ellipse-vs-tile test, emission order, 64-bit key) and the sort/range glue of
metal_gauss/metal_backend.py:246-260. Every float operation is a single fp32
numpy ufunc, so each product, sum, quotient and floor rounds exactly once as
IEEE fp32, in the same order as the kernel (which is compiled without FP
contraction for this test). The threshold 2 ln(255 op) is taken in float64 and
rounded once to fp32 (the correctly rounded value) on both sides.

Order contract: keys sort ascending by (tile << 32 | depth bits); equal keys
keep emission order (Gaussian, tile row, tile column). The reference's
torch.argsort leaves that tie order unspecified; a stable sort pins it.

Pinned by tests/test_oracle_binning.py:
  * min_q_over_rect against a dense float64 sampling of the rectangle (the
    closed form is the minimum: no sample is below it, one is close to it);
  * every dropped (Gaussian, tile) pair has alpha < 1/255 at every pixel
    centre of the tile, in float64 - the reference's own exactness argument
    (metal_backend.py:149-165) checked by brute force;
  * offsets monotone, offsets[0] = 0, offsets[-1] = total
    (tests/test_metal_binning.py:62-78); keys sorted; ids grouped by tile.
"""

from __future__ import annotations

import math
import os

import numpy as np

f32 = np.float32


def level_threshold(opacity: np.ndarray):
    """(thr fp32, live bool): thr = 2 ln(255 op) correctly rounded; live when
    255 op > 1 (binning.metal:64-68)."""
    oa = f32(255.0) * opacity.astype(f32)
    live = oa > f32(1.0)
    thr = (2.0 * np.log(np.where(live, oa, f32(1.0)).astype(np.float64))).astype(f32)
    return np.where(live, thr, f32(0.0)), live


def min_q_over_rect(mux, muy, ca, cb, cc, x0, x1, y0, y1):
    """Minimum over [x0,x1]x[y0,y1] of a ex^2 + 2 b ex ey + c ey^2
    (binning.metal:25-44), vectorised, fp32, kernel operation order."""
    mux, muy, ca, cb, cc = (np.asarray(t, dtype=f32) for t in (mux, muy, ca, cb, cc))
    x0, x1, y0, y1 = (np.asarray(t, dtype=f32) for t in (x0, x1, y0, y1))
    inside = (mux >= x0) & (mux <= x1) & (muy >= y0) & (muy <= y1)
    a = np.maximum(ca, f32(1e-12))
    b = cb
    c = np.maximum(cc, f32(1e-12))
    two = f32(2.0)
    best = np.full(np.broadcast(mux, x0).shape, np.inf, dtype=f32)
    for yc in (y0, y1):
        xs = np.minimum(np.maximum(mux - b * (yc - muy) / a, x0), x1)
        ex, ey = xs - mux, yc - muy
        best = np.minimum(best, a * ex * ex + two * b * ex * ey + c * ey * ey)
    for xc in (x0, x1):
        ys = np.minimum(np.maximum(muy - b * (xc - mux) / c, y0), y1)
        ex, ey = xc - mux, ys - muy
        best = np.minimum(best, a * ex * ex + two * b * ex * ey + c * ey * ey)
    return np.where(inside, f32(0.0), best).astype(f32)


def tile_rects(uv, rxy, W, H, tile):
    """Inclusive tile index ranges of uv +- rxy, clamped (binning.metal:58-61)."""
    tx_n, ty_n = math.ceil(W / tile), math.ceil(H / tile)
    tf = f32(tile)
    u, v = uv[:, 0].astype(f32), uv[:, 1].astype(f32)
    rx, ry = rxy[:, 0].astype(f32), rxy[:, 1].astype(f32)
    # Gaussians that are not valid may carry non-finite extents; their
    # rectangles are never used.
    with np.errstate(invalid="ignore"):
        x0 = np.clip(np.floor((u - rx) / tf).astype(np.int64), 0, tx_n - 1)
        x1 = np.clip(np.floor((u + rx) / tf).astype(np.int64), 0, tx_n - 1)
        y0 = np.clip(np.floor((v - ry) / tf).astype(np.int64), 0, ty_n - 1)
        y1 = np.clip(np.floor((v + ry) / tf).astype(np.int64), 0, ty_n - 1)
    return x0, x1, y0, y1, tx_n, ty_n


# Candidate (Gaussian, tile) tests per chunk of Gaussians: large scenes are
# cut into chunks of whole Gaussians so the temporaries stay small, and the
# chunks run on a thread pool (numpy releases the GIL inside its loops).
_CHUNK_PAIRS = 1 << 21


def emit_pairs(uv, rxy, conic, opacity, valid, depth, W, H, tile, ellipse=True, workers=None):
    """All surviving (Gaussian, tile) pairs in emission order.

    Returns (keys uint64, ids int32, counts int32 per Gaussian). With
    ``ellipse`` False (no conic), every tile of the rectangle is kept, the
    circular-bounds contract of metal_backend.py:111-147. Gaussians are
    processed in chunks, concatenated in Gaussian order, so the result does
    not depend on the chunking.
    """
    N = uv.shape[0]
    x0, x1, y0, y1, tx_n, _ = tile_rects(uv, rxy, W, H, tile)
    nx, ny = x1 - x0 + 1, y1 - y0 + 1
    per = np.where(valid.astype(bool), nx * ny, 0)
    thr = live = None
    if ellipse:
        thr, live = level_threshold(opacity)
        per = np.where(live, per, 0)
    cum = np.cumsum(per)
    bounds = [0]
    while bounds[-1] < N:
        base = int(cum[bounds[-1] - 1]) if bounds[-1] else 0
        nxt = int(np.searchsorted(cum, base + _CHUNK_PAIRS, side="right"))
        bounds.append(min(N, max(nxt, bounds[-1] + 1)))
    spans = list(zip(bounds[:-1], bounds[1:]))

    def run(span):
        a, b = span
        return _emit_span(a, b, uv, conic, depth, x0, y0, nx, per, thr, ellipse, W, H, tile,
                          tx_n)

    if len(spans) > 1:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(max_workers=workers or min(16, os.cpu_count() or 1)) as ex:
            parts = list(ex.map(run, spans))
    else:
        parts = [run(s) for s in spans]
    keys = np.concatenate([k for k, _ in parts]) if parts else np.zeros(0, np.uint64)
    owner = np.concatenate([o for _, o in parts]) if parts else np.zeros(0, np.int64)
    counts = np.bincount(owner, minlength=N).astype(np.int32)
    return keys, owner.astype(np.int32), counts


def _emit_span(a, b, uv, conic, depth, x0, y0, nx, per, thr, ellipse, W, H, tile, tx_n):
    """Pairs of Gaussians a..b-1, in emission order: (keys, owner int64)."""
    per = per[a:b]
    total = int(per.sum())
    owner = np.repeat(np.arange(a, b, dtype=np.int64), per)
    k = np.arange(total, dtype=np.int64) - np.repeat(np.cumsum(per) - per, per)
    ty = y0[owner] + k // nx[owner]
    tx = x0[owner] + k % nx[owner]
    keep = np.ones(total, dtype=bool)
    if ellipse and total:
        X0 = (tx * tile).astype(f32)
        X1 = np.minimum((tx + 1) * tile, W).astype(f32)
        Y0 = (ty * tile).astype(f32)
        Y1 = np.minimum((ty + 1) * tile, H).astype(f32)
        mq = min_q_over_rect(uv[owner, 0], uv[owner, 1], conic[owner, 0], conic[owner, 1],
                             conic[owner, 2], X0, X1, Y0, Y1)
        keep = mq < thr[owner]
    owner, tx, ty = owner[keep], tx[keep], ty[keep]
    tid = (ty * tx_n + tx).astype(np.uint64)
    dbits = depth.astype(f32).view(np.uint32).astype(np.uint64)[owner]
    return (tid << np.uint64(32)) | dbits, owner


def sort_pairs(keys, ids):
    """Stable ascending sort by key (the radix sort's contract)."""
    order = np.argsort(keys, kind="stable")
    return keys[order], ids[order]


def tile_offsets(sorted_keys, n_tiles):
    """offsets[t] = first index with tile >= t, t = 0..n_tiles
    (metal_backend.py:257-260)."""
    tiles = (sorted_keys >> np.uint64(32)).astype(np.int64)
    return np.searchsorted(tiles, np.arange(n_tiles + 1), side="left").astype(np.int32)


def build_tile_lists(uv, rxy, conic, opacity, valid, depth, W, H, tile, ellipse=True):
    """(gauss_ids int32, tile_offsets int32, tiles_x, sorted keys uint64)."""
    keys, ids, _ = emit_pairs(uv, rxy, conic, opacity, valid, depth, W, H, tile, ellipse)
    sk, sid = sort_pairs(keys, ids)
    tx_n, ty_n = math.ceil(W / tile), math.ceil(H / tile)
    return sid, tile_offsets(sk, tx_n * ty_n), tx_n, sk
