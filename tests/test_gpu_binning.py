"""Tile binning on the GPU against the bit-exact numpy oracle
(oracle/binning_ref.py): per-Gaussian counts, emitted keys and ids in
emission order, sorted keys, gauss_ids and tile offsets must be IDENTICAL,
given identical preprocess outputs (the reference's own framing,
tests/test_metal_binning.py:44-59). Also the scan and sort primitives on their
own, and the invariants of tests/test_metal_binning.py:62-104."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import binning_ref

pytestmark = pytest.mark.gpu


def ref_scene(N=20000, W=240, H=320, seed=1):
    """tests/test_metal_binning.py:20-31: rotated, elongated splats at z ~ 3."""
    g = torch.Generator().manual_seed(seed)
    means = torch.randn(N, 3, generator=g) * 0.5
    means[:, 2] += 3.0
    return dict(means=means, quats=torch.randn(N, 4, generator=g),
                scales=torch.rand(N, 3, generator=g) * 0.08 + 0.005,
                op=torch.rand(N, generator=g) * 0.9 + 0.05,
                sh=torch.randn(N, 16, 3, generator=g) * 0.3, W=W, H=H, f=200.0)


def gpu_preprocess(s, dev, viewmat=None):
    from metal_gauss_amd.backend import _PreprocessMetal, _camera

    W, H, f = s["W"], s["H"], s["f"]
    K = torch.tensor([[f, 0, W / 2], [0, f, H / 2], [0, 0, 1.0]])
    vm = torch.eye(4) if viewmat is None else viewmat
    fx, fy, cx, cy, vm_h, cc = _camera(K, vm)
    with torch.no_grad():
        return _PreprocessMetal.apply(
            s["means"].to(dev), s["quats"].to(dev), s["scales"].to(dev), s["sh"].to(dev), None,
            s["op"].to(dev), vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3, float(max(W, H)),
            cc, 3)


def keys_of(gids, offs, depth):
    """Sorted 64-bit keys implied by a list: (tile << 32) | bits(depth[id])."""
    tiles = np.repeat(np.arange(offs.size - 1, dtype=np.uint64), np.diff(offs))
    dbits = depth.astype(np.float32).view(np.uint32).astype(np.uint64)[gids]
    return (tiles << np.uint64(32)) | dbits


def run_both(s, dev, tile, ellipse=True):
    """GPU lists from both pipelines (depth-first, and the 64-bit-key ABI
    chain) and the oracle's; the two GPU pipelines must agree exactly."""
    from metal_gauss_amd.backend import _bin, _bin_keys64

    uv, conic, depth, rxy, valid, _ = gpu_preprocess(s, dev)
    op = s["op"].to(dev)
    args = (uv, rxy, depth, valid, conic if ellipse else None, op if ellipse else None,
            s["W"], s["H"], tile)
    gids, offs, tx = (t.cpu().numpy() if hasattr(t, "cpu") else t for t in _bin(*args))
    g64, o64, _, k64 = _bin_keys64(*args)
    cpu = [t.cpu().numpy() for t in (uv, rxy, conic, op, valid, depth)]
    skeys = keys_of(gids, offs, cpu[5])
    assert np.array_equal(g64.cpu().numpy(), gids) and np.array_equal(o64.cpu().numpy(), offs)
    assert np.array_equal(k64.cpu().numpy().view(np.uint64), skeys)
    rids, roffs, rtx, rkeys = binning_ref.build_tile_lists(
        cpu[0], cpu[1], cpu[2], cpu[3], cpu[4], cpu[5], s["W"], s["H"], tile, ellipse=ellipse)
    return (gids, offs, tx, skeys), (rids, roffs, rtx, rkeys)


@pytest.mark.parametrize("tile", [8, 12, 16, 32])
def test_tile_lists_bit_exact(dev, tile):
    gpu, ref = run_both(ref_scene(), dev, tile)
    assert gpu[2] == ref[2]
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids (sorted order incl. ties) differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


@pytest.mark.parametrize("tile", [8, 16])
@pytest.mark.parametrize("ellipse", [True, False])
def test_large_rectangles_bit_exact(dev, tile, ellipse):
    """Near, wide splats whose rectangles span tens to hundreds of tiles take
    the wave-parallel strip walk (more than 32 tiles), where each tile's edge
    minima are selects between row, column and corner values; mixed with
    small ones, the sorted lists must still equal the oracle's."""
    s = ref_scene(N=6000, seed=11)
    g = torch.Generator().manual_seed(12)
    k = 600
    s["means"][:k, 2] = torch.rand(k, generator=g) * 1.5 + 1.2
    s["scales"][:k] = torch.rand(k, 3, generator=g) * 0.3 + 0.02
    gpu, ref = run_both(s, dev, tile, ellipse=ellipse)
    uv, conic, depth, rxy, valid, _ = gpu_preprocess(s, dev)
    rxy = rxy.cpu().numpy()
    big = ((2 * rxy[:, 0] / tile + 1) * (2 * rxy[:, 1] / tile + 1) > 32) & \
        (valid.cpu().numpy() != 0)
    assert big.sum() > 100, big.sum()
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


@pytest.mark.parametrize("tile", [8, 16])
def test_rectangles_taller_than_the_row_slice_bit_exact(dev, tile):
    """Rectangles of more than 127 tile rows do not fit the strip walk's LDS
    row slice and test each tile from scratch. On a 96 x 4096 image, near
    splats stretched along y span a few hundred tile rows (tile 8 also takes
    the radix route: 6144 tiles). The lists must equal the oracle's."""
    s = ref_scene(N=3000, W=96, H=4096, seed=41)
    g = torch.Generator().manual_seed(42)
    k = 40
    s["means"][:k, 0] = (torch.rand(k, generator=g) - 0.5) * 0.4
    s["means"][:k, 1] = (torch.rand(k, generator=g) - 0.5) * 4.0
    s["means"][:k, 2] = torch.rand(k, generator=g) * 0.6 + 1.2
    s["scales"][:k, 0] = 0.05
    s["scales"][:k, 1] = torch.rand(k, generator=g) * 2.0 + 1.5
    s["scales"][:k, 2] = 0.05
    s["quats"][:k] = torch.tensor([1.0, 0.0, 0.0, 0.0])
    gpu, ref = run_both(s, dev, tile)
    _, _, _, rxy, valid, _ = gpu_preprocess(s, dev)
    ry, v = rxy[:, 1].cpu().numpy(), valid.cpu().numpy() != 0
    assert ((2 * ry / 16 > 130) & v).sum() >= 5, "no rectangle taller than the row slice"
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


@pytest.mark.parametrize("seed", [51, 52])
def test_synthetic_conics_on_large_rectangles_bit_exact(dev, seed):
    """The strip walk's selects against the oracle's per-tile test over
    geometries a scene rarely produces: near-singular conics (b^2 within
    1e-3 of ac), very anisotropic ones, both signs of b, a and c at the
    1e-12 clamp, centres off the image (clamped rectangles) and on tile
    boundaries, on rectangles of 33 to a few thousand tiles. Inputs are
    drawn directly, not projected."""
    from metal_gauss_amd.backend import _bin

    rng = np.random.default_rng(seed)
    N, W, H, tile = 3000, 640, 480, 16
    f32 = np.float32
    uv = np.stack([rng.uniform(-80, W + 80, N), rng.uniform(-80, H + 80, N)], 1).astype(f32)
    on_edge = rng.random(N) < 0.1   # centres exactly on tile boundaries
    uv[on_edge] = (np.round(uv[on_edge] / tile) * tile).astype(f32)
    rxy = rng.uniform(40, 400, (N, 2)).astype(f32)
    a = np.exp(rng.uniform(np.log(1e-5), np.log(1.0), N)).astype(f32)
    c = np.exp(rng.uniform(np.log(1e-5), np.log(1.0), N)).astype(f32)
    corr = rng.uniform(-1.0, 1.0, N)
    near = rng.random(N) < 0.3      # |b| within 1e-3 of sqrt(ac)
    corr[near] = np.sign(corr[near]) * (1.0 - rng.uniform(0.0, 1e-3, near.sum()))
    b = (corr * np.sqrt(a.astype(np.float64) * c)).astype(f32)
    tiny = rng.random(N) < 0.05
    a[tiny] = f32(1e-13)
    conic = np.stack([a, b, c], 1).astype(f32)
    op = rng.uniform(0.01, 0.99, N).astype(f32)
    valid = (rng.random(N) < 0.9).astype(np.int32)
    depth = rng.uniform(0.5, 20.0, N).astype(f32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    gids, offs, _ = _bin(t(uv), t(rxy), t(depth), t(valid), t(conic), t(op), W, H, tile)
    rids, roffs, _, _ = binning_ref.build_tile_lists(uv, rxy, conic, op, valid, depth, W, H,
                                                     tile, ellipse=True)
    area = ((np.floor((uv[:, 0] + rxy[:, 0]) / tile) - np.floor((uv[:, 0] - rxy[:, 0]) / tile) + 1)
            * (np.floor((uv[:, 1] + rxy[:, 1]) / tile) - np.floor((uv[:, 1] - rxy[:, 1]) / tile) + 1))
    assert ((area > 32) & (valid != 0)).sum() > 1000
    assert gids.numel() > 10000, gids.numel()
    assert np.array_equal(offs.cpu().numpy(), roffs), "tile offsets differ"
    assert np.array_equal(gids.cpu().numpy(), rids), "gauss_ids differ"


@pytest.mark.parametrize("ellipse", [True, False])
def test_kept_and_rewalked_large_rectangles_bit_exact(dev, ellipse):
    """The count pass keeps a large rectangle's claims as one 64-bit word per
    walk step, up to 256 words per wave of its workgroup, and the write pass
    replays them; a rectangle that no longer fits is walked again. At
    1920x1080 and tile 16 a rectangle over the whole image (120 x 68 tiles)
    takes 136 steps. Eight of them lead the first 256-Gaussian block, dealt
    two to each of its four waves: each wave keeps the first (136 words) and
    walks the second again (272 > 256). The second block holds a hundred
    rectangles of about 120 to 4000 tiles (near-singular conics among them),
    25 per wave: each wave keeps them until its words run out and walks the
    rest again. The lists must equal the oracle's."""
    from metal_gauss_amd.backend import _bin

    rng = np.random.default_rng(61)
    N, W, H, tile = 512, 1920, 1080, 16
    f32 = np.float32
    uv = np.stack([rng.uniform(0, W, N), rng.uniform(0, H, N)], 1).astype(f32)
    rxy = rng.uniform(2, 7, (N, 2)).astype(f32)
    a = np.exp(rng.uniform(np.log(1e-4), np.log(0.5), N))
    c = np.exp(rng.uniform(np.log(1e-4), np.log(0.5), N))
    corr = rng.uniform(-0.999, 0.999, N)
    # First block: eight whole-image rectangles, wide ellipses.
    uv[:8] = (W / 2, H / 2)
    rxy[:8] = (1500, 900)
    a[:8], c[:8], corr[:8] = 1e-6, 2e-6, rng.uniform(-0.5, 0.5, 8)
    # Second block: a hundred large rectangles.
    big = np.arange(300, 400)
    rxy[big] = rng.uniform(80, 500, (100, 2))
    corr[big[:30]] = np.sign(corr[big[:30]]) * (1.0 - rng.uniform(0.0, 1e-3, 30))
    b = corr * np.sqrt(a * c)
    conic = np.stack([a, b, c], 1).astype(f32)
    op = rng.uniform(0.05, 0.99, N).astype(f32)
    valid = np.ones(N, np.int32)
    depth = rng.uniform(0.5, 20.0, N).astype(f32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    cn, o = (t(conic), t(op)) if ellipse else (None, None)
    gids, offs, _ = _bin(t(uv), t(rxy), t(depth), t(valid), cn, o, W, H, tile)
    rids, roffs, _, _ = binning_ref.build_tile_lists(uv, rxy, conic, op, valid, depth, W, H,
                                                     tile, ellipse=ellipse)
    counts = np.bincount(rids, minlength=N)
    assert (counts[:8] == (W // tile) * ((H + tile - 1) // tile)).all(), counts[:8]
    assert np.array_equal(offs.cpu().numpy(), roffs), "tile offsets differ"
    assert np.array_equal(gids.cpu().numpy(), rids), "gauss_ids differ"


@pytest.mark.parametrize("spread", [0.0, 2e-6, 2e-3, 0.5, 3.0])
def test_depth_windows_of_every_pass_count_bit_exact(dev, spread):
    """The per-tile depth sort takes 8-bit passes over only the bits in which
    a tile's depth keys differ: all depths equal (no pass), a few bits (one),
    about 20 bits (three), and a wide range. The lists must equal the
    oracle's every time."""
    s = ref_scene(N=4000, seed=21)
    g = torch.Generator().manual_seed(22)
    s["means"][:, 2] = 3.0 + spread * torch.randn(4000, generator=g).clamp(-0.9, 0.9)
    gpu, ref = run_both(s, dev, 16)
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


@pytest.mark.parametrize("bits", [8, 9, 12, 17, 18, 24, 25, 27, 28, 29, 30])
def test_depth_key_spans_of_every_digit_plan_bit_exact(dev, bits):
    """Depth keys spanning exactly `bits` bits (positive floats drawn as
    bit patterns, a tenth of them repeated for ties): the depth sort takes
    8-bit passes, or 9-bit ones where they save a pass (9, 17-18, 25-27
    bits) or are needed (29); 30 bits take the long-list path. The lists
    must equal the oracle's."""
    from metal_gauss_amd.backend import _bin

    N, W, H, tile = 3000, 64, 64, 16
    rng = np.random.default_rng(bits)
    f32 = np.float32
    uv = rng.uniform(0, W, (N, 2)).astype(f32)
    rxy = np.full((N, 2), 6.0, f32)
    valid = np.ones(N, np.int32)
    kb = (0x00800000 + rng.integers(0, 1 << bits, N)).astype(np.uint32)
    kb[0], kb[1] = 0x00800000, 0x00800000 + (1 << bits) - 1   # the full span
    rep = rng.random(N) < 0.1
    kb[rep] = kb[rng.integers(0, N, int(rep.sum()))]
    depth = kb.view(f32)
    zeros3, zeros1 = np.zeros((N, 3), f32), np.zeros(N, f32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    gids, offs, _ = _bin(t(uv), t(rxy), t(depth), t(valid), None, None, W, H, tile)
    rids, roffs, _, _ = binning_ref.build_tile_lists(uv, rxy, zeros3, zeros1, valid, depth, W,
                                                     H, tile, ellipse=False)
    assert np.array_equal(offs.cpu().numpy(), roffs), "tile offsets differ"
    assert np.array_equal(gids.cpu().numpy(), rids), "gauss_ids differ"


@pytest.mark.parametrize("crowd", [False, True])
def test_depth_ties_and_long_tile_lists_bit_exact(dev, crowd):
    """Exact depth ties (Gaussians copied onto others, as MCMC's relocation
    does) must come out in id order inside every tile, and lists longer than
    one workgroup's 4096 entries (a crowd of splats over a few tiles) take the
    chunked path; both must equal the oracle's lists."""
    s = ref_scene(N=14000 if crowd else 6000, seed=31)
    g = torch.Generator().manual_seed(32)
    N = s["means"].shape[0]
    if crowd:
        s["means"][:, :2] = (torch.rand(N, 2, generator=g) - 0.5) * 0.06
        s["scales"] = torch.rand(N, 3, generator=g) * 0.01 + 0.004
    src = torch.randint(0, N, (N // 5,), generator=g)
    dst = torch.randperm(N, generator=g)[:N // 5]
    for k in ("means", "quats", "scales", "op"):
        s[k][dst] = s[k][src]
    gpu, ref = run_both(s, dev, 16)
    if crowd:
        assert int(np.diff(gpu[1]).max()) > 4096, int(np.diff(gpu[1]).max())
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


@pytest.mark.parametrize("seed", [51, 52])
def test_long_lists_crowding_one_depth_bucket_bit_exact(dev, seed):
    """Lists of over 4096 entries are first grouped by the top 8 of their key
    bits, and runs of whole groups are sorted as short lists. Here most of a
    list sits at one depth (3.0 plus under 1e-4) with a few splats far in
    front and behind (depths 0.05 to 90: a 27-bit key span), so one group
    holds more than 4096 entries and takes the long passes on its own, and
    a fifth of the splats are exact copies of others (depth ties, id order);
    the lists must equal the oracle's."""
    N, W, H, f = 12000, 64, 48, 200.0
    g = torch.Generator().manual_seed(seed)
    z = 3.0 + torch.rand(N, generator=g) * 1e-4
    far = torch.randperm(N, generator=g)[:600]
    z[far] = torch.exp(torch.rand(600, generator=g) * (math.log(90.0) - math.log(0.05))
                       + math.log(0.05))
    uv = (torch.rand(N, 2, generator=g) - 0.5) * torch.tensor([20.0, 16.0])
    means = torch.stack([uv[:, 0] * z / f, uv[:, 1] * z / f, z], 1)
    quats = torch.randn(N, 4, generator=g)
    scales = (z * 2.0 / f)[:, None] * (torch.rand(N, 3, generator=g) + 0.5)
    op = torch.rand(N, generator=g) * 0.9 + 0.05
    src = torch.randint(0, N, (N // 5,), generator=g)
    dst = torch.randperm(N, generator=g)[:N // 5]
    for t in (means, quats, scales, op):
        t[dst] = t[src]
    s = dict(means=means, quats=quats, scales=scales, op=op, sh=torch.zeros(N, 16, 3),
             W=W, H=H, f=f)
    gpu, ref = run_both(s, dev, 16)
    lens = np.diff(gpu[1])
    assert lens.max() > 4096, lens.max()
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


def test_lists_over_2048_entries_with_four_passes_bit_exact(dev):
    """Every tile's list between 2048 and 4096 entries (one workgroup, its
    four waves' quarters past the 2048 LDS words the lane masks share with the
    exchange buffer) and depth keys spanning about 27 bits (four 8-bit
    passes): 400k small splats placed by pixel over a 256x256 image, depths
    log-uniform in [0.05, 40]. A pass that cleared the masks before every
    wave's read of the shared words had returned gave these lists index 0 in
    their first 2048 positions."""
    N, W, H, f = 400_000, 256, 256, 200.0
    g = torch.Generator().manual_seed(41)
    u = torch.rand(N, generator=g) * W
    v = torch.rand(N, generator=g) * H
    z = torch.exp(torch.rand(N, generator=g) * (math.log(40.0) - math.log(0.05))
                  + math.log(0.05))
    means = torch.stack([(u - W / 2) * z / f, (v - H / 2) * z / f, z], 1)
    quats = torch.zeros(N, 4)
    quats[:, 0] = 1.0
    scales = (z * 1.3 / f)[:, None].expand(N, 3).contiguous()
    s = dict(means=means, quats=quats, scales=scales, op=torch.full((N,), 0.6),
             sh=torch.zeros(N, 16, 3), W=W, H=H, f=f)
    gpu, ref = run_both(s, dev, 16)
    lens = np.diff(gpu[1])
    assert (lens > 2048).mean() > 0.9 and lens.max() <= 4096, (lens.min(), lens.max())
    span_bits = [int(int(k[-1] & 0xFFFFFFFF) - int(k[0] & 0xFFFFFFFF)).bit_length()
                 for k in np.split(gpu[3], gpu[1][1:-1]) if k.size > 1]
    assert min(span_bits) > 24, min(span_bits)
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"
    # The same build repeated in one process: a read-after-barrier race shows
    # up as a run-to-run difference; every repetition must equal the oracle.
    from metal_gauss_amd.backend import _bin

    uv, conic, depth, rxy, valid, _ = gpu_preprocess(s, dev)
    op = s["op"].to(dev)
    for rep in range(8):
        gids, offs, _ = _bin(uv, rxy, depth, valid, conic, op, W, H, 16)
        assert np.array_equal(offs.cpu().numpy(), ref[1]), f"repetition {rep}: offsets differ"
        assert np.array_equal(gids.cpu().numpy(), ref[0]), f"repetition {rep}: gauss_ids differ"


def test_rect_only_lists_bit_exact_and_longer(dev):
    s = ref_scene(seed=3)
    gpu_r, ref_r = run_both(s, dev, 16, ellipse=False)
    assert np.array_equal(gpu_r[3], ref_r[3]) and np.array_equal(gpu_r[0], ref_r[0])
    assert np.array_equal(gpu_r[1], ref_r[1])
    gpu_e, _ = run_both(s, dev, 16, ellipse=True)
    assert gpu_e[0].size < gpu_r[0].size, "the ellipse test removed nothing"


def test_counts_and_emission_order_bit_exact(dev):
    """The unsorted (key, id) stream in (Gaussian, row, column) order."""
    from metal_gauss_amd import _lib

    s = ref_scene(seed=2)
    uv, conic, depth, rxy, valid, _ = gpu_preprocess(s, dev)
    op = s["op"].to(dev)
    W, H, tile = s["W"], s["H"], 16
    tx, ty = math.ceil(W / tile), math.ceil(H / tile)
    lib = _lib.load()
    N = uv.shape[0]
    counts = torch.empty(N, dtype=torch.int32, device=dev)
    st = _lib.stream(uv)
    _lib.check(lib.mg_bin_count(N, uv.data_ptr(), rxy.data_ptr(), conic.data_ptr(), op.data_ptr(),
                                valid.data_ptr(), W, H, tile, tx, ty, counts.data_ptr(), st))
    offs = torch.empty(N, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.mg_scan_workspace_bytes(N), dtype=torch.uint8, device=dev)
    tot = torch.empty(1, dtype=torch.int64, device=dev)
    _lib.check(lib.mg_exclusive_scan_i32(counts.data_ptr(), N, offs.data_ptr(), tot.data_ptr(),
                                         None, ws.data_ptr(), ws.numel(), st))
    total = int(tot.item())
    keys = torch.empty(total, dtype=torch.int64, device=dev)
    ids = torch.empty(total, dtype=torch.int32, device=dev)
    _lib.check(lib.mg_bin_write(N, uv.data_ptr(), rxy.data_ptr(), conic.data_ptr(), op.data_ptr(),
                                valid.data_ptr(), depth.data_ptr(), offs.data_ptr(), total, W, H,
                                tile, tx, ty, keys.data_ptr(), ids.data_ptr(), st))
    cpu = [t.cpu().numpy() for t in (uv, rxy, conic, op, valid, depth)]
    rkeys, rids, rcounts = binning_ref.emit_pairs(*cpu, W, H, tile)
    assert np.array_equal(counts.cpu().numpy(), rcounts)
    assert np.array_equal(offs.cpu().numpy(), np.cumsum(rcounts) - rcounts)
    assert np.array_equal(keys.cpu().numpy().view(np.uint64), rkeys)
    assert np.array_equal(ids.cpu().numpy(), rids)


def test_offsets_are_monotonic_and_complete(dev):
    gpu, _ = run_both(ref_scene(seed=2), dev, 16)
    o = gpu[1].astype(np.int64)
    assert o[0] == 0 and o[-1] == gpu[0].size and (o[1:] >= o[:-1]).all()


def test_all_invalid_scene_gives_empty_lists(dev):
    """tests/test_metal_binning.py:81-104: everything behind the camera."""
    N = 128
    s = dict(means=torch.zeros(N, 3), quats=torch.tensor([[1.0, 0, 0, 0]]).repeat(N, 1),
             scales=torch.full((N, 3), 0.01), op=torch.full((N,), 0.5),
             sh=torch.zeros(N, 16, 3), W=64, H=64, f=100.0)
    s["means"][:, 2] = -5.0
    gpu, _ = run_both(s, dev, 16)
    assert gpu[0].size == 0 and int(gpu[1][-1]) == 0 and gpu[1].shape == (17,)


def test_config2_scale_bit_exact(dev):
    """Full BASELINE configs[1] scene and camera: 300k Gaussians at 800x800."""
    from metal_gauss_amd import scenes

    sc, cam, _ = scenes.config2()
    m, q, sca, op, sh = sc.activated()
    s = dict(means=m, quats=q, scales=sca, op=op, sh=sh, W=cam.W, H=cam.H,
             f=float(cam.K[0, 0]))
    from metal_gauss_amd.backend import _bin, _camera, _PreprocessMetal

    fx, fy, cx, cy, vm_h, cc = _camera(cam.K, cam.viewmat)
    with torch.no_grad():
        uv, conic, depth, rxy, valid, _ = _PreprocessMetal.apply(
            m.to(dev), q.to(dev), sca.to(dev), sh.to(dev), None, op.to(dev), vm_h, fx, fy, cx, cy,
            cam.W, cam.H, 0.01, 100.0, 0.3, float(max(cam.W, cam.H)), cc, 3)
    gids, offs, tx = _bin(uv, rxy, depth, valid, conic, op.to(dev), cam.W, cam.H, 16)
    cpu = [t.cpu().numpy() for t in (uv, rxy, conic, op, valid, depth)]
    rids, roffs, _, rkeys = binning_ref.build_tile_lists(*cpu, cam.W, cam.H, 16)
    print(f"config 2: {int(valid.sum())} valid of {m.shape[0]}, {rids.size} intersections")
    gids, offs = gids.cpu().numpy(), offs.cpu().numpy()
    assert np.array_equal(keys_of(gids, offs, cpu[5]), rkeys)
    assert np.array_equal(gids, rids)
    assert np.array_equal(offs, roffs)


# ------------------------------------------------------------- primitives

@pytest.mark.parametrize("n,bits", [(2_500_001, (0, 44)), (5_000_003, (0, 44)),
                                    (5_000_003, (8, 20))])
def test_radix_sort_large_tiles(dev, n, bits):
    """Sizes that take the 2048- and 4096-key tiles (the small ones above
    take 1024)."""
    test_radix_sort_is_stable_and_exact(dev, n, bits)


@pytest.mark.parametrize("n", [1, 7, 2047, 2048, 2049, 100_003])
@pytest.mark.parametrize("bits", [(0, 44), (0, 40), (0, 64), (8, 20)])
def test_radix_sort_is_stable_and_exact(dev, n, bits):
    from metal_gauss_amd import _lib

    lib = _lib.load()
    g = np.random.default_rng(n * 131 + bits[1])
    # Few distinct values so that ties are everywhere.
    keys = g.integers(0, 2 ** 63, size=n, dtype=np.int64)
    keys = np.where(g.random(n) < 0.5, keys % 977, keys)
    lo, hi = bits
    mask = np.uint64(((1 << (hi - lo)) - 1) << lo) if hi - lo < 64 else np.uint64(2 ** 64 - 1)
    want_order = np.argsort(keys.view(np.uint64) & mask, kind="stable")
    kin = torch.from_numpy(keys).to(dev)
    vin = torch.arange(n, dtype=torch.int32, device=dev)
    kout = torch.empty_like(kin)
    vout = torch.empty_like(vin)
    ws = torch.empty(lib.mg_sort_workspace_bytes(n), dtype=torch.uint8, device=dev)
    _lib.check(lib.mg_sort_pairs_u64(kin.data_ptr(), vin.data_ptr(), kout.data_ptr(),
                                     vout.data_ptr(), n, lo, hi, ws.data_ptr(), ws.numel(),
                                     _lib.stream(kin)))
    assert np.array_equal(vout.cpu().numpy(), want_order.astype(np.int32))
    assert np.array_equal(kout.cpu().numpy(), keys[want_order])


@pytest.mark.parametrize("n,n_tiles,kind", [
    (1, 1, "uniform"), (7, 3, "uniform"), (2049, 300, "uniform"), (300_001, 2500, "uniform"),
    (300_001, 4096, "descending"), (1_000_003, 1, "uniform"), (2_000_000, 2500, "one_hot"),
    (5_000_011, 2500, "uniform"), (7_000_001, 4096, "uniform"), (100_000, 2500, "dropped")])
def test_sort_pairs_by_tile_is_stable_and_exact(dev, n, n_tiles, kind):
    """The one-pass counting sort behind mg_bin_lists_finish against numpy's
    stable argsort: chunk plans from 8 to 64 pairs per lane (n up to 7M),
    one tile, every pair in one tile, reversed input, and tiles past n_tiles
    (dropped; the last offset counts the rest)."""
    from metal_gauss_amd import _lib

    lib = _lib.load()
    g = np.random.default_rng(n + 7 * n_tiles)
    tiles = g.integers(0, n_tiles, size=n, dtype=np.int64)
    if kind == "descending":
        tiles = np.sort(tiles)[::-1].copy()
    elif kind == "one_hot":
        tiles[:] = n_tiles // 3
        tiles[g.random(n) < 0.01] = 0
    elif kind == "dropped":
        tiles[g.random(n) < 0.1] = n_tiles + 5
    ids = g.integers(0, 2 ** 31 - 1, size=n, dtype=np.int64).astype(np.int32)
    keep = tiles < n_tiles
    order = np.argsort(np.where(keep, tiles, n_tiles), kind="stable")[:int(keep.sum())]
    want_offs = np.searchsorted(tiles[order], np.arange(n_tiles + 1))
    t_dev = torch.from_numpy(tiles.astype(np.uint32).view(np.int32)).to(dev)
    i_dev = torch.from_numpy(ids).to(dev)
    out = torch.full((n,), -1, dtype=torch.int32, device=dev)
    offs = torch.full((n_tiles + 1,), -1, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.mg_sort_pairs_by_tile_workspace_bytes(n, n_tiles), dtype=torch.uint8,
                     device=dev)
    _lib.check(lib.mg_sort_pairs_by_tile(n, t_dev.data_ptr(), i_dev.data_ptr(), n_tiles,
                                         out.data_ptr(), offs.data_ptr(), ws.data_ptr(),
                                         ws.numel(), _lib.stream(t_dev)))
    got = out.cpu().numpy()
    assert np.array_equal(offs.cpu().numpy(), want_offs)
    assert np.array_equal(got[:order.size], ids[order])
    assert (got[order.size:] == -1).all(), "wrote past the kept pairs"


@pytest.mark.parametrize("W,H,tile", [(640, 480, 8), (1920, 1080, 16), (2048, 2048, 8)])
def test_more_tiles_bit_exact(dev, W, H, tile):
    """4800, 8160 and 65536 tiles: past 4096 tiles the lists come from the
    radix passes instead of the counting sort, and must equal the
    oracle's."""
    s = ref_scene(N=20000, W=W, H=H, seed=5)
    s["f"] = 200.0 * W / 640
    gpu, ref = run_both(s, dev, tile)
    assert (W // tile) * (H // tile) > 4096
    assert np.array_equal(gpu[3], ref[3]), "sorted keys differ"
    assert np.array_equal(gpu[0], ref[0]), "gauss_ids differ"
    assert np.array_equal(gpu[1], ref[1]), "tile offsets differ"


@pytest.mark.parametrize("n", [1, 2048, 2049, 1_000_003])
def test_exclusive_scan(dev, n):
    from metal_gauss_amd import _lib

    lib = _lib.load()
    counts = torch.randint(0, 40, (n,), dtype=torch.int32, generator=torch.Generator().manual_seed(n))
    want = np.cumsum(counts.numpy().astype(np.int64)) - counts.numpy()
    c = counts.to(dev)
    out = torch.empty_like(c)
    tot = torch.empty(1, dtype=torch.int64, device=dev)
    host = torch.zeros(1, dtype=torch.int64, pin_memory=True)
    ws = torch.empty(lib.mg_scan_workspace_bytes(n), dtype=torch.uint8, device=dev)
    _lib.check(lib.mg_exclusive_scan_i32(c.data_ptr(), n, out.data_ptr(), tot.data_ptr(),
                                         host.data_ptr(), ws.data_ptr(), ws.numel(),
                                         _lib.stream(c)))
    assert np.array_equal(out.cpu().numpy(), want.astype(np.int32))
    assert int(host[0]) == int(counts.sum()) == int(tot.item())


def test_tile_ranges_fill_empty_tiles(dev):
    from metal_gauss_amd import _lib

    lib = _lib.load()
    tiles = np.array([0, 0, 3, 3, 3, 7, 9, 9], dtype=np.uint64)
    keys = torch.from_numpy(((tiles << np.uint64(32)) | np.uint64(5)).view(np.int64)).to(dev)
    offs = torch.empty(12, dtype=torch.int32, device=dev)
    _lib.check(lib.mg_tile_ranges(keys.data_ptr(), 8, 11, offs.data_ptr(), _lib.stream(keys)))
    want = np.searchsorted(tiles.astype(np.int64), np.arange(12))
    assert np.array_equal(offs.cpu().numpy(), want)
