"""Tile lists without a host read: mg_bin_lists_capped, render(list_capacity=)
and ListCapacity, against the two-call lists of mg_bin_lists_begin/_finish
(which the binning tests hold bit-exact to the oracle).

Within capacity the lists must be IDENTICAL to the two-call lists and the
status must read (total, 0); past it the status must read (total, 1) and
every list must be empty (the ids buffer is scratch then); an optimizer step given an
overflowed status must leave parameters, moments and step counts exactly as
they were, and the step run again with the reported capacity must match the
reference order of work (sync-sized lists, backward, step())."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import intrinsics, scene
from test_gpu_binning import gpu_preprocess, ref_scene

pytestmark = pytest.mark.gpu


def _both(s, dev, tile, ellipse, capacity_of, block_work=None, proj=None):
    """Two-call lists, then capacity-bounded lists at capacity_of(total)
    into a sentinel-filled ids buffer (with a block order from
    ``block_work`` if given)."""
    from metal_gauss_amd import _lib, backend

    uv, conic, depth, rxy, valid, _ = gpu_preprocess(s, dev) if proj is None else proj
    op = s["op"].to(dev) if proj is None else proj[5]
    args = (uv, rxy, depth, valid, conic if ellipse else None, op if ellipse else None,
            s["W"], s["H"], tile)
    ids, offs, tx = backend._bin(*args)
    total = ids.numel()
    cap = capacity_of(total)
    lib = _lib.load()
    n_tiles = offs.numel() - 1
    got_ids = torch.full((max(cap, 1),), -7, dtype=torch.int32, device=dev)
    got_offs = torch.full((n_tiles + 1,), -7, dtype=torch.int32, device=dev)
    status = torch.full((2,), -7, dtype=torch.int64, device=dev)
    host = torch.full((3,), -7, dtype=torch.int64, pin_memory=True)
    N = uv.shape[0]
    ws = torch.empty(lib.mg_bin_lists_capped_workspace_bytes(N, cap), dtype=torch.uint8,
                     device=dev)
    _lib.check(lib.mg_bin_lists_capped(
        N, uv.data_ptr(), rxy.data_ptr(), conic.data_ptr() if ellipse else None,
        op.data_ptr() if ellipse else None, valid.data_ptr(), depth.data_ptr(), s["W"], s["H"],
        tile, tx, n_tiles // tx, cap, got_ids.data_ptr() if cap else None, got_offs.data_ptr(),
        status.data_ptr(), host.data_ptr(), 99, ws.data_ptr(), ws.numel(),
        None if block_work is None else block_work.data_ptr(), _lib.stream(uv)))
    torch.cuda.synchronize()
    st = status.cpu().numpy()
    assert host.tolist() == [int(st[0]), int(st[1]), 99], "host slot differs from the device words"
    return (ids.cpu().numpy(), offs.cpu().numpy(), total, cap, got_ids.cpu().numpy(),
            got_offs.cpu().numpy(), st)


CAPS = {
    "exact": lambda t: t,
    "roomy": lambda t: t + 777,
    "double": lambda t: 2 * t + 1,
    "one_short": lambda t: max(t - 1, 0),
    "zero": lambda t: 0,
}


@pytest.mark.parametrize("case", [
    # (N, W, H, tile, ellipse): the counting sort at 300 tiles, once with
    # rectangles only; past 4096 tiles the radix route, at 4800 and 65536
    # tiles, and at 2^13 and 2^15 tiles, where the tile key of the unused
    # slots needs one more bit than the tiles.
    (20000, 240, 320, 16, True), (20000, 240, 320, 16, False), (20000, 640, 480, 8, True),
    (6000, 2048, 1024, 16, True), (6000, 4096, 2048, 16, True), (6000, 2048, 2048, 8, True)])
@pytest.mark.parametrize("cap", list(CAPS))
def test_capped_lists_equal_the_two_call_lists(dev, case, cap):
    n, W, H, tile, ellipse = case
    s = ref_scene(N=n, W=W, H=H, seed=7)
    if W >= 2048:
        s["f"] = 900.0 * W / 2048
    ids, offs, total, capacity, got_ids, got_offs, status = _both(
        s, dev, tile, ellipse, CAPS[cap])
    assert total > 0
    assert status[0] == total, (status, total)
    if total <= capacity:
        assert status[1] == 0
        assert np.array_equal(got_offs, offs), "tile offsets differ"
        assert np.array_equal(got_ids[:total], ids), "gauss_ids differ"
    else:
        assert status[1] == 1
        assert (got_offs == 0).all(), "an overflowed build must leave every list empty"


def _mip_projection(s, dev, tile):
    """The mip projection with its per-block binning work estimate:
    (uv, conic, depth, rxy, valid, opacity_eff), block_work."""
    from metal_gauss_amd.backend import _PreprocessMip, _camera

    W, H, f = s["W"], s["H"], s["f"]
    K = torch.tensor([[f, 0, W / 2], [0, f, H / 2], [0, 0, 1.0]])
    fx, fy, cx, cy, vm_h, cc = _camera(K, torch.eye(4))
    n = s["means"].shape[0]
    bw = torch.full(((n + 255) // 256,), -7, dtype=torch.int32, device=dev)
    with torch.no_grad():
        uv, conic, depth, rxy, valid, _, op = _PreprocessMip.apply(
            s["means"].to(dev), s["quats"].to(dev), s["scales"].to(dev), s["op"].to(dev),
            s["sh"].to(dev), None, None, False, vm_h, fx, fy, cx, cy, W, H, 0.01, 100.0, 0.3,
            float(max(W, H)), cc, 3, None, 0, None, None, None, (tile, bw))
    return (uv, conic, depth, rxy, valid, op), bw


def _host_block_work(uv, rxy, valid, W, H, tile):
    """Per 256 Gaussians: the tiles of each visible Gaussian's clamped
    rectangle (floor((u -+ rx) / tile), exact in float32 for a tile of a power
    of two), capped at 2^22, or 4 for a rectangle of at most 32 tiles."""
    assert tile & (tile - 1) == 0
    tx, ty = -(-W // tile), -(-H // tile)
    it = np.float32(1.0) / np.float32(tile)
    u, v = uv[:, 0], uv[:, 1]
    rx, ry = rxy[:, 0], rxy[:, 1]
    with np.errstate(invalid="ignore", over="ignore"):
        cl = lambda a, hi: np.clip(np.nan_to_num(np.floor(a), nan=0.0, posinf=hi,
                                                 neginf=0.0), 0, hi).astype(np.int64)
        x0, x1 = cl((u - rx) * it, tx - 1), cl((u + rx) * it, tx - 1)
        y0, y1 = cl((v - ry) * it, ty - 1), cl((v + ry) * it, ty - 1)
    area = (x1 - x0 + 1) * (y1 - y0 + 1)
    w = np.where(area > 32, np.minimum(area, 1 << 22), 4)
    w = np.where(valid != 0, w, 0)
    pad = (-w.size) % 256
    return np.concatenate([w, np.zeros(pad, np.int64)]).reshape(-1, 256).sum(1)


@pytest.mark.parametrize("case", [
    # (N, W, H, tile): the counting sort's tile count, then the radix route
    # at 8192 and 2^15 tiles (the sizes render orders blocks at).
    (20000, 240, 320, 16), (6000, 2048, 1024, 16), (6000, 2048, 2048, 8)])
def test_block_order_changes_no_list(dev, case):
    """mg_bin_lists_capped with a block order: the projection's estimate
    (equal to its host recomputation, so heavy blocks go first), or any
    contents at all (random words, negatives, all equal), gives exactly
    the lists without one."""
    n, W, H, tile = case
    s = ref_scene(N=n, W=W, H=H, seed=7)
    if W >= 2048:
        s["f"] = 900.0 * W / 2048
    proj, bw = _mip_projection(s, dev, tile)
    torch.cuda.synchronize()
    cpu = [t.cpu().numpy() for t in proj]
    want = _host_block_work(cpu[0], cpu[3], cpu[4], W, H, tile)
    assert np.array_equal(bw.cpu().numpy(), want), "block work differs from the host's"
    assert want.sum() > 0
    base = _both(s, dev, tile, True, CAPS["roomy"], None, proj)
    g = torch.Generator().manual_seed(3)
    nb = bw.numel()
    for work in (bw, torch.randint(-2 ** 31, 2 ** 31 - 1, (nb,), generator=g,
                                   dtype=torch.int64).to(torch.int32).to(dev),
                 torch.full((nb,), -5, dtype=torch.int32, device=dev),
                 torch.arange(nb, dtype=torch.int32, device=dev) * 997):
        got = _both(s, dev, tile, True, CAPS["roomy"], work, proj)
        total = base[2]
        assert got[2] == total and np.array_equal(got[6], base[6])
        assert np.array_equal(got[5], base[5]), "a block order changed the tile offsets"
        assert np.array_equal(got[4][:total], base[4][:total]), "a block order changed the ids"
        assert np.array_equal(got[4][:total], base[0])


def test_render_with_block_order_equals_render(dev):
    """render past 4096 tiles with capacity lists (the blocks ordered by the
    projection's estimate) gives the image of the sync-sized lists, bit for
    bit, and the same intersection total."""
    from metal_gauss_amd import backend, render

    Wb, Hb = 1920, 1080
    assert -(-Wb // 16) * -(-Hb // 16) > backend._BLOCK_ORDER_TILES
    s = scene(n=20000, seed=5, sh=True)
    p = _leaves(s, dev)
    with torch.no_grad():
        kw = dict(sh_degree=3, sh_rest=p["sh_rest"], background=(0.1, 0.2, 0.3),
                  activations=True)
        args = (p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"],
                intrinsics(Wb, Hb), torch.eye(4), Wb, Hb)
        rgb0, a0, info0 = render(*args, **kw)
        total = info0["isect_total"]
        assert total > 0
        rgb, a, info = render(*args, list_capacity=total + 100, **kw)
        assert info["lists_status"].tolist() == [total, 0]
        assert torch.equal(rgb, rgb0) and torch.equal(a, a0)


def test_capped_lists_of_no_gaussians(dev):
    from metal_gauss_amd import backend

    e = torch.zeros(0, 2, device=dev)
    ids, offs, tx, status = backend._bin_capped(
        e, e, torch.zeros(0, device=dev), torch.zeros(0, dtype=torch.int32, device=dev), None,
        None, 64, 48, 16, 100)
    torch.cuda.synchronize()
    assert status.tolist() == [0, 0]
    assert (offs == 0).all() and offs.numel() == 4 * 3 + 1


def _leaves(s, dev):
    base = dict(means=s["means"], quats=s["quats"], log_scales=s["scales"].log(),
                logits=torch.logit(s["opacities"]), sh_dc=s["sh"][:, :1].contiguous(),
                sh_rest=s["sh"][:, 1:].contiguous())
    return {k: t.clone().to(dev).requires_grad_(True) for k, t in base.items()}


LRS = {"means": 1.6e-4, "quats": 1e-3, "log_scales": 5e-3, "logits": 5e-2, "sh_dc": 2.5e-3,
       "sh_rest": 1.25e-4}
W, H = 200, 150


def _render(p, capacity, opt=None, bg=(0.1, 0.2, 0.3)):
    from metal_gauss_amd import render

    return render(p["means"], p["quats"], p["log_scales"], p["logits"], p["sh_dc"],
                  intrinsics(W, H), torch.eye(4), W, H, sh_degree=3, sh_rest=p["sh_rest"],
                  background=bg, activations=True, optimizer=opt, list_capacity=capacity)


def test_render_with_capacity_equals_render(dev):
    """Same image bit for bit within capacity; the background past it."""
    s = scene(n=3000, seed=21, sh=True)
    p = _leaves(s, dev)
    with torch.no_grad():
        rgb0, a0, info0 = _render(p, None)
        total = info0["isect_total"]
        for cap in (total, total + 5000):
            rgb, a, info = _render(p, cap)
            assert info["lists_status"].tolist() == [total, 0]
            assert int(info["isect_total"]) == total
            assert torch.equal(rgb, rgb0) and torch.equal(a, a0)
        rgb, a, info = _render(p, total - 1)
        assert info["lists_status"].tolist() == [total, 1]
        assert (a == 0).all()
        assert torch.equal(rgb, torch.tensor([0.1, 0.2, 0.3], device=dev).expand_as(rgb))


def test_list_capacity_host_slots_and_device_copies(dev):
    """ListCapacity given to render gets the status words in its pinned
    slots from the kernel itself (several renders outstanding, checked out
    of order); with int capacities, watch() copies them behind an event.
    Both report the total, flag the overflow and grow the capacity."""
    from metal_gauss_amd import ListCapacity

    s = scene(n=3000, seed=21, sh=True)
    p = _leaves(s, dev)
    with torch.no_grad():
        total = _render(p, None)[2]["isect_total"]
        cap = ListCapacity(initial=total - 1, depth=4)
        tickets = [_render(p, cap)[2]["lists_ticket"] for _ in range(3)]
        assert tickets == [0, 1, 2]
        assert cap.overflowed(tickets[2]) and cap.last_total == total
        assert cap.overflowed(tickets[0])
        assert cap.value >= total and cap.overflows == 2
        rgb, _, info = _render(p, cap)
        assert not cap.overflowed(info["lists_ticket"]) and cap.last_total == total
        _render(p, cap)                      # a fifth render reuses ticket 0's slot
        with pytest.raises(RuntimeError, match="no outstanding render"):
            cap.overflowed(0)
        # More than `depth` renders without a poll: the oldest is read before
        # its slot is reused; one that overflowed unchecked is an error.
        quiet = ListCapacity(initial=total + 10, depth=2)
        for _ in range(5):
            _render(p, quiet)
        assert quiet.overflows == 0 and not quiet.overflowed()
        lost = ListCapacity(initial=total - 1, depth=2)
        _render(p, lost)
        _render(p, lost)
        with pytest.raises(RuntimeError, match="never checked"):
            _render(p, lost)
        old = ListCapacity(initial=total - 1)
        _, _, info = _render(p, old.value)
        assert old.overflowed(old.watch(info["lists_status"])) and old.last_total == total
        _, _, info = _render(p, old.value)
        assert not old.overflowed(old.watch(info["lists_status"]))


def _state(opt, p):
    out = {}
    for k, t in p.items():
        st = opt.state[t]
        out[k] = (t.detach().clone(), st["exp_avg"].clone(), st["exp_avg_sq"].clone(),
                  st["step"])
    return out


@pytest.mark.parametrize("epilogue", [True, False])
def test_overflowed_step_changes_nothing_and_the_rerun_matches(dev, epilogue):
    """Three training steps two ways: sync-sized lists with backward and
    step() (the reference's order), and ListCapacity starting at 0, whose
    first render overflows. The overflowed step must leave every parameter,
    moment and step count exactly as it was; after rewind() and the rerun,
    the parameters must match the reference run (the rasteriser's float
    atomics reorder gradient sums run to run: same closeness bar as the
    epilogue's whole-render test)."""
    from metal_gauss_amd import FusedAdam, ListCapacity

    s = scene(n=4000, seed=22, sh=True)
    gt = torch.rand(H, W, 3, generator=torch.Generator().manual_seed(5)).to(dev)

    def make():
        p = _leaves(s, dev)
        return p, FusedAdam([{"params": [t], "lr": LRS[k]} for k, t in p.items()], eps=1e-15)

    p_ref, o_ref = make()
    for _ in range(3):
        rgb, _, _ = _render(p_ref, None)
        o_ref.zero_grad(set_to_none=True)
        (rgb - gt).abs().mean().backward()
        o_ref.step()

    p, opt = make()
    cap = ListCapacity(initial=0)
    for t in p.values():        # moments exist before the first (overflowed) step
        opt._state_of(t)
    before = _state(opt, p)
    reruns = 0
    for step in range(3):
        while True:
            rgb, _, info = _render(p, cap, opt if epilogue else None)
            opt.zero_grad(set_to_none=True)
            (rgb - gt).abs().mean().backward()
            opt.step(skip=info["lists_status"])
            if not cap.overflowed(info["lists_ticket"]):
                break
            reruns += 1
            opt.rewind()
            if step == 0 and reruns == 1:
                after = _state(opt, p)
                for k in p:
                    for a, b in zip(after[k][:3], before[k][:3]):
                        assert torch.equal(a, b), k
                    assert after[k][3] == before[k][3] == 0, k
    assert reruns == 1 and cap.overflows == 1
    assert cap.value >= cap.last_total > 0
    for k in p:
        a, b = p[k].detach(), p_ref[k].detach()
        close = torch.isclose(a, b, rtol=1e-3, atol=1e-4 * LRS[k])
        assert float(close.double().mean()) > 0.999, k
        assert opt.state[p[k]]["step"] == o_ref.state[p_ref[k]]["step"] == 3


def test_forward_frame_captured_in_a_graph_replays_exactly(dev):
    """With capacity-sized lists a render has no host read, so a whole
    forward frame (projection, binning, sorts, compositing) can be captured
    in a HIP graph. Replayed three times, with eager renders and
    synchronisations between the replays, every replay must give the eager
    image bit for bit; moving the camera's scene (the parameters, in place)
    between replays must give the eager image of the moved scene."""
    s = scene(n=3000, seed=23, sh=True)
    p = _leaves(s, dev)
    with torch.no_grad():
        _, _, info = _render(p, None)
        cap = int(info["isect_total"]) * 2
        want, want_a, _ = _render(p, cap)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            _render(p, cap)                     # warm the allocator on this stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            g_rgb, g_a, g_info = _render(p, cap)
        for rep in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(g_rgb, want) and torch.equal(g_a, want_a), rep
            assert g_info["lists_status"].tolist() == [int(info["isect_total"]), 0]
            eager, _, _ = _render(p, cap)       # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(eager, want)
        p["means"].add_(0.01)
        moved, moved_a, _ = _render(p, cap)
        graph.replay()
        torch.cuda.synchronize()
        assert not torch.equal(moved, want)
        assert torch.equal(g_rgb, moved) and torch.equal(g_a, moved_a)


def test_selective_adam_skips_an_overflowed_step(dev):
    """SelectiveAdam given an overflowed status leaves parameters, moments and
    the per-row step counts exactly as they were (row-wise and dense groups);
    after rewind() the step run again with a good status equals an
    optimizer that never saw the overflow, bit for bit."""
    from metal_gauss_amd import SelectiveAdam

    g = torch.Generator().manual_seed(31)
    a0 = torch.randn(5000, 45, generator=g)
    b0 = torch.randn(7, 2, generator=g)
    ga = [torch.randn(5000, 45, generator=g) * 1e-3 for _ in range(2)]
    gb = [torch.randn(7, 2, generator=g) * 1e-3 for _ in range(2)]
    vis = [(torch.rand(5000, generator=g) < 0.6).to(dev) for _ in range(2)]

    def make():
        a = a0.clone().to(dev).requires_grad_(True)
        b = b0.clone().to(dev).requires_grad_(True)
        opt = SelectiveAdam([{"params": [a], "lr": 1e-2}], eps=1e-15)
        opt.add_param_group({"params": [b], "lr": 3e-3, "rowwise": False})
        return a, b, opt

    def snap(a, b, opt):
        out = [a.detach().clone(), b.detach().clone()]
        for t in (a, b):
            st = opt.state[t]
            out += [st["exp_avg"].clone(), st["exp_avg_sq"].clone()]
        out.append(opt.state[a]["steps"].clone())
        return out

    over = torch.tensor([123, 1], dtype=torch.int64, device=dev)
    good = torch.tensor([123, 0], dtype=torch.int64, device=dev)
    a, b, opt = make()
    ra, rb, ref = make()
    for k, (x, y, o) in enumerate(((a, b, opt), (ra, rb, ref))):
        x.grad, y.grad = ga[0].to(dev), gb[0].to(dev)
        o.step(vis[0])
    before = snap(a, b, opt)
    a.grad, b.grad = ga[1].to(dev), gb[1].to(dev)
    opt.step(vis[1], skip=over)
    torch.cuda.synchronize()
    for i, (x, y) in enumerate(zip(snap(a, b, opt), before)):
        assert torch.equal(x, y), i
    assert opt.state[b]["step"] == 2
    opt.rewind()
    assert opt.state[b]["step"] == 1
    opt.step(vis[1], skip=good)
    ra.grad, rb.grad = ga[1].to(dev), gb[1].to(dev)
    ref.step(vis[1])
    for i, (x, y) in enumerate(zip(snap(a, b, opt), snap(ra, rb, ref))):
        assert torch.equal(x, y), i
    assert opt.state[b]["step"] == ref.state[rb]["step"] == 2
