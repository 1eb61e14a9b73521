"""Benchmark: one full training step of the splatting hot path on one MI355X.

Workload ("config 4"): 1,000,000 Gaussians with SH
degree 3, 800x800 views from 100 seeded cameras on a radius-4 sphere, loss
0.8 L1 + 0.2 (1 - SSIM) against smooth random targets, then fused Adam over the
six parameter groups. A step is: activations, render forward (preprocess,
binning, raster with the background blend), the fused L1 + SSIM loss,
backward (loss, raster, preprocess), Adam. Inputs and
targets are resident in HBM before timing.

Prints ONE JSON line with the driver's fields plus:
  roofline      the dominant kernel's algorithmic bytes per launch / its mean
                launch time (HIP events on its own stream, inside the library)
                against MI355X's 8 TB/s HBM peak;
  cpu_baseline  the CPU oracle (oracle/render_ref.py, a restatement of the
                reference's torch renderer, + torch.optim.Adam) on a bounded
                sample of the same step, scaled to full-step steps/s;
  kernels       mean ms per launch of every library kernel in the step.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "train steps/sec & fwd+bwd ms at 1M Gaussians 800×800 SH3; % HBM roofline"
HBM_PEAK_GBS = 8000.0
# Opacity and scale regulariser weights of the reference's step.
REG = 0.01
# Seconds of sustained load before the warm-up steps (bench/quick.py:110-133).
RAMP_S = 2.0

# Kernels timed by the library (names used in mg_timing_query).
KERNELS = ["preprocess_forward", "bin_count", "exclusive_scan", "bin_write", "tile_sort",
           "depth_sort", "rasterize_forward", "rasterize_backward",
           "preprocess_backward", "preprocess_backward_adam", "ssim_fused_forward",
           "ssim_fused_backward", "adam_step", "tile_ranges"]

# Library timing label -> the kernel name rocprofv3 reports for it (for the
# tile sort, its scatter kernel; the scan runs three kernels and is left out).
PROF_NAMES = {
    "preprocess_forward": "preprocess_fwd_kernel", "preprocess_backward": "preprocess_bwd_kernel",
    "preprocess_backward_adam": "preprocess_bwd_adam_kernel",
    "bin_count": "bin_count_rec_kernel", "bin_write": "bin_write_rec_kernel",
    "tile_sort": "count_scatter_kernel", "depth_sort": "tile_depth_sort_kernel",
    "rasterize_forward": "raster_fwd_kernel",
    "rasterize_backward": "raster_bwd_kernel", "ssim_fused_forward": "ssim_fused_fwd_kernel",
    "ssim_fused_backward": "ssim_fused_bwd_kernel", "adam_step": "adam_multi_kernel",
}
TRAFFIC_FILE = ROOT / "profiles" / "pmc_traffic_config4.txt"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--gaussians", type=int, default=1_000_000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--variant", default="base",
                    choices=["base", "unfused-adam", "torch-act", "mip", "mip-torch"],
                    help="base: the config-4 step, exp/sigmoid of the parameters inside the "
                         "projection kernel (render(activations=True)) and FusedAdam's "
                         "update inside its backward (render(optimizer=)); unfused-adam: the "
                         "same with FusedAdam.step() as its own launch after the backward; "
                         "torch-act: the same "
                         "step with exp/sigmoid in torch before render (train.py:221-222); "
                         "mip: with Mip-Splatting's 3D filter and the 2D antialias "
                         "compensation folded into the projection kernel "
                         "(render(filter_3d=, antialias=True)); mip-torch: the same step with "
                         "the activations and the 3D filter applied as the reference's torch "
                         "reparameterisation (apply_3d_filter, train.py:223-227) before render")
    ap.add_argument("--ramp", type=float, default=RAMP_S,
                    help="seconds of sustained forward+backward load before the warm-up "
                         "steps (the reference's clock ramp); 0 for profiling runs")
    ap.add_argument("--counter-summary", nargs="+", metavar="DIR",
                    help="print the per-kernel counter summary of rocprofv3 --pmc runs (one "
                         "directory per pass, with a kernel_stats.csv among them) and exit")
    ap.add_argument("--lists", choices=["capacity", "sync"], default="capacity",
                    help="tile-list sizing in the timed step: capacity-sized with a device "
                         "overflow check (no host read inside the step; default), or by a "
                         "host read of the total in every render as the reference")
    ap.add_argument("--reg", action="store_true",
                    help="add the reference trainer's opacity and scale regularisers, "
                         "0.01 mean sigmoid(logit) + 0.01 mean exp(log_scales) "
                         "(bench/step_profile.py:101-102), to the configuration's loss "
                         "0.8 L1 + 0.2 (1 - SSIM)")
    ap.add_argument("--cpu-only", action="store_true", help="time only the CPU baseline")
    ap.add_argument("--config", type=int, choices=[1, 2, 3, 5], default=None,
                    help="time another BASELINE configuration instead of the config-4 step: "
                         "1 forward at 10k/256^2; 2 fwd+bwd at 300k/800^2; 3 FusedAdam and "
                         "SelectiveAdam over 1M Gaussians; 5 fwd+bwd at 3M/1920x1080")
    ap.add_argument("--crowded", action="store_true",
                    help="with --config 5: the crowded variant (a dense cluster in front of the "
                         "camera: tile lists over 10k entries, over 30M intersections)")
    ap.add_argument("--chunked-backward", choices=["off", "on"], default="off",
                    help="with --config 2/5: render(chunked_backward=...)")
    ap.add_argument("--render-fps", action="store_true",
                    help="forward-only frames per second at the reference's published points "
                         "(bench/render_fps.py, README.md:145-148)")
    ap.add_argument("--ply", action="store_true",
                    help="time writing and reading a 1M-Gaussian SH3 .ply (export_ply from the "
                         "GPU, load_ply to the GPU and to the CPU)")
    ap.add_argument("--mcmc", action="store_true",
                    help="time the MCMC densification kernels (add_noise, relocate, grow) on the "
                         "config-4 parameters instead of the step")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the HBM traffic summary of two rocprofv3 --pmc runs and exit")
    ap.add_argument("--stats-summary", metavar="KERNEL_STATS_CSV",
                    help="print a rocprofv3 kernel-stats summary and exit")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device 3 times (a plain copy of "
                         "known size, to calibrate the FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def copy_calibration(mib):
    import torch

    n = mib * (1 << 18)                       # floats
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


class Step:
    """The config-4 training step on the GPU."""

    def __init__(self, n, dev, variant="base", reg=False, lists="capacity"):
        import torch

        from metal_gauss_amd import FusedAdam, ListCapacity, gaussian_kernel, scenes

        sc, cams, self.bg = scenes.config4(n)
        sc = sc.to(dev)
        self.cams = cams
        self.p = {k: getattr(sc, k).clone().requires_grad_(True)
                  for k in ("means", "log_scales", "quats", "logit_opac", "sh_dc", "sh_rest")}
        lr = {name: l for name, _, l in scenes.config3_groups()}
        self.opt = FusedAdam([
            {"params": [self.p["means"]], "lr": lr["means"]},
            {"params": [self.p["log_scales"]], "lr": lr["scales"]},
            {"params": [self.p["quats"]], "lr": lr["quats"]},
            {"params": [self.p["logit_opac"]], "lr": lr["opac"]},
            {"params": [self.p["sh_dc"]], "lr": lr["sh_dc"]},
            {"params": [self.p["sh_rest"]], "lr": lr["sh_rest"]},
        ], eps=1e-15)
        self.targets = [scenes.config4_target(v).to(dev) for v in range(len(cams))]
        self.window = gaussian_kernel(device=dev, groups=15)
        # d loss / d loss, allocated once: loss.backward() would fill a new
        # one every step (a kernel launch of its own).
        self.seed = torch.ones((), device=dev)
        g = torch.Generator().manual_seed(3)
        self.order = torch.randperm(len(cams), generator=g).tolist()
        self.k = 0
        self.last_isect = 0
        self.variant = variant
        self.reg = reg
        # "capacity": tile lists sized by a ListCapacity, no host read inside
        # the step (an overflowed step changes nothing and runs again);
        # "sync": sized by reading the total on the host, as the reference.
        self.cap = ListCapacity() if lists == "capacity" else None
        self.reruns = 0
        self.f3d = None
        self.f3d_ms = None
        if variant in ("mip", "mip-torch"):
            self.f3d_ms = self.refresh_filter()

    def refresh_filter(self):
        """Mip 3D filter sizes over all views (compute_3d_filter), as the
        reference's trainer recomputes them every 100 steps; returns ms."""
        import torch

        from metal_gauss_amd import compute_3d_filter

        class _V:
            def __init__(self, c):
                self.K, self.viewmat = c.K, c.viewmat
                self.image = torch.empty(c.H, c.W, 0)

        views = [_V(c) for c in self.cams]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        self.f3d = compute_3d_filter(self.p["means"], views)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3

    def __call__(self, adam=True):
        v = self.order[self.k % len(self.order)]
        self.k += 1
        while True:
            loss, info = self.once(v, adam)
            if self.cap is None:
                self.last_isect = info["isect_total"]
                return loss
            if not self.cap.overflowed():
                self.last_isect = self.cap.last_total
                return loss
            # The lists overflowed: the kernels changed nothing; the step
            # counts are taken back and the step runs again, larger.
            self.reruns += 1
            if adam:
                self.opt.rewind()

    def once(self, v, adam):
        import torch

        from metal_gauss_amd import photometric_loss, render

        cam, gt, p = self.cams[v], self.targets[v], self.p
        # exp(log_scales) and sigmoid(logit_opac) (train.py:221-222) run inside
        # the projection kernel and its backward; the "-torch" variants take
        # them in torch as the reference's trainer does.
        # With adam, "base" and "mip" run FusedAdam's update inside the
        # projection backward (render(optimizer=)); the other variants, and
        # "unfused-adam", take it as a separate launch after the backward.
        # With reg, the reference trainer's opacity and scale regularisers,
        # 0.01 mean(sigmoid(logit)) + 0.01 mean(exp(log_scales))
        # (bench/step_profile.py:101-102, train.py:396-398 with the defaults
        # at 733-734), join the configuration's loss: inside the projection
        # backward for "base" and "mip" (render(opacity_reg=, scale_reg=)),
        # in torch for the others.
        reg = dict(opacity_reg=REG, scale_reg=REG) if self.reg else {}
        scales, opac = p["log_scales"], p["logit_opac"]
        epi = self.opt if adam else None
        kw = dict(activations=True, optimizer=epi, **reg)
        torch_reg = False
        if self.variant == "unfused-adam":
            kw = dict(activations=True)
            torch_reg = self.reg
        elif self.variant == "mip":
            kw = dict(filter_3d=self.f3d, antialias=True, activations=True, optimizer=epi, **reg)
        elif self.variant == "torch-act":
            scales, opac = torch.exp(scales), torch.sigmoid(opac)
            kw = {}
            torch_reg = self.reg
        elif self.variant == "mip-torch":
            from metal_gauss_amd import apply_3d_filter
            scales, opac = apply_3d_filter(torch.exp(scales), torch.sigmoid(opac), self.f3d)
            kw = dict(antialias=True)
            torch_reg = self.reg
        rgb, alpha, info = render(p["means"], p["quats"], scales, opac, p["sh_dc"], cam.K,
                                  cam.viewmat, cam.W, cam.H, sh_degree=3, sh_rest=p["sh_rest"],
                                  background=self.bg, list_capacity=self.cap, **kw)
        # 0.8 * |rgb - gt|.mean() + 0.2 * (1 - ssim(rgb, gt)) (train.py:389-390), fused.
        loss, _ = photometric_loss(rgb, gt, self.window, 0.2)
        if torch_reg:
            loss = loss + REG * torch.sigmoid(p["logit_opac"]).mean() \
                + REG * torch.exp(p["log_scales"]).mean()
        elif info["regularizer"] is not None:
            # The loss value the trainer reports; the regularisers' gradient
            # is already in render's backward.
            loss = loss + info["regularizer"]()
        self.opt.zero_grad(set_to_none=True)
        loss.backward(self.seed)
        if adam:
            self.opt.step(skip=info["lists_status"])
        self.last_valid = info["valid_mask"]
        return loss, info


def algorithmic_bytes(kernel, N, I, P, T, f_valid, n_floats):
    """HBM bytes one launch must move, each tensor read or written once."""
    return {
        # + the activated opacity written (forward); the logit read, its
        # record gradient read and the logit gradient written (backward).
        "preprocess_forward": (96 + 192 * f_valid) * N,
        "preprocess_backward": (320 + 192 * f_valid) * N,
        "bin_count": 80 * N,                      # 40 B read; count, 32 B record, claim mask
        "exclusive_scan": 16 * N // 256,          # per-workgroup totals read, block offsets written
        "bin_write": 40 * N + 12 * I,             # count, record, mask; tile key + {id, depth} per pair
        "tile_sort": 24 * I,                      # tiles read twice, 8-byte values read and written
        "depth_sort": 12 * I,                     # per tile list: ids read, depths gathered, ids written
        "tile_ranges": 4 * I + 4 * (T + 1),
        "rasterize_forward": 40 * I + 24 * P + 8 * T,
        "rasterize_backward": 40 * I + 24 * P + 36 * N,
        "ssim_fused_forward": 60 * P,
        "ssim_fused_backward": 72 * P,
        "adam_step": 28 * n_floats,
        # With the optimizer epilogue: the 59 floats of parameters and their
        # two moments read and written, the valid flag and the record
        # gradient read; no gradient written.
        "preprocess_backward_adam": (1416 + 44) * N,
    }[kernel]


def gpu_bench(args):
    import torch

    from metal_gauss_amd import _lib

    dev = torch.device("cuda:0")
    step = Step(args.gaussians, dev, args.variant, reg=args.reg, lists=args.lists)
    # Clock ramp as the reference's bench/quick.py:110-133 does (2 s of
    # sustained load), with forward + backward only so the parameters the
    # timed steps start from are untouched; then the warm-up steps.
    ramp_end = time.perf_counter() + args.ramp
    while time.perf_counter() < ramp_end:
        step(adam=False)
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    # K timed steps: wall clock around all of them (the value), and a HIP
    # event between consecutive steps on the stream the kernels run on (the
    # median per step).
    reruns0 = step.reruns
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    reruns = step.reruns - reruns0
    # The median step from HIP events recorded between consecutive steps, in
    # a loop of its own (an event on the stream costs each step a few us).
    ne = max(10, args.steps // 5)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(ne + 1)]
    for k in range(ne):
        events[k].record()
        step()
    events[-1].record()
    torch.cuda.synchronize()
    per_step = sorted(events[k].elapsed_time(events[k + 1]) for k in range(ne))
    median_ms = per_step[len(per_step) // 2]

    # The same steps with the lists sized by a host read in every render (the
    # reference's way), fewer of them.
    sync_ms = None
    if step.cap is not None:
        cap, step.cap = step.cap, None
        nsync = max(10, args.steps // 4)
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(nsync):
            step()
        torch.cuda.synchronize()
        sync_ms = (time.perf_counter() - t0) * 1e3 / nsync
        step.cap = cap

    # fwd+bwd alone (no optimizer step), fewer iterations.
    nfb = max(10, args.steps // 4)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(nfb):
        step(adam=False)
    torch.cuda.synchronize()
    fb_ms = (time.perf_counter() - t0) * 1e3 / nfb

    # Per-kernel mean launch time, HIP events recorded inside the library.
    nt = 10
    isects = []
    with _lib.KernelTimer():
        for _ in range(nt):
            step()
            isects.append(step.last_isect)
        torch.cuda.synchronize()
        kern = {}
        for k in KERNELS:
            tot, cnt = _lib.KernelTimer.query(k)
            if cnt:
                kern[k] = (tot / cnt, cnt / nt)      # ms per launch, launches per step
    N = args.gaussians
    I = sum(isects) / len(isects)
    P = 800 * 800
    T = 50 * 50
    f_valid = float(step.last_valid.float().mean())
    n_floats = sum(p.numel() for p in step.p.values())
    def nbytes_of(k):
        return algorithmic_bytes(k, N, I, P, T, f_valid, n_floats)

    dominant = max(kern, key=lambda k: kern[k][0] * kern[k][1])
    avg_ms = kern[dominant][0]
    nbytes = nbytes_of(dominant)
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    rows = {k: {"ms": round(v[0], 4), "per_step": v[1],
                "GBps": round(nbytes_of(k) / (v[0] * 1e-3) / 1e9, 1)}
            for k, v in kern.items()}
    f3d_ms = None
    if args.variant in ("mip", "mip-torch"):
        with _lib.KernelTimer():
            wall = step.refresh_filter()
            tot, cnt = _lib.KernelTimer.query("compute_3d_filter")
        f3d_ms = (tot / max(cnt, 1), wall)
    work = raster_work(step, kern)
    return dict(ms=ms, median_ms=median_ms, fb_ms=fb_ms, kernels=rows, dominant=dominant,
                achieved=achieved, nbytes=nbytes, I=I, f_valid=f_valid, n_floats=n_floats,
                f3d_ms=f3d_ms, work=work, copy=stream_copy(), reruns=reruns, sync_ms=sync_ms,
                fwd=forward_fps(step))


def valu_roofline(kernels):
    """The rasteriser's kernels against the VALU issue rate: wave
    instructions per launch (SQ_INSTS_VALU from the committed counter
    summary of this step) over the live mean launch time."""
    out = {}
    for label in ("rasterize_backward", "rasterize_forward"):
        n = committed_valu(label)
        row = kernels.get(label)
        if n is None or row is None:
            continue
        achieved = n / (row["ms"] * 1e-3) / 1e9
        out[label] = {"bound": "valu", "achieved": round(achieved, 1), "peak": VALU_PEAK_GIPS,
                      "unit": "G wave-instructions/s", "frac": round(achieved / VALU_PEAK_GIPS, 4),
                      "instructions_per_launch": int(n)}
    return out


def forward_fps(step, frames=100):
    """Forward-only rendering of the step's views at its current
    parameters (no autograd): frames enqueued back to back with
    capacity-sized lists (an overflowed frame found one frame later is
    rendered again), and one synchronised frame at a time with the lists
    sized by a host read, the reference's way (bench/render_fps.py:30-44)."""
    import torch

    from metal_gauss_amd import ListCapacity, render

    p = step.p
    views = [step.cams[step.order[i % len(step.order)]] for i in range(frames)]

    def frame(cam, cap):
        return render(p["means"], p["quats"], p["log_scales"], p["logit_opac"], p["sh_dc"],
                      cam.K, cam.viewmat, cam.W, cam.H, sh_degree=3, sh_rest=p["sh_rest"],
                      background=step.bg, activations=True, list_capacity=cap)

    cap = ListCapacity(initial=step.cap.value if step.cap is not None else 0)
    redo = 0
    with torch.no_grad():
        for rep in range(2):              # the first pass sizes the capacity
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            tickets = []
            for i, cam in enumerate(views):
                _, _, info = frame(cam, cap)
                tickets.append(info["lists_ticket"])
                if i and cap.overflowed(tickets[i - 1]):
                    redo += rep
                    _, _, info = frame(views[i - 1], cap)
                    cap.overflowed(info["lists_ticket"])
            if cap.overflowed(tickets[-1]):
                redo += rep
                frame(views[-1], cap)
            torch.cuda.synchronize()
            pipelined = (time.perf_counter() - t0) * 1e3 / frames
        ts = []
        for cam in views[:30]:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            frame(cam, None)
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
    ts.sort()
    sync_ms = 1e3 * ts[len(ts) // 2]

    # One view, frames back to back: eager, and captured once as a HIP graph
    # (no host read in the frame) and replayed.
    cam = views[0]
    with torch.no_grad():
        def one_view_ms(run):
            for _ in range(5):
                run()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(frames):
                run()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / frames

        eager_ms = one_view_ms(lambda: frame(cam, cap))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            frame(cam, cap.value)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _, _, g_info = frame(cam, cap.value)
        graph_ms = one_view_ms(graph.replay)
        if int(g_info["lists_status"][1]):
            raise RuntimeError("graph-captured frame overflowed its lists")
        del graph
    return {"pipelined_capacity_lists": {"ms_per_frame": round(pipelined, 4),
                                         "fps": round(1e3 / pipelined, 1), "rerendered": redo},
            "synchronised_sync_lists": {"ms_per_frame": round(sync_ms, 4),
                                        "fps": round(1e3 / sync_ms, 1)},
            "one_view_eager": {"ms_per_frame": round(eager_ms, 4),
                               "fps": round(1e3 / eager_ms, 1)},
            "one_view_graph_replay": {"ms_per_frame": round(graph_ms, 4),
                                      "fps": round(1e3 / graph_ms, 1)},
            "frames": frames, "workload": "config-4 views, 1M Gaussians, 800x800"}


def raster_work(step, kern, views=8):
    """The rasteriser's work count E over `views` of the step's cameras at the
    current parameters: E_fwd = sum over pixels of the list entries the
    per-pixel compositing evaluates (up to the stop entry when the pixel's
    transmittance fell below 1e-4, else the whole tile list), E_bwd = sum of
    the entries the backward replays (tile start to stop index). From the
    forward's own stop indices and final T; per second against the step's
    mean raster kernel times."""
    import torch

    from metal_gauss_amd import _lib, backend

    lib = _lib.load()
    p = step.p
    e_f = e_b = 0.0
    n = 0
    for v in step.order[:views]:
        cam = step.cams[v]
        fx, fy, cx, cy, vm_h, cc = backend._camera(cam.K, cam.viewmat)
        with torch.no_grad():
            valid_b = torch.empty(p["means"].shape[0], dtype=torch.bool, device=p["means"].device)
            uv, conic, depth, rxy, valid, color, op = backend._PreprocessMip.apply(
                p["means"], p["quats"], p["log_scales"], p["logit_opac"], p["sh_dc"],
                p["sh_rest"], None, False, vm_h, fx, fy, cx, cy, cam.W, cam.H, 0.01, 100.0, 0.3,
                float(max(cam.W, cam.H)), cc, 3, valid_b, 3)
            ids, offs, tx = backend._bin(uv, rxy, depth, valid, conic, op, cam.W, cam.H, 16)
            W, H = cam.W, cam.H
            rgb = torch.empty(H, W, 3, device=uv.device)
            alpha = torch.empty(H, W, device=uv.device)
            T = torch.empty(H, W, device=uv.device)
            stop = torch.empty(H, W, dtype=torch.int32, device=uv.device)
            _lib.check(lib.mg_rasterize_forward(
                uv.shape[0], uv.data_ptr(), conic.data_ptr(), op.data_ptr(), color.data_ptr(),
                ids.data_ptr(), offs.data_ptr(), W, H, 16, tx, backend.DEFAULT_T_MIN, None,
                ids.numel(), None, 0, rgb.data_ptr(), alpha.data_ptr(), T.data_ptr(),
                stop.data_ptr(), None, None, _lib.stream(uv)))
            ty_ = torch.arange(H, device=uv.device) // 16
            tx_ = torch.arange(W, device=uv.device) // 16
            tile = ty_[:, None] * tx + tx_[None, :]
            start = offs[tile].long()
            end = offs[tile + 1].long()
            done = T < backend.DEFAULT_T_MIN
            e_f += float(torch.where(done, stop.long() - start, end - start).sum())
            e_b += float((stop.long() - start).sum())
            n += 1
    e_f, e_b = e_f / n, e_b / n
    out = {"views": n, "E_fwd": int(e_f), "E_bwd": int(e_b)}
    if "rasterize_forward" in kern:
        out["fwd_E_per_s"] = round(e_f / (kern["rasterize_forward"][0] * 1e-3), 1)
    if "rasterize_backward" in kern:
        out["bwd_E_per_s"] = round(e_b / (kern["rasterize_backward"][0] * 1e-3), 1)
    return out


def stream_copy(mib=1024, reps=20):
    """STREAM Copy bandwidth on this GPU: the library's float4 copy kernel
    (mg_stream_copy) over `mib` MiB, timed with HIP events on its stream;
    bytes moved = read + write."""
    import torch

    from metal_gauss_amd import _lib

    lib = _lib.load()
    n = mib * (1 << 20)
    src = torch.ones(n // 4, device="cuda")
    dst = torch.empty_like(src)
    s = _lib.stream(src)
    for _ in range(3):
        _lib.check(lib.mg_stream_copy(src.data_ptr(), dst.data_ptr(), n, s))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        _lib.check(lib.mg_stream_copy(src.data_ptr(), dst.data_ptr(), n, s))
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    assert bool((dst == 1.0).all())
    del src, dst
    return {"GBps": round(2 * n / (ms * 1e-3) / 1e9, 1), "bytes_per_copy": 2 * n,
            "kernel": "stream_copy_kernel (mg_stream_copy, float4)"}


def mcmc_bench(args):
    """MCMC densification at config 4: the 1M-Gaussian parameter dict with
    FusedAdam state, as the reference's trainer holds it between steps.

    add_noise runs every step in the reference's trainer (train.py:417);
    relocate and grow every 100 steps (train.py:450-457). relocate is timed
    with a stated 5% of rows made dead (logit -8, a seeded choice) before each
    call; grow from 900k to 1M active rows. Wall times include the one host
    sync each of relocate and grow makes; kernel times are HIP events.
    """
    import torch

    from metal_gauss_amd import _lib, mcmc

    dev = torch.device("cuda:0")
    step = Step(args.gaussians, dev)
    step()                                  # optimizer state exists
    torch.cuda.synchronize()
    p = {k: v for k, v in step.p.items()}
    N = args.gaussians
    g = torch.Generator().manual_seed(7)
    dead = torch.randperm(N, generator=g)[: N // 20].to(dev)
    keep_logit = p["logit_opac"].detach().clone()
    out = {}

    def timed(fn, reps, label, prep=None):
        walls = []
        with _lib.KernelTimer():
            for r in range(reps):
                if prep is not None:
                    prep()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                walls.append(time.perf_counter() - t0)
            kern = {}
            for k in label:
                tot, cnt = _lib.KernelTimer.query(k)
                if cnt:
                    kern[k] = round(tot / cnt, 4)
        walls.sort()
        return round(1e3 * walls[len(walls) // 2], 4), kern

    with torch.no_grad():
        for _ in range(10):
            mcmc.add_noise(p, lr_means=1.6e-4)
        wall, kern = timed(lambda: mcmc.add_noise(p, lr_means=1.6e-4), 100, ["add_noise"])
        out["add_noise"] = {"wall_ms": wall, "kernel_ms": kern.get("add_noise"),
                            "GBps": round(56 * N / (kern["add_noise"] * 1e-3) / 1e9, 1)}

        def kill():
            p["logit_opac"].copy_(keep_logit)
            p["logit_opac"][dead] = -8.0

        moved = []
        wall, kern = timed(lambda: moved.append(mcmc.relocate(p, opt=step.opt)), 10,
                           ["mcmc_weights", "mcmc_apply"], prep=kill)
        out["relocate"] = {"wall_ms": wall, "kernel_ms": kern, "moved": moved[-1],
                           "dead_fraction": 0.05}
        p["logit_opac"].copy_(keep_logit)
        wall, kern = timed(lambda: mcmc.grow(p, target=N, active=N - N // 10, opt=step.opt), 10,
                           ["mcmc_weights", "mcmc_apply"])
        out["grow"] = {"wall_ms": wall, "kernel_ms": kern, "added": N // 10}
    return out


def _timed_ms(fn, reps, warm=3):
    """Median wall ms of `reps` synchronised calls after `warm` untimed ones."""
    import torch

    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return 1e3 * ts[len(ts) // 2]


def _kernel_means(fn, reps, labels):
    """Mean ms per launch of each library kernel over `reps` calls of fn."""
    import torch

    from metal_gauss_amd import _lib

    with _lib.KernelTimer():
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        out = {}
        for k in labels:
            tot, cnt = _lib.KernelTimer.query(k)
            if cnt:
                out[k] = {"ms": round(tot / cnt, 4), "per_call": cnt / reps}
    return out


def render_config(which, reps, crowded=False, chunked=False):
    """Configs 1, 2 and 5 ([1], [4]): one view, render
    forward (config 1) or forward + L1 loss + backward (2, 5), on the
    configuration's seeded scene and camera (config 5 ``crowded``: the
    variant that reaches the configuration's stated stress). As in the
    config-4 step, exp and sigmoid of the log-scales and opacity logits run
    inside the projection kernels (render(activations=True)) and the tile
    lists are capacity-sized (a ListCapacity, no host read inside the call;
    a call whose lists overflowed runs again and is counted). The same
    calls with the lists sized by the host read, the reference's way, are
    timed beside them."""
    import torch

    from metal_gauss_amd import ListCapacity, render, scenes

    dev = torch.device("cuda:0")
    if which == 1:
        sc, cam, bg = scenes.config1()
        target = None
    elif which == 2:
        sc, cam, bg = scenes.config2()
        target = scenes.config2_target(cam.H, cam.W).to(dev)
    else:
        sc, cam, bg = scenes.config5_crowded() if crowded else scenes.config5()
        target = torch.zeros(cam.H, cam.W, 3, device=dev)
    sc = sc.to(dev)
    leaves = {k: getattr(sc, k).clone().requires_grad_(which != 1)
              for k in ("means", "log_scales", "quats", "logit_opac", "sh_dc", "sh_rest")}
    info = {}
    cap = ListCapacity()
    reruns = [0]

    def fwd(sized):
        L = leaves
        rgb, alpha, inf = render(L["means"], L["quats"], L["log_scales"], L["logit_opac"],
                                 L["sh_dc"], cam.K, cam.viewmat, cam.W, cam.H,
                                 sh_degree=sc.sh_degree, sh_rest=L["sh_rest"], background=bg,
                                 chunked_backward=chunked, activations=True,
                                 list_capacity=cap if sized else None)
        info.update(inf)
        return rgb

    def overflowed(sized):
        # Polled once the whole call is enqueued, so the GPU is not left idle.
        if sized and cap.overflowed(info["lists_ticket"]):
            reruns[0] += 1
            return True
        return False

    def fwd_only(sized=True):
        while True:
            fwd(sized)
            if not overflowed(sized):
                return

    def fwd_bwd(sized=True):
        while True:
            for t in leaves.values():
                t.grad = None
            torch.nn.functional.l1_loss(fwd(sized), target).backward()
            if not overflowed(sized):
                return

    with torch.no_grad():
        fwd_only()                        # sizes the lists
        reruns[0] = 0
        fwd_ms = _timed_ms(fwd_only, reps)
        fwd_ms_host = _timed_ms(lambda: fwd_only(False), reps)
    out = {"fwd_ms": round(fwd_ms, 4), "fwd_ms_host_read_lists": round(fwd_ms_host, 4)}
    step = fwd_only if which == 1 else fwd_bwd
    if which != 1:
        out["fwd_bwd_ms"] = round(_timed_ms(fwd_bwd, reps), 4)
        out["fwd_bwd_ms_host_read_lists"] = round(_timed_ms(lambda: fwd_bwd(False), reps), 4)
    out["reruns_after_sizing"] = reruns[0]
    out["kernels"] = _kernel_means(step, 5, KERNELS)
    gids_len = None
    with torch.no_grad():
        from metal_gauss_amd.backend import _PreprocessMetal, _camera, build_tile_lists_metal

        fx, fy, cx, cy, vm_h, cc = _camera(cam.K, cam.viewmat)
        m, q, s_, o, sh = sc.activated()
        uv, conic, depth, rxy, valid, _ = _PreprocessMetal.apply(
            m, q, s_, sh, None, o, vm_h, fx, fy, cx, cy, cam.W, cam.H, 0.01, 100.0, 0.3,
            float(max(cam.W, cam.H)), cc, sc.sh_degree)
        gids, offs, _ = build_tile_lists_metal(uv, rxy, depth, valid, conic, o, cam.W, cam.H, 16)
        lens = (offs[1:] - offs[:-1]).cpu()
        gids_len = int(gids.numel())
    out.update({"intersections": gids_len, "max_tile_list": int(lens.max()),
                "mean_tile_list": round(float(lens.float().mean()), 1),
                "tiles_over_10k": int((lens > 10_000).sum()),
                "valid": int(valid.sum()), "n_gaussians": sc.n,
                "width": cam.W, "height": cam.H})
    return out


def ply_bench(n=1_000_000):
    """PLY I/O at config-4 size: export_ply of the trainer's parameters from the
    GPU (one encode kernel, one copy to the host, one file write), load_ply to
    the GPU (file read, one upload, one decode kernel) and to the CPU (numpy).
    Files go to a temporary directory (page cache warm after the write)."""
    import tempfile

    import torch

    from metal_gauss_amd import _lib, scenes
    from metal_gauss_amd.io import export_ply, load_ply

    dev = torch.device("cuda:0")
    sc = scenes.config4(n)[0].to(dev)
    p = {k: getattr(sc, k) for k in ("means", "log_scales", "quats", "logit_opac", "sh_dc",
                                     "sh_rest")}
    out = {}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "scene.ply")
        out["export_ms"] = round(_timed_ms(lambda: export_ply(p, path), 5, warm=1), 2)
        size = os.path.getsize(path)
        out["file_MB"] = round(size / 1e6, 1)
        out["load_gpu_ms"] = round(_timed_ms(lambda: load_ply(path, device="cuda"), 5, warm=1), 2)
        out["load_cpu_ms"] = round(_timed_ms(lambda: load_ply(path), 3, warm=1), 2)
        k = _kernel_means(lambda: (export_ply(p, path), load_ply(path, device="cuda")), 3,
                          ["ply_encode", "ply_decode"])
        out["kernels"] = k
        for name in ("ply_encode", "ply_decode"):
            if name in k:
                out[name + "_GBps"] = round(2 * size / (k[name]["ms"] * 1e-3) / 1e9, 1)
    return out


# The reference's published forward-only rates on an Apple M5 (README.md:145-148,
# bench/results/render_fps.json): (splats, resolution) -> frames per second.
REF_FPS = {(100_000, 256): 508.2, (100_000, 384): 481.3, (100_000, 512): 377.0,
           (100_000, 768): 256.5, (600_000, 512): 91.0, (600_000, 768): 69.0}


def render_fps(ramp_s=1.0, k=21):
    """Forward-only render rate, timed like bench/render_fps.py:30-44: a ramp
    of continuous frames, then the median of k synchronised frames (trimmed),
    with a constant black background and no autograd."""
    import torch

    from metal_gauss_amd import ListCapacity, render, scenes

    dev = torch.device("cuda:0")
    rows = []
    for n in (100_000, 300_000, 600_000):
        sc = scenes.fps_scene(n).to(dev)
        m, q, sca, op, sh = sc.activated()
        for res in (256, 384, 512, 768):
            K = scenes.intrinsics(res, res, 45.0)
            vm = torch.eye(4)

            def frame(cap=None):
                return render(m, q, sca, op, sh, K, vm, res, res, sh_degree=3,
                              list_capacity=cap)

            with torch.no_grad():
                end = time.perf_counter() + ramp_s
                while time.perf_counter() < end:
                    frame()
                torch.cuda.synchronize()
                ts = []
                for _ in range(k):
                    t0 = time.perf_counter()
                    _, _, info = frame()
                    torch.cuda.synchronize()
                    ts.append(time.perf_counter() - t0)
                # Frames enqueued back to back with capacity-sized lists (no
                # host read in a frame; each frame's overflow word checked
                # one frame later).
                cap = ListCapacity()
                while True:
                    _, _, ci = frame(cap)
                    if not cap.overflowed(ci["lists_ticket"]):
                        break
                nf = 4 * k
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                prev = None
                for _ in range(nf):
                    _, _, ci = frame(cap)
                    t = ci["lists_ticket"]
                    if prev is not None and cap.overflowed(prev):
                        raise RuntimeError("a frame overflowed its sized lists")
                    prev = t
                torch.cuda.synchronize()
                pipe = (time.perf_counter() - t0) * 1e3 / nf
            ts.sort()
            ms = 1e3 * float(sum(ts[1:-1]) / len(ts[1:-1])) if k > 2 else 1e3 * ts[0]
            med = 1e3 * ts[len(ts) // 2]
            row = {"splats": n, "res": res, "ms": round(med, 4), "fps": round(1e3 / med, 1),
                   "trimmed_mean_ms": round(ms, 4), "intersections": info["isect_total"],
                   "pipelined_ms": round(pipe, 4), "pipelined_fps": round(1e3 / pipe, 1)}
            if (n, res) in REF_FPS:
                row["reference_m5_fps"] = REF_FPS[(n, res)]
            rows.append(row)
    return rows


def adam_config(reps):
    """Config 3: 1M Gaussians x 59 floats in the six
    trainer groups, gradients N(0, 1e-3); FusedAdam one step then 100 steps,
    and SelectiveAdam with a Bernoulli(0.6) visibility mask."""
    import torch

    from metal_gauss_amd import FusedAdam, SelectiveAdam, scenes

    dev = torch.device("cuda:0")
    N = 1_000_000
    g = torch.Generator().manual_seed(2)
    groups = scenes.config3_groups(N)
    params = [torch.randn(N, w, generator=g).to(dev).requires_grad_(True) for _, w, _ in groups]
    grads = [(torch.randn(N, w, generator=g) * 1e-3).to(dev) for _, w, _ in groups]
    vis = (torch.rand(N, generator=g) < 0.6).to(dev)
    n_floats = sum(p.numel() for p in params)

    def run(opt_cls, selective):
        ps = [p.detach().clone().requires_grad_(True) for p in params]
        opt = opt_cls([{"params": [p], "lr": lr} for p, (_, _, lr) in zip(ps, groups)],
                      eps=1e-15)
        for p, gr in zip(ps, grads):
            p.grad = gr
        stepf = (lambda: opt.step(vis)) if selective else opt.step
        first = _timed_ms(stepf, 1, warm=0)
        ms = _timed_ms(stepf, 100, warm=3)
        label = "selective_adam_step" if selective else "adam_step"
        kern = _kernel_means(stepf, 50, [label])[label]["ms"]
        return first, ms, kern

    f_first, f_ms, f_kern = run(FusedAdam, False)
    s_first, s_ms, s_kern = run(SelectiveAdam, True)
    f_vis = float(vis.float().mean())
    fused_bytes = 28 * n_floats
    sel_bytes = (28 * n_floats + 4 * 2 * 6 * N) * f_vis + N      # + per-row steps r/w, mask
    # GBps: algorithmic bytes over the kernel's own time (HIP events around
    # the launch); ms_per_step is the synchronised wall time of step().
    return {"fused": {"first_step_ms": round(f_first, 4), "ms_per_step": round(f_ms, 4),
                      "kernel_ms": round(f_kern, 4),
                      "GBps": round(fused_bytes / (f_kern * 1e-3) / 1e9, 1)},
            "selective": {"first_step_ms": round(s_first, 4), "ms_per_step": round(s_ms, 4),
                          "kernel_ms": round(s_kern, 4), "visible_fraction": round(f_vis, 4),
                          "GBps": round(sel_bytes / (s_kern * 1e-3) / 1e9, 1)},
            "n_floats": n_floats}


def _counter_rows(d):
    import csv

    files = sorted(Path(d).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def _per_kernel(rows):
    acc = {}
    for r in rows:
        acc.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return acc


def pmc_summary(fetch_dir, write_dir, copy_mib):
    """Text summary of HBM traffic per launch from two rocprofv3 --pmc runs.

    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are each scaled by what they
    read for the run's own plain copy of copy_mib MiB (its largest
    __amd_rocclr_copyBuffer dispatch), which reads and writes exactly that
    many bytes.
    """
    fetch = _per_kernel(_counter_rows(fetch_dir))
    write = _per_kernel(_counter_rows(write_dir))
    nbytes = copy_mib * (1 << 20)
    cf = nbytes / (max(fetch["__amd_rocclr_copyBuffer"]) * 1024)
    cw = nbytes / (max(write["__amd_rocclr_copyBuffer"]) * 1024)
    lines = [
        "# HBM traffic per launch, config-4 step (1M Gaussians SH3, 800x800, tile 16), MI355X",
        "# made by (from the repository root, TMPDIR=/tmp):",
        f"#   rocprofv3 --pmc FETCH_SIZE --kernel-include-regex '{COUNTER_REGEX}' -f csv -T "
        "-d F -o pmc -- python3 -u bench.py --steps 3 --warmup 2 --no-cpu-baseline --ramp 0 "
        f"--copy-mib {copy_mib}",
        "#   (the same with --pmc WRITE_SIZE -d W)",
        f"#   python bench.py --pmc-summary F W --copy-mib {copy_mib}",
        f"# calibration: a {copy_mib} MiB device copy reads FETCH_SIZE "
        f"{max(fetch['__amd_rocclr_copyBuffer']):.0f} KiB (factor {cf:.3f}) and WRITE_SIZE "
        f"{max(write['__amd_rocclr_copyBuffer']):.0f} KiB (factor {cw:.3f})",
        "# traffic_bytes = factor_f * FETCH_SIZE + factor_w * WRITE_SIZE, mean per dispatch",
        f"{'kernel':28s} {'dispatches':>10s} {'FETCH_KiB':>12s} {'WRITE_KiB':>12s} "
        f"{'read_MB':>9s} {'write_MB':>9s} {'traffic_bytes':>14s}",
    ]
    for name in sorted(fetch):
        if name == "__amd_rocclr_copyBuffer" or name not in write:
            continue
        fk = sum(fetch[name]) / len(fetch[name])
        wk = sum(write[name]) / len(write[name])
        rd, wr = cf * fk * 1024, cw * wk * 1024
        lines.append(f"{name:28s} {len(fetch[name]):10d} {fk:12.1f} {wk:12.1f} "
                     f"{rd / 1e6:9.2f} {wr / 1e6:9.2f} {int(rd + wr):14d}")
    return "\n".join(lines)


COUNTER_REGEX = ("raster_bwd|raster_fwd|tile_order|adam_multi|preprocess_fwd|preprocess_bwd|"
                 "scan_|bin_write|bin_count|bin_offsets|count_hist|count_colscan|count_scatter|"
                 "tile_depth_sort|radix_|tile_ranges|ssim_fused|photometric_loss|stream_copy|"
                 "copyBuffer|block_order|tile_len_order")


def _kernel_base(name):
    """'void mg::raster_bwd_kernel<4, false, true>(mg::RasterArgs, ...)' ->
    'raster_bwd_kernel'."""
    n = name.split("(")[0].replace("void ", "").strip()
    n = n.split("<")[0]
    return n.split("::")[-1]


def counter_summary(dirs, copy_mib=1024, config=None, crowded=False):
    """Per-kernel table from rocprofv3 runs of the config-4 step (or, with
    config 5, its fwd + bwd, crowded or not): one
    --kernel-trace --stats run (kernel_stats.csv) and --pmc passes (one
    *counter_collection.csv each). Counters are averaged over a kernel's
    dispatches; FETCH_SIZE and WRITE_SIZE are calibrated by the run's own
    copy of copy_mib MiB (__amd_rocclr_copyBuffer) when it is there."""
    import csv

    dur, vgpr, lds = {}, {}, {}
    cnt = {}
    for d in dirs:
        for f in sorted(Path(d).rglob("*kernel_stats.csv")):
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    dur[_kernel_base(r["Name"])] = float(r["AverageNs"])
        for f in sorted(Path(d).rglob("*counter_collection.csv")):
            with open(f, newline="") as fh:
                for r in csv.DictReader(fh):
                    k = _kernel_base(r["Kernel_Name"])
                    cnt.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(
                        float(r["Counter_Value"]))
                    vgpr[k] = r.get("VGPR_Count", "")
                    lds[k] = r.get("LDS_Block_Size", "")
    mean = {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in cnt.items()}
    nbytes = copy_mib * (1 << 20)
    cp = mean.get("__amd_rocclr_copyBuffer", {})
    cf = nbytes / (max(cnt["__amd_rocclr_copyBuffer"]["FETCH_SIZE"]) * 1024) \
        if "FETCH_SIZE" in cp else None
    cw = nbytes / (max(cnt["__amd_rocclr_copyBuffer"]["WRITE_SIZE"]) * 1024) \
        if "WRITE_SIZE" in cp else None
    head = (f"{'kernel':26s} {'avg_us':>7s} {'VGPR':>4s} {'LDS_B':>6s} {'occ_w/CU':>8s} "
            f"{'VALUbusy%':>9s} {'VALU_Minst':>10s} {'VALU_G/s':>9s} {'LDS_Minst':>9s} "
            f"{'bankconf%':>9s} {'wait%':>6s} {'atomics_M':>9s} {'HBM_rd_MB':>9s} "
            f"{'HBM_wr_MB':>9s} {'HBM_GB/s':>8s}")
    lines = [head]

    def g(k, c):
        return mean.get(k, {}).get(c)

    order = sorted((k for k in mean if k != "__amd_rocclr_copyBuffer"),
                   key=lambda k: -dur.get(k, 0.0))
    for k in order:
        t = dur.get(k)
        vi = g(k, "SQ_INSTS_VALU")
        li = g(k, "SQ_INSTS_LDS")
        bc, al = g(k, "SQ_LDS_BANK_CONFLICT"), g(k, "SQ_ACTIVE_INST_LDS")
        wa, wc = g(k, "SQ_WAIT_INST_ANY"), g(k, "SQ_WAVE_CYCLES")
        at = sum(x for x in (g(k, "TCP_TCC_ATOMIC_WITH_RET_REQ_sum"),
                             g(k, "TCP_TCC_ATOMIC_WITHOUT_RET_REQ_sum")) if x is not None)
        rd = cf * g(k, "FETCH_SIZE") * 1024 if cf and g(k, "FETCH_SIZE") is not None else None
        wr = cw * g(k, "WRITE_SIZE") * 1024 if cw and g(k, "WRITE_SIZE") is not None else None

        def fmt(x, w, p=1, scale=1.0):
            return f"{x * scale:{w}.{p}f}" if x is not None else f"{'-':>{w}s}"
        vp = vi / (t * 1e-9) / 1e9 if vi and t else None
        bcp = 100 * bc / al if bc is not None and al else None
        wp = 100 * wa / wc if wa is not None and wc else None
        gbs = (rd + wr) / (t * 1e-9) / 1e9 if rd is not None and wr is not None and t else None
        lines.append(
            f"{k[:26]:26s} {fmt(t, 7, 1, 1e-3)} {str(vgpr.get(k, '')):>4s} "
            f"{str(lds.get(k, '')):>6s} {fmt(g(k, 'MeanOccupancyPerCU'), 8, 1)} "
            f"{fmt(g(k, 'VALUBusy'), 9, 1)} {fmt(vi, 10, 2, 1e-6)} {fmt(vp, 9, 1)} "
            f"{fmt(li, 9, 2, 1e-6)} {fmt(bcp, 9, 2)} {fmt(wp, 6, 1)} "
            f"{fmt(at if at else None, 9, 2, 1e-6)} {fmt(rd, 9, 1, 1e-6)} {fmt(wr, 9, 1, 1e-6)} "
            f"{fmt(gbs, 8, 0)}")
    if config == 5:
        what = ("config 5 crowded: forward + L1 + backward, 3.6M Gaussians SH3, 1920x1080, "
                "over 30M intersections" if crowded else
                "config 5: forward + L1 + backward, 3M Gaussians SH3, 1920x1080")
        bflag = "--config 5 --crowded --steps 3" if crowded else "--config 5 --steps 3"
        sflag = " --config 5 --crowded" if crowded else " --config 5"
    else:
        what = "config-4 step (1M Gaussians SH3, 800x800, tile 16)"
        bflag = "--steps 3 --warmup 2 --no-cpu-baseline --ramp 0"
        sflag = ""
    notes = [
        f"# Per-kernel counters, {what}, MI355X",
        f"# made by (from the repository root; TMPDIR=/tmp; B='bench.py {bflag}",
        "#   --copy-mib 1024'; R = the --kernel-include-regex",
        f"#   '{COUNTER_REGEX}'):",
        "#   rocprofv3 --kernel-trace --stats -f csv -T -d KT -o kt -- python3 -u $B",
        "#   rocprofv3 --pmc <pass> --kernel-include-regex $R -f csv -T -d P<i> -o pmc -- "
        "python3 -u $B",
        "#   for the passes: P1 'SQ_WAVES SQ_INSTS_VALU SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT",
        "#   SQ_ACTIVE_INST_LDS SQ_WAIT_INST_ANY SQ_WAVE_CYCLES GRBM_GUI_ACTIVE', P2 VALUBusy,",
        "#   P3 MeanOccupancyPerCU, P4 'TCP_TCC_ATOMIC_WITH_RET_REQ_sum",
        "#   TCP_TCC_ATOMIC_WITHOUT_RET_REQ_sum', P5 FETCH_SIZE, P6 WRITE_SIZE; then",
        f"#   python bench.py --counter-summary KT P1 P2 P3 P4 P5 P6 --copy-mib 1024{sflag}",
        "# columns: avg_us from the kernel trace; VGPR and LDS bytes per workgroup as",
        "#   rocprofv3 reports them; occ_w/CU = MeanOccupancyPerCU (waves resident per CU);",
        "#   VALUbusy% = VALUBusy; VALU_Minst = SQ_INSTS_VALU (wave instructions) per",
        "#   dispatch; VALU_G/s = SQ_INSTS_VALU / avg time (wave instructions per second);",
        "#   LDS_Minst = SQ_INSTS_LDS; bankconf% = SQ_LDS_BANK_CONFLICT / SQ_ACTIVE_INST_LDS;",
        "#   wait% = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES; atomics_M = TCP->TCC atomic requests",
        "#   (with + without return); HBM rd/wr = FETCH_SIZE, WRITE_SIZE calibrated by a",
        f"#   {copy_mib} MiB device copy (factors "
        f"{'-' if cf is None else f'{cf:.3f}'} / {'-' if cw is None else f'{cw:.3f}'}).",
    ]
    return "\n".join(notes + lines)


def stats_summary(stats_csv, steps, variant="base", mcmc=False, config=None, render_fps=False,
                  crowded=False):
    """Text summary of a rocprofv3 --kernel-trace --stats kernel_stats.csv."""
    import csv

    with open(stats_csv, newline="") as f:
        rows = list(csv.DictReader(f))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    if config is not None:
        what = {1: "config 1: forward, 10k Gaussians SH0, 256x256",
                2: "config 2: forward + L1 + backward, 300k Gaussians SH3, 800x800",
                3: "config 3: FusedAdam and SelectiveAdam over 1M Gaussians x 59 floats",
                5: "config 5: forward + L1 + backward, 3M Gaussians SH3, 1920x1080"}[config]
        cflag = f"--config {config}"
        if crowded:
            what = ("config 5 crowded: forward + L1 + backward, 3.6M Gaussians SH3, 1920x1080, "
                    "over 30M intersections")
            cflag += " --crowded"
        lines = [
            f"# rocprofv3 kernel statistics, {what}, MI355X",
            "# made by (from the repository root, TMPDIR=/tmp):",
            "#   rocprofv3 --kernel-trace --stats -f csv -T -d P -o kt -- python -u bench.py "
            f"{cflag} --steps {steps}",
            f"#   python bench.py --stats-summary P/kt_kernel_stats.csv {cflag}",
        ]
    elif render_fps:
        lines = [
            "# rocprofv3 kernel statistics, forward-only render sweep (100k/300k/600k Gaussians "
            "SH3 x 256..768^2, fixed view), MI355X",
            "# made by (from the repository root, TMPDIR=/tmp):",
            "#   rocprofv3 --kernel-trace --stats -f csv -T -d P -o kt -- python -u bench.py "
            "--render-fps",
            "#   python bench.py --stats-summary P/kt_kernel_stats.csv --render-fps",
        ]
    elif mcmc:
        lines = [
            "# rocprofv3 kernel statistics, MCMC densification on the config-4 parameters "
            "(1M Gaussians, 59 floats each, FusedAdam state), MI355X",
            "# made by (from the repository root, TMPDIR=/tmp):",
            "#   rocprofv3 --kernel-trace --stats -f csv -T -d P -o kt -- python -u bench.py "
            "--mcmc",
            "#   python bench.py --stats-summary P/kt_kernel_stats.csv --mcmc",
            "# The run covers one config-4 step (to create optimizer state), 110 add_noise "
            "calls, 10 relocates (5% dead rows) and 10 grows (900k -> 1M).",
        ]
    else:
        vflag = "" if variant == "base" else f" --variant {variant}"
        what = {"base": "", "unfused-adam": ", FusedAdam.step() after the backward",
                "torch-act": ", exp/sigmoid of the parameters in torch",
                "mip": ", Mip 3D filter + 2D antialias in the projection kernel",
                "mip-torch": ", Mip 3D filter as torch reparameterisation"}[variant]
        lines = [
            "# rocprofv3 kernel statistics, config-4 step (1M Gaussians SH3, 800x800, tile 16"
            f"{what}), MI355X",
            "# made by (from the repository root, TMPDIR=/tmp):",
            "#   rocprofv3 --kernel-trace --stats -f csv -T -d P -o kt -- python -u bench.py "
            f"--steps {steps} --warmup 5 --ramp 0.5 --no-cpu-baseline{vflag}",
            f"#   python bench.py --stats-summary P/kt_kernel_stats.csv{vflag}",
            "# The run covers a 0.5 s ramp of fwd+bwd steps, warmup + timed steps, the same "
            "steps with host-read list sizing, the fwd+bwd-only loop, 10 per-kernel timing "
            "steps and the forward-only frames.",
        ]
    lines += [
        f"{'kernel':36s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'share_%':>8s}",
    ]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        lines.append(f"{r['Name'][:36]:36s} {int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.1f} "
                     f"{float(r['MinNs']) / 1e3:9.1f} {float(r['MaxNs']) / 1e3:9.1f} "
                     f"{100 * float(r['TotalDurationNs']) / total:8.2f}")
    return "\n".join(lines)


# Issue rate of non-packed 32-bit VALU wave64 instructions: 256 CUs x 4
# SIMDs, one instruction every 4 clocks (16 lanes wide) at 2.4 GHz. The
# published 157.3 TFLOP/s vector FP32 peak counts packed FP32 (two lanes'
# worth per instruction), which this build does not emit.
VALU_PEAK_GIPS = 256 * 4 * 2.4 / 4
COUNTERS_FILE = ROOT / "profiles" / "counters_config4.txt"


def committed_valu(label):
    """SQ_INSTS_VALU (wave instructions) per launch of a kernel from the
    committed counter summary, or None."""
    name = PROF_NAMES.get(label)
    if name is None or not COUNTERS_FILE.exists():
        return None
    lines = COUNTERS_FILE.read_text().splitlines()
    head = next((ln.split() for ln in lines if ln.startswith("kernel ")), None)
    if head is None or "VALU_Minst" not in head:
        return None
    col = head.index("VALU_Minst")
    for ln in lines:
        parts = ln.split()
        if parts and parts[0] == name and not ln.startswith("#"):
            try:
                return float(parts[col]) * 1e6
            except (IndexError, ValueError):
                return None
    return None


def committed_traffic(label):
    """HBM bytes per launch of a kernel from the committed PMC summary, or None."""
    name = PROF_NAMES.get(label)
    if name is None or not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        parts = line.split()
        if parts and parts[0] == name and not line.startswith("#"):
            return int(parts[-1])
    return None


def cpu_baseline(n_gaussians=1_000_000, crop=800, k=3):
    """The CPU oracle on one config-4 step.

    The full config-4 scene (all N Gaussians projected, SH evaluated, and
    differentiated), rasterised forward+backward over a crop x crop window at
    the image centre (by default the whole 800x800 view, so nothing is
    extrapolated), the loss on it, and torch.optim.Adam over all 59N
    parameters; reported as steps/s. With a smaller crop, whose centre is
    denser than the frame, the crop's time is scaled by the ratio of the
    oracle's own intersection counts (3-sigma boxes at tile 16,
    render_ref.tile_lists) over the full view and over the crop. The
    projection is run once untimed first (allocator and thread-pool warm-up);
    each part is then timed k times and its median taken. The whole view
    needs about 40 GB of host memory.
    """
    import torch

    from metal_gauss_amd import scenes
    from oracle import render_ref as R
    from oracle import ssim_ref

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    sc, cams, _ = scenes.config4(n_gaussians)
    cam = cams[0]
    W = H = 800
    x0 = y0 = (W - crop) // 2
    K = cam.K.clone()
    K[0, 2] -= x0
    K[1, 2] -= y0
    leaves = {k: getattr(sc, k).clone().requires_grad_(True)
              for k in ("means", "log_scales", "quats", "logit_opac", "sh_dc", "sh_rest")}
    gt = scenes.config4_target(0)[y0:y0 + crop, x0:x0 + crop].contiguous()
    vm = cam.viewmat
    fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])

    def project_part():
        scales = torch.exp(leaves["log_scales"])
        op = torch.sigmoid(leaves["logit_opac"])
        sh = torch.cat([leaves["sh_dc"], leaves["sh_rest"]], dim=1)
        cov = R.build_cov3d(leaves["quats"], scales)
        uv, conic, depth, radius, valid, _ = R.project(leaves["means"], cov, vm, fx, fy, cx, cy,
                                                       crop, crop, 0.01, 100.0,
                                                       max_radius_frac=W / crop)
        cc = -vm[:3, :3].T @ vm[:3, 3]
        d = leaves["means"] - cc
        d = d / d.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        col = (R.eval_sh(3, sh, d) + 0.5).clamp_min(0.0)
        return uv, conic, op, col, depth, radius, valid

    def isect_count(Kc, w, h):
        with torch.no_grad():
            cov = R.build_cov3d(leaves["quats"], torch.exp(leaves["log_scales"]))
            uvc, _, dc, rc, vc, _ = R.project(leaves["means"], cov, vm, float(Kc[0, 0]),
                                              float(Kc[1, 1]), float(Kc[0, 2]), float(Kc[1, 2]),
                                              w, h, 0.01, 100.0, max_radius_frac=W / w)
            return R.tile_lists(uvc, rc, vc, dc, w, h, 16)[3]

    def median(xs):
        return sorted(xs)[len(xs) // 2]

    # Projection of all N (forward + backward through a dummy reduction of the
    # same outputs the rasteriser consumes); once untimed, then k timed runs.
    for t in (project_part(),):
        (t[0].sum() + t[1].sum() + t[3].sum() + t[2].sum()).backward()
    t_proj = []
    for _ in range(k):
        for t in leaves.values():
            t.grad = None
        t0 = time.perf_counter()
        uv, conic, op, col, depth, radius, valid = project_part()
        (uv.sum() + conic.sum() + col.sum() + op.sum()).backward()
        t_proj.append(time.perf_counter() - t0)
    for t in leaves.values():
        t.grad = None
    # Raster + loss on the crop (the projection repeated outside the timer).
    t_crop = []
    for _ in range(k):
        uv, conic, op, col, depth, radius, valid = project_part()
        t0 = time.perf_counter()
        rgb, alpha, info = R.rasterize(uv, conic, op, col, depth, radius, valid, crop, crop,
                                       tile=16, background=(0.0, 0.0, 0.0))
        loss = 0.8 * (rgb - gt).abs().mean() + 0.2 * (1.0 - ssim_ref.ssim(rgb, gt))
        loss.backward()
        t_crop.append(time.perf_counter() - t0)
        del rgb, alpha, loss
    # Adam over all parameters.
    opt = torch.optim.Adam(list(leaves.values()), lr=1e-3, eps=1e-15)
    t_adam = []
    for _ in range(k):
        for t in leaves.values():
            t.grad = torch.zeros_like(t)
        t0 = time.perf_counter()
        opt.step()
        t_adam.append(time.perf_counter() - t0)
    tp, tc, ta = median(t_proj), median(t_crop), median(t_adam)
    i_full = isect_count(cam.K, W, H) if crop < W else info["isect_total"]
    scale = i_full / max(1, info["isect_total"])
    t_step = tp + ta + tc * scale
    return {
        "value": round(1.0 / t_step, 6), "unit": "steps/s", "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config-4 step, CPU oracle (torch_ref restatement), median of {k} runs of "
                   f"each part: projection+SH fwd+bwd of all {n_gaussians} Gaussians {tp:.2f}s + "
                   f"Adam over all params {ta:.2f}s + raster/loss fwd+bwd on a {crop}x{crop} "
                   f"centre crop {tc:.2f}s x {scale:.2f} (oracle intersections, full view "
                   f"{i_full} / crop {info['isect_total']}); os.cpu_count()={cores}"),
    }


def _cpu_crop():
    """The whole view when the host has room for the oracle's slab tensors
    (about 40 GB), else a 384x384 centre crop scaled by intersections."""
    try:
        import psutil
        avail = psutil.virtual_memory().available
    except Exception:
        avail = 0
    return 800 if avail > 96 * (1 << 30) else 384


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported by this build "
              f"(the splatting step has no multi-GPU path here).", file=sys.stderr)
        sys.exit(2)
    if args.pmc_summary:
        print(pmc_summary(*args.pmc_summary, args.copy_mib or 1024))
        return
    if args.counter_summary:
        print(counter_summary(args.counter_summary, args.copy_mib or 1024, args.config,
                              args.crowded))
        return
    if args.stats_summary:
        print(stats_summary(args.stats_summary, args.steps if args.config else 20,
                            args.variant, args.mcmc, args.config, args.render_fps, args.crowded))
        return
    if args.cpu_only:
        print(json.dumps(cpu_baseline(args.gaussians, crop=_cpu_crop())))
        return
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(2)
    if args.copy_mib:
        copy_calibration(args.copy_mib)
    if args.ply:
        r = ply_bench(args.gaussians)
        print(json.dumps({"metric": "PLY export + load ms at 1M Gaussians SH3",
                          "value": round(r["export_ms"] + r["load_gpu_ms"], 2), "unit": "ms",
                          "n_gpus": 1, "higher_is_better": False, "dtype": "f32",
                          "data": "synthetic (config-4 parameters)",
                          "config": {"workload": "export_ply from the GPU, load_ply to the GPU "
                                                 "and to the CPU", "n_gaussians": args.gaussians},
                          "result": r}))
        return
    if args.render_fps:
        rows = render_fps()
        head = next(r for r in rows if r["splats"] == 600_000 and r["res"] == 768)
        print(json.dumps({"metric": "forward-only render frames/s (600k Gaussians SH3, 768^2)",
                          "value": head["fps"], "unit": "frames/s", "n_gpus": 1,
                          "higher_is_better": True, "dtype": "f32",
                          "data": "synthetic (seeded frustum scene; the reference renders a ply)",
                          "config": {"workload": "forward-only render, fixed view, fov 45 deg"},
                          "vs_reference_m5": round(head["fps"] / REF_FPS[(600_000, 768)], 2),
                          "pipelined_fps": head["pipelined_fps"],
                          "rows": rows}))
        return
    if args.config is not None:
        c = args.config
        if args.crowded and c != 5:
            print("--crowded applies to --config 5 only", file=sys.stderr)
            sys.exit(2)
        res = adam_config(args.steps) if c == 3 else render_config(
            c, min(args.steps, 50), args.crowded, args.chunked_backward == "on")
        metric = {1: "forward ms at 10k Gaussians 256x256 SH0",
                  2: "fwd+bwd ms at 300k Gaussians 800x800 SH3",
                  3: "Adam ms per step over 1M Gaussians x 59 floats",
                  5: "fwd+bwd ms at 3M Gaussians 1920x1080 SH3"}[c]
        if args.crowded:
            metric = "fwd+bwd ms at 3.6M Gaussians 1920x1080 SH3 (crowded: >30M intersections)"
        value = (res["fused"]["ms_per_step"] if c == 3 else
                 res["fwd_ms"] if c == 1 else res["fwd_bwd_ms"])
        print(json.dumps({"metric": metric, "value": value, "unit": "ms", "n_gpus": 1,
                          "higher_is_better": False, "dtype": "f32", "data": "synthetic",
                          "config": {"workload": f"BASELINE configs[{c - 1}] (config {c})"
                                                 + (", crowded variant" if args.crowded else ""),
                                     "chunked_backward": args.chunked_backward},
                          "result": res}))
        return
    if args.mcmc:
        print(json.dumps({
            "metric": "MCMC densification ms at 1M Gaussians (config-4 parameters + FusedAdam "
                      "state)",
            "unit": "ms", "n_gpus": 1, "higher_is_better": False, "dtype": "f32",
            "data": "synthetic",
            "config": {"workload": "config-4 parameter set, 59 floats per Gaussian, "
                                   "relocate with 5% dead rows, grow 900k -> 1M",
                       "n_gaussians": args.gaussians},
            "mcmc": mcmc_bench(args)}))
        return
    r = gpu_bench(args)
    out = {
        "metric": METRIC,
        "value": round(1000.0 / r["ms"], 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 4),
        "median_ms_per_step": round(r["median_ms"], 4),
        "ramp_s": args.ramp,
        "fwd_bwd_ms": round(r["fb_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": ("config 4: 1M Gaussians SH3, 800x800, 100 seeded views, "
                         "fwd + bwd + FusedAdam, loss 0.8 L1 + 0.2 (1-SSIM)"
                         + (" + 0.01 mean sigmoid(logit) + 0.01 mean exp(log scale)"
                            if args.reg else "")),
            "n_gaussians": args.gaussians, "width": 800, "height": 800, "sh_degree": 3,
            "tile": 16, "mean_intersections": int(r["I"]),
            "valid_fraction": round(r["f_valid"], 4),
        },
        "roofline": {
            "bound": "hbm", "kernel": r["dominant"], "achieved": round(r["achieved"], 2),
            "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(r["achieved"] / HBM_PEAK_GBS, 5),
            "traffic": committed_traffic(r["dominant"]),
            "algorithmic_bytes_per_launch": int(r["nbytes"]),
        },
        "roofline_valu": valu_roofline(r["kernels"]),
        "kernels": r["kernels"],
        "raster_work": r["work"],
        "stream_copy": r["copy"],
        "tile_lists": {
            "sizing": args.lists,
            "reruns_in_timed_steps": r["reruns"],
            "sync_lists_ms_per_step": None if r["sync_ms"] is None else round(r["sync_ms"], 4),
        },
        "forward_fps": r["fwd"],
    }
    if args.variant != "base":
        out["config"]["workload"] += {
            "unfused-adam": "; FusedAdam.step() after the backward, not in it",
            "torch-act": "; exp/sigmoid of the parameters in torch before render",
            "mip": "; Mip 3D filter + 2D antialias in the projection kernel",
            "mip-torch": "; Mip 3D filter as torch reparameterisation, 2D antialias in kernel",
        }[args.variant]
        out["config"]["variant"] = args.variant
    if args.variant in ("mip", "mip-torch"):
        # Once per densify interval in the reference's trainer, not per step:
        # the kernel alone, and with building the per-view table on the host.
        out["compute_3d_filter_ms"] = {"kernel": round(r["f3d_ms"][0], 4),
                                       "with_host_views": round(r["f3d_ms"][1], 3)}
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.gaussians, crop=_cpu_crop())
    print(json.dumps(out))


if __name__ == "__main__":
    main()
