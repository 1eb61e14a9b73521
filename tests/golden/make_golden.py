"""Golden fixtures for the splatting path, written from the CPU oracle.

    python tests/golden/make_golden.py        (from the repository root)

writes three small compressed .npz files beside this script:

config1.npz
    BASELINE configs[0] in full: 10,000 Gaussians (seed 0), SH degree 0,
    256x256, fov 40 degrees, tile 16, black background. It holds the
    activated inputs and the camera. It holds the float32 preprocess contract
    (uv, conic, depth, rxy, valid, colour; preprocess.metal:114-221). It holds
    the exact tile lists that the binning oracle builds from those outputs
    (metal_backend.py:217-285, binning.metal:25-90). It holds the float64
    image and alpha with every listed Gaussian composited (torch_ref.py:298-337).
    It also holds the pixels that are ill-conditioned at float32, as flagged
    by the C raster contract (oracle/raster_seq.c): some alpha lies within a
    relative 1e-5 of the 1/255 cutoff, so one ulp of exp flips whether that
    Gaussian is composited.
fwd_bwd_small.npz
    A 300-Gaussian SH-3 scene at 64x48 in the style of tests/test_metal.py.
    Its loss is sum(w_rgb * rgb) + sum(w_alpha * alpha) with seeded weights.
    The file holds the float64 image, alpha and every parameter gradient.
adam_small.npz
    FusedAdam (adam.metal:34-41 with rasterize.mm:338-342) over 20 steps on
    1,024 floats, for eps 1e-15 and 1e-8. Then SelectiveAdam
    (selective_adam.py:116-187) over 20 steps on 256 rows of width 3, with
    Bernoulli(0.6) visibility.

The oracle that writes these is pinned separately, by known answers,
gradcheck, brute force and closed forms. The fixtures freeze its outputs, so
the GPU tests can compare against data, and so a later change to the oracle
cannot pass unnoticed. Nothing here reads or runs the reference.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import adam_ref, binning_ref, raster_ref, render_ref  # noqa: E402


def _f32(t):
    return t.detach().cpu().to(torch.float32).numpy()


def config1_case() -> dict:
    from metal_gauss_amd import scenes

    sc, cam, bg = scenes.config1()
    means, quats, scales, op, sh = sc.activated()
    K, vm, W, H = cam.K, cam.viewmat, cam.W, cam.H
    fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])
    with torch.no_grad():
        uv, conic, depth, rxy, valid, color = render_ref.preprocess(
            means, quats, scales, op, sh[:, :1], vm, fx, fy, cx, cy, W, H, sh_degree=0)
        rgb, alpha, _ = render_ref.render(
            means.double(), quats.double(), scales.double(), op.double(), sh[:, :1].double(),
            K.double(), vm.double(), W, H, sh_degree=0, tile=16, min_transmittance=0.0,
            background=bg)
    ids, offsets, _, _ = binning_ref.build_tile_lists(
        _f32(uv), _f32(rxy), _f32(conic), _f32(op), valid.numpy(), _f32(depth), W, H, 16)
    amb = raster_ref.forward(_f32(uv), _f32(conic), _f32(op), _f32(color), ids, offsets, W, H, 16,
                             t_min=0.0)[4]
    return dict(
        means=_f32(means), quats=_f32(quats), scales=_f32(scales), opacities=_f32(op),
        sh_dc=_f32(sh[:, :1]), K=_f32(K), viewmat=_f32(vm), W=np.int32(W), H=np.int32(H),
        uv=_f32(uv), conic=_f32(conic), depth=_f32(depth), rxy=_f32(rxy),
        valid=valid.numpy().astype(np.uint8), color=_f32(color),
        gauss_ids=ids.astype(np.int32), tile_offsets=offsets.astype(np.int32),
        rgb=_f32(rgb), alpha=_f32(alpha), ambiguous=amb.astype(np.uint8))


def fwd_bwd_case() -> dict:
    n, W, H = 300, 64, 48
    g = torch.Generator().manual_seed(20)
    means = torch.randn(n, 3, generator=g) * 0.6 + torch.tensor([0.0, 0.0, 4.0])
    quats = torch.randn(n, 4, generator=g)
    scales = torch.rand(n, 3, generator=g) * 0.10 + 0.03
    op = torch.rand(n, generator=g) * 0.7 + 0.15
    sh = torch.randn(n, 16, 3, generator=g) * 0.25
    w_rgb = torch.rand(H, W, 3, generator=g)
    w_alpha = torch.rand(H, W, generator=g)
    f = 0.8 * max(W, H)
    K = torch.tensor([[f, 0.0, W / 2], [0.0, f, H / 2], [0.0, 0.0, 1.0]])
    vm = torch.eye(4)
    leaves = [t.double().requires_grad_(True) for t in (means, quats, scales, op, sh)]
    rgb, alpha, _ = render_ref.render(*leaves, K.double(), vm.double(), W, H, sh_degree=3,
                                      tile=16, min_transmittance=0.0)
    ((rgb * w_rgb.double()).sum() + (alpha * w_alpha.double()).sum()).backward()
    return dict(
        means=_f32(means), quats=_f32(quats), scales=_f32(scales), opacities=_f32(op),
        sh=_f32(sh), w_rgb=_f32(w_rgb), w_alpha=_f32(w_alpha), K=_f32(K), viewmat=_f32(vm),
        W=np.int32(W), H=np.int32(H), rgb=rgb.detach().numpy(), alpha=alpha.detach().numpy(),
        d_means=leaves[0].grad.numpy(), d_quats=leaves[1].grad.numpy(),
        d_scales=leaves[2].grad.numpy(), d_opacities=leaves[3].grad.numpy(),
        d_sh=leaves[4].grad.numpy())


def adam_case() -> dict:
    rng = np.random.default_rng(30)
    f32 = np.float32
    steps, n = 20, 1024
    p0 = rng.standard_normal(n).astype(f32)
    grads = (rng.standard_normal((steps, n)) * 1e-3).astype(f32)
    out = dict(p0=p0, grads=grads, lr=np.float64(1e-3), b1=np.float64(0.9),
               b2=np.float64(0.999))
    for tag, eps in (("e15", 1e-15), ("e8", 1e-8)):
        p, m, v = p0.copy(), np.zeros(n, f32), np.zeros(n, f32)
        for k in range(steps):
            adam_ref.adam_step(p, grads[k], m, v, 1e-3, 0.9, 0.999, eps, k + 1)
        out[f"p_{tag}"], out[f"m_{tag}"], out[f"v_{tag}"] = p, m, v
    rows, width = 256, 3
    sp0 = rng.standard_normal((rows, width)).astype(f32)
    sgrads = (rng.standard_normal((steps, rows, width)) * 1e-3).astype(f32)
    masks = rng.random((steps, rows)) < 0.6
    p, m, v = sp0.copy(), np.zeros_like(sp0), np.zeros_like(sp0)
    st = np.zeros(rows, f32)
    for k in range(steps):
        adam_ref.selective_adam_step(p, sgrads[k], m, v, st, masks[k], 1e-3, 0.9, 0.999, 1e-15)
    out.update(sel_p0=sp0, sel_grads=sgrads, sel_masks=masks.astype(np.uint8), sel_p=p, sel_m=m,
               sel_v=v, sel_steps=st)
    return out


CASES = {"config1": config1_case, "fwd_bwd_small": fwd_bwd_case, "adam_small": adam_case}


def load(name: str) -> dict:
    with np.load(HERE / f"{name}.npz") as z:
        return {k: z[k] for k in z.files}


def main() -> None:
    torch.set_num_threads(8)
    for name, fn in CASES.items():
        arrays = fn()
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        size = (HERE / f"{name}.npz").stat().st_size
        print(f"{name}.npz: {len(arrays)} arrays, {size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
