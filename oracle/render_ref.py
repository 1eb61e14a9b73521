"""PyTorch-CPU restatement of the reference renderer. TEST INFRASTRUCTURE ONLY.

Restates metal_gauss/torch_ref.py (projection 49-144, tile assignment 147-196,
depth-slab compositing 199-295, render 298-337) and metal_gauss/sh.py (real SH
basis, 24-62), plus the fused preprocess contract of
metal_gauss/csrc/preprocess.metal:180-221 (SnugBox extents, validity test and
colour only for valid Gaussians). Differentiable end to end through torch
autograd, in any float dtype.

Pinned by tests/test_oracle_render.py:
  * the reference's known-answer tests (tests/test_torch_ref.py:36-284):
    principal point, occlusion, culling, alpha linear in opacity, the 0.999
    clamp, area ~ 1/z^2, camera translation, off-axis blow-up guard;
  * float64 gradcheck on the reference's 2-Gaussian 12x12 scene
    (tests/test_torch_ref.py:218-251);
  * an independent brute-force float64 per-pixel loop (test file) on tiny
    scenes, which pins the slab/cumprod compositing and the 1/255 cutoff;
  * the SH basis against scipy's complex spherical harmonics (textbook real
    SH with the Condon-Shortley phase), which pins every constant and
    polynomial of sh.py:11-62;
  * the projected covariance against J Sigma J^T with J from autograd of the
    projection map, which pins the closed-form Jacobian of torch_ref.py:90-98.
"""

from __future__ import annotations

import math

import torch

# Real SH normalisations (sh.py:11-17).
SH_C0 = 0.28209479177387814
SH_C1 = 0.4886025119029199
SH_C2 = (1.0925484305920792, -1.0925484305920792, 0.31539156525252005,
         -1.0925484305920792, 0.5462742152960396)
SH_C3 = (-0.5900435899266435, 2.890611442640554, -0.4570457994644658,
         0.3731763325901154, -0.4570457994644658, 1.445305721320277,
         -0.5900435899266435)


def num_sh_bases(degree: int) -> int:
    return (degree + 1) ** 2


def sh_basis(degree: int, dirs: torch.Tensor) -> torch.Tensor:
    """(N,3) unit directions -> (N,(degree+1)^2) basis values (sh.py:39-62)."""
    x, y, z = dirs[:, 0], dirs[:, 1], dirs[:, 2]
    cols = [torch.full_like(x, SH_C0)]
    if degree >= 1:
        cols += [-SH_C1 * y, SH_C1 * z, -SH_C1 * x]
    if degree >= 2:
        xx, yy, zz = x * x, y * y, z * z
        cols += [SH_C2[0] * x * y, SH_C2[1] * y * z, SH_C2[2] * (2.0 * zz - xx - yy),
                 SH_C2[3] * x * z, SH_C2[4] * (xx - yy)]
    if degree >= 3:
        cols += [SH_C3[0] * y * (3.0 * xx - yy), SH_C3[1] * x * y * z,
                 SH_C3[2] * y * (4.0 * zz - xx - yy),
                 SH_C3[3] * z * (2.0 * zz - 3.0 * xx - 3.0 * yy),
                 SH_C3[4] * x * (4.0 * zz - xx - yy), SH_C3[5] * z * (xx - yy),
                 SH_C3[6] * x * (xx - 3.0 * yy)]
    return torch.stack(cols, dim=1)


def eval_sh(degree: int, sh: torch.Tensor, dirs: torch.Tensor) -> torch.Tensor:
    """sh (N,K,3), dirs (N,3) -> (N,3) radiance before +0.5 (sh.py:24-62)."""
    k = num_sh_bases(degree)
    if sh.shape[1] < k:
        raise ValueError(f"need {k} SH bases for degree {degree}, got {sh.shape[1]}")
    B = sh_basis(degree, dirs)                       # (N,k)
    return (B[:, :, None] * sh[:, :k, :]).sum(dim=1)


def quat_to_rotmat(q: torch.Tensor) -> torch.Tensor:
    """(N,4) wxyz, normalised internally -> (N,3,3) (torch_ref.py:31-39)."""
    q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    w, x, y, z = q.unbind(-1)
    rows = [
        [1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
        [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
        [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
    ]
    return torch.stack([torch.stack(r, dim=-1) for r in rows], dim=-2)


def build_cov3d(quats: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Sigma = (R diag s)(R diag s)^T (torch_ref.py:42-46)."""
    M = quat_to_rotmat(quats) * scales[:, None, :]
    return M @ M.transpose(1, 2)


def _cov2d(means, cov3d, viewmat, fx, fy, W, H, near):
    """Camera-space centre, clamped depth and the undilated EWA covariance
    T Sigma T^T with T = J(clamped point) Rw (torch_ref.py:63-98)."""
    R, t = viewmat[:3, :3], viewmat[:3, 3]
    p = means @ R.T + t
    zc = p[:, 2].clamp_min(near)
    lim_x = 1.3 * (0.5 * W / fx)
    lim_y = 1.3 * (0.5 * H / fy)
    tx = (p[:, 0] / zc).clamp(-lim_x, lim_x) * zc
    ty = (p[:, 1] / zc).clamp(-lim_y, lim_y) * zc
    zero = torch.zeros_like(zc)
    J = torch.stack([
        torch.stack([fx / zc, zero, -fx * tx / (zc * zc)], dim=-1),
        torch.stack([zero, fy / zc, -fy * ty / (zc * zc)], dim=-1),
    ], dim=1)
    T = J @ R
    return p, zc, T @ cov3d @ T.transpose(1, 2)


def project(means, cov3d, viewmat, fx, fy, cx, cy, W, H, near, far, blur: float = 0.3,
            max_radius_frac: float = 1.0, antialias: bool = False):
    """-> (uv, conic, depth, radius, valid, opacity_scale) (torch_ref.py:49-144)."""
    p, zc, cov = _cov2d(means, cov3d, viewmat, fx, fy, W, H, near)
    z = p[:, 2]
    uv = torch.stack([fx * p[:, 0] / zc + cx, fy * p[:, 1] / zc + cy], dim=-1)
    det0 = cov[:, 0, 0] * cov[:, 1, 1] - cov[:, 0, 1] * cov[:, 1, 0]
    a = cov[:, 0, 0] + blur
    b = cov[:, 0, 1]
    c = cov[:, 1, 1] + blur
    det = a * c - b * b
    if antialias:
        scale = (det0.clamp_min(0.0) / det.clamp_min(1e-12)).clamp(0.0, 1.0).sqrt()
    else:
        scale = torch.ones_like(det)
    ds = det.clamp_min(1e-12)
    conic = torch.stack([c / ds, -b / ds, a / ds], dim=-1)
    mid = 0.5 * (a + c)
    lam = (mid + (mid * mid - ds).clamp_min(0).sqrt()).clamp_min(1e-12)
    radius = 3.0 * lam.sqrt()
    u, v = uv[:, 0], uv[:, 1]
    valid = ((z > near) & (z < far) & (det > 1e-12)
             & (radius < max_radius_frac * max(W, H))
             & (u + radius > 0) & (u - radius < W) & (v + radius > 0) & (v - radius < H))
    return uv, conic, z, radius, valid, scale


def preprocess(means, quats, scales, opacities, sh, viewmat, fx, fy, cx, cy, W, H,
               near=0.01, far=100.0, blur=0.3, max_radius=None, sh_degree=3):
    """The fused preprocess contract (preprocess.metal:114-221).

    Returns (uv, conic, depth, rxy, valid, color). rxy are the SnugBox
    half-extents sqrt(2 ln(255 op)) sqrt(cov_axis) capped at the 3-sigma
    radius; validity uses them for the screen test; colour is the SH colour
    (+0.5, clamped at 0) for valid Gaussians and 0 otherwise. ``sh`` is
    (N,16,3) or None (no colour).
    """
    if max_radius is None:
        max_radius = float(max(W, H))
    cov3d = build_cov3d(quats, scales)
    p, zc, cov = _cov2d(means, cov3d, viewmat, fx, fy, W, H, near)
    z = p[:, 2]
    u = fx * p[:, 0] / zc + cx
    v = fy * p[:, 1] / zc + cy
    a = cov[:, 0, 0] + blur
    b = cov[:, 0, 1]
    c = cov[:, 1, 1] + blur
    det = a * c - b * b
    ds = det.clamp_min(1e-12)
    conic = torch.stack([c / ds, -b / ds, a / ds], dim=-1)
    mid = 0.5 * (a + c)
    lam = (mid + (mid * mid - ds).clamp_min(0).sqrt()).clamp_min(1e-12)
    radius = 3.0 * lam.sqrt()
    rs = (2.0 * torch.log((255.0 * opacities.detach()).clamp_min(1.0))).sqrt()
    rx = torch.minimum(rs * a.detach().clamp_min(0).sqrt(), radius.detach())
    ry = torch.minimum(rs * c.detach().clamp_min(0).sqrt(), radius.detach())
    ud, vd = u.detach(), v.detach()
    valid = ((z > near) & (z < far) & (det > 1e-12) & (radius < max_radius) & (rx > 0)
             & (ry > 0) & (ud + rx > 0) & (ud - rx < W) & (vd + ry > 0) & (vd - ry < H))
    uv = torch.stack([u, v], dim=-1)
    color = None
    if sh is not None:
        cam_center = -viewmat[:3, :3].T @ viewmat[:3, 3]
        d = means - cam_center
        d = d / d.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        col = (eval_sh(sh_degree, sh[:, :num_sh_bases(sh_degree)], d) + 0.5).clamp_min(0.0)
        color = torch.where(valid[:, None], col, torch.zeros_like(col))
    return uv, conic, z.detach(), torch.stack([rx, ry], dim=-1), valid, color


def tile_lists(uv, radius, valid, depth, W, H, tile):
    """Per-tile depth-sorted Gaussian indices, padded with -1 (torch_ref.py:147-196).

    Returns (tiles_x, tiles_y, buf (n_tiles, K) long, total pairs). Every
    Gaussian is listed in every tile of its 3-sigma box; within a tile the
    order is by depth (ties by Gaussian order, a stable sort).
    """
    tx, ty = math.ceil(W / tile), math.ceil(H / tile)
    n_tiles = tx * ty
    dev = uv.device
    idx = torch.nonzero(valid, as_tuple=True)[0]
    if idx.numel() == 0:
        return tx, ty, torch.full((n_tiles, 1), -1, dtype=torch.long, device=dev), 0
    u, v, r = uv[idx, 0], uv[idx, 1], radius[idx]
    x0 = ((u - r) / tile).floor().clamp(0, tx - 1).long()
    x1 = ((u + r) / tile).floor().clamp(0, tx - 1).long()
    y0 = ((v - r) / tile).floor().clamp(0, ty - 1).long()
    y1 = ((v + r) / tile).floor().clamp(0, ty - 1).long()
    nx, ny = x1 - x0 + 1, y1 - y0 + 1
    per = nx * ny
    total = int(per.sum())
    owner = torch.repeat_interleave(torch.arange(idx.numel(), device=dev), per)
    k = torch.arange(total, device=dev) - (torch.cumsum(per, 0) - per)[owner]
    tile_id = (y0[owner] + k // nx[owner]) * tx + (x0[owner] + k % nx[owner])
    order = torch.argsort(depth[idx][owner], stable=True)
    order = order[torch.argsort(tile_id[order], stable=True)]
    t_sorted, g_sorted = tile_id[order], idx[owner][order]
    counts = torch.bincount(t_sorted, minlength=n_tiles)
    first = torch.cumsum(counts, 0) - counts
    rank = torch.arange(t_sorted.numel(), device=dev) - first[t_sorted]
    buf = torch.full((n_tiles, int(counts.max())), -1, dtype=torch.long, device=dev)
    buf[t_sorted, rank] = g_sorted
    return tx, ty, buf, total


def rasterize(uv, conic, opacity, color, depth, radius, valid, W, H, tile: int = 16,
              tile_chunk: int = 32, slab: int = 256, background=None,
              min_transmittance: float = 1e-4):
    """Front-to-back compositing over depth slabs (torch_ref.py:199-295).

    Within a slab the weights are alpha_i * T_in * prod_{j<i}(1 - alpha_j),
    with the exclusive product formed as cumprod / (1 - alpha) as in the
    reference; transmittance carries across slabs. A chunk of tiles stops at
    a slab boundary once its largest transmittance is below
    ``min_transmittance`` (0 composites everything). Returns (rgb, alpha, info).
    """
    dev, dt = uv.device, uv.dtype
    tx, ty, buf, total = tile_lists(uv, radius, valid, depth, W, H, tile)
    n_tiles, P = tx * ty, tile * tile
    out_rgb = torch.zeros(n_tiles, P, 3, device=dev, dtype=dt)
    out_a = torch.zeros(n_tiles, P, device=dev, dtype=dt)
    py, px = torch.meshgrid(torch.arange(tile, device=dev, dtype=dt),
                            torch.arange(tile, device=dev, dtype=dt), indexing="ij")
    offs = torch.stack([px.reshape(-1), py.reshape(-1)], dim=-1) + 0.5
    t_all = torch.arange(n_tiles, device=dev)
    origin = torch.stack([(t_all % tx) * tile, (t_all // tx) * tile], dim=-1).to(dt)
    K = buf.shape[1]
    rgb_chunks, a_chunks = [], []
    for lo in range(0, n_tiles, tile_chunk):
        hi = min(lo + tile_chunk, n_tiles)
        lists = buf[lo:hi]
        C = hi - lo
        acc_rgb = torch.zeros(C, P, 3, device=dev, dtype=dt)
        acc_a = torch.zeros(C, P, device=dev, dtype=dt)
        if bool((lists >= 0).any()):
            pix = origin[lo:hi, None, :] + offs[None]
            T = torch.ones(C, P, device=dev, dtype=dt)
            for s0 in range(0, K, slab):
                ids = lists[:, s0:s0 + slab]
                present = ids >= 0
                if not bool(present.any()):
                    break
                if float(T.detach().max()) < min_transmittance:
                    break
                g = ids.clamp_min(0)
                d = pix[:, None] - uv[g][:, :, None, :]
                cg = conic[g]
                q = (cg[..., 0:1] * d[..., 0] * d[..., 0] + 2.0 * cg[..., 1:2] * d[..., 0] * d[..., 1]
                     + cg[..., 2:3] * d[..., 1] * d[..., 1])
                alpha = (opacity[g][..., None] * (-0.5 * q).exp()).clamp(max=0.999)
                alpha = torch.where(present[..., None], alpha, torch.zeros_like(alpha))
                alpha = torch.where(alpha > 1.0 / 255.0, alpha, torch.zeros_like(alpha))
                keep = 1.0 - alpha
                cp = torch.cumprod(keep, dim=1)
                w = alpha * (cp / keep.clamp_min(1e-10)) * T[:, None, :]
                acc_rgb = acc_rgb + torch.einsum("csp,csj->cpj", w, color[g])
                acc_a = acc_a + w.sum(dim=1)
                T = T * cp[:, -1]
        rgb_chunks.append(acc_rgb)
        a_chunks.append(acc_a)
    out_rgb = torch.cat(rgb_chunks, 0)
    out_a = torch.cat(a_chunks, 0)
    img = out_rgb.reshape(ty, tx, tile, tile, 3).permute(0, 2, 1, 3, 4).reshape(ty * tile, tx * tile, 3)
    alp = out_a.reshape(ty, tx, tile, tile).permute(0, 2, 1, 3).reshape(ty * tile, tx * tile)
    img, alp = img[:H, :W], alp[:H, :W]
    if background is not None:
        bg = torch.as_tensor(background, device=dev, dtype=dt)
        img = img + (1.0 - alp).clamp_min(0)[..., None] * bg
    return img, alp, {"tiles": n_tiles, "isect_total": total, "max_gaussians_in_a_tile": K,
                      "visible_gaussians": int(valid.sum())}


def render(means, quats, scales, opacities, sh, K, viewmat, W, H, sh_degree: int = 3,
           tile: int = 16, tile_chunk: int = 32, near: float = 0.01, far: float = 100.0,
           slab: int = 256, background=(0.0, 0.0, 0.0), colors=None,
           max_radius_frac: float = 1.0, antialias: bool = False,
           min_transmittance: float = 1e-4):
    """One camera (torch_ref.py:298-337). Note the default tile here is the
    kernel's 16 (the reference's torch renderer defaults to 32)."""
    fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])
    cov3d = build_cov3d(quats, scales)
    uv, conic, depth, radius, valid, op_scale = project(
        means, cov3d, viewmat, fx, fy, cx, cy, W, H, near, far,
        max_radius_frac=max_radius_frac, antialias=antialias)
    opacities = opacities * op_scale
    if colors is None:
        cam_center = -viewmat[:3, :3].T @ viewmat[:3, 3]
        d = means - cam_center
        d = d / d.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        colors = (eval_sh(sh_degree, sh[:, :num_sh_bases(sh_degree)], d) + 0.5).clamp_min(0.0)
    return rasterize(uv, conic, opacities, colors, depth, radius, valid, W, H, tile=tile,
                     tile_chunk=tile_chunk, slab=slab, background=background,
                     min_transmittance=min_transmittance)
