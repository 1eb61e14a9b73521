"""Seeded synthetic scenes and cameras for the benchmark configurations.

Scenes are drawn on the CPU from ``torch.Generator().manual_seed(seed)`` in a
fixed order (means, log-scales, quaternions, opacity logits, SH DC, SH rest),
so every machine produces the same bits; callers move them to the device.
Cameras are look-at pinholes with OpenCV axes (+x right, +y down, +z forward),
as the reference's camera paths use (metal_gauss/render_path.py:125-139), with
f = (W/2) / tan(fov/2) and the principal point at the image centre.

The five configurations are those of BASELINE.json ``configs``:
  1  10k Gaussians, means U[-1,1]^3, log-scales N(-4,0.4), SH degree 0,
     256x256, camera at distance 4, fov 40 deg
  2  300k, means U[-1.3,1.3]^3, log-scales N(-4.5,0.5), logits N(0,1.5),
     SH 3 (DC N(0,0.3), rest N(0,0.05)), 800x800 at radius 4, azimuth and
     elevation U[-30,60] deg, fov 39.6 deg, white background
  3  1M parameter groups for Adam (see config3_groups)
  4  1M Gaussians as config 2, 100 cameras on a radius-4 sphere at 800x800
  5  3M Gaussians in a 4x4x4 domain, log-scales N(-5,0.7), logits N(0.5,1.5),
     SH 3, 1920x1080 from inside the cloud at 2.0 from the centre, fov 60 deg
     (horizontal); config5_crowded adds a dense cluster in front of the
     camera so that tile lists exceed 10k entries and the keys 30M
Quaternions are N(0,1)^4 (normalised by the renderer) everywhere.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class Camera:
    K: torch.Tensor          # (3,3)
    viewmat: torch.Tensor    # (4,4) world -> camera
    W: int
    H: int


@dataclass
class Scene:
    means: torch.Tensor      # (N,3)
    log_scales: torch.Tensor  # (N,3)
    quats: torch.Tensor      # (N,4)
    logit_opac: torch.Tensor  # (N,)
    sh_dc: torch.Tensor      # (N,1,3)
    sh_rest: torch.Tensor    # (N,15,3)  (zeros past the degree)
    sh_degree: int

    def to(self, device) -> "Scene":
        return Scene(*(t.to(device) for t in (self.means, self.log_scales, self.quats,
                                               self.logit_opac, self.sh_dc, self.sh_rest)),
                     self.sh_degree)

    @property
    def n(self) -> int:
        return self.means.shape[0]

    def activated(self):
        """(means, quats, scales, opacities, sh (N,16,3)) as render() takes them."""
        return (self.means, self.quats, torch.exp(self.log_scales), torch.sigmoid(self.logit_opac),
                torch.cat([self.sh_dc, self.sh_rest], dim=1))


def intrinsics(W: int, H: int, fov_deg: float, horizontal: bool = True) -> torch.Tensor:
    f = (0.5 * (W if horizontal else H)) / math.tan(0.5 * math.radians(fov_deg))
    return torch.tensor([[f, 0.0, W / 2], [0.0, f, H / 2], [0.0, 0.0, 1.0]])


def look_at(eye, target, world_up=(0.0, 0.0, 1.0)) -> torch.Tensor:
    """World->camera 4x4 with OpenCV axes looking from eye at target."""
    eye = torch.as_tensor(eye, dtype=torch.float64)
    target = torch.as_tensor(target, dtype=torch.float64)
    up = torch.as_tensor(world_up, dtype=torch.float64)
    fwd = target - eye
    fwd = fwd / fwd.norm()
    if abs(float(fwd @ up)) > 0.999:      # looking along the up axis
        up = torch.tensor([0.0, 1.0, 0.0], dtype=torch.float64)
    right = torch.linalg.cross(fwd, up)
    right = right / right.norm()
    down = torch.linalg.cross(fwd, right)
    Rc2w = torch.stack([right, down, fwd], dim=1)   # columns: camera axes in world
    vm = torch.eye(4, dtype=torch.float64)
    vm[:3, :3] = Rc2w.T
    vm[:3, 3] = -Rc2w.T @ eye
    return vm.to(torch.float32)


def orbit_camera(W, H, fov_deg, radius, az_deg, el_deg, target=(0.0, 0.0, 0.0)) -> Camera:
    az, el = math.radians(az_deg), math.radians(el_deg)
    eye = (radius * math.cos(el) * math.cos(az), radius * math.cos(el) * math.sin(az),
           radius * math.sin(el))
    return Camera(intrinsics(W, H, fov_deg), look_at(eye, target), W, H)


def _scene(n, seed, lo, hi, ls_mu, ls_sd, lg_mu, lg_sd, deg, dc_sd=0.3, rest_sd=0.05,
           heavy_tail=False) -> Scene:
    g = torch.Generator().manual_seed(seed)
    means = torch.rand(n, 3, generator=g) * (hi - lo) + lo
    if heavy_tail:
        # Student-t (3 dof) log-scales: a heavy upper tail of large splats.
        z = torch.randn(n, 3, generator=g)
        chi = sum(torch.randn(n, 1, generator=g) ** 2 for _ in range(3)) / 3.0
        log_scales = ls_mu + ls_sd * z / chi.sqrt()
    else:
        log_scales = torch.randn(n, 3, generator=g) * ls_sd + ls_mu
    quats = torch.randn(n, 4, generator=g)
    logit = torch.randn(n, generator=g) * lg_sd + lg_mu
    dc = torch.randn(n, 1, 3, generator=g) * dc_sd
    rest = torch.randn(n, 15, 3, generator=g) * rest_sd
    nb = (deg + 1) ** 2
    rest[:, nb - 1:] = 0.0
    return Scene(means, log_scales, quats, logit, dc, rest, deg)


def config1():
    """(scene, camera, background) of BASELINE configs[0]."""
    s = _scene(10_000, 0, -1.0, 1.0, -4.0, 0.4, 0.0, 1.0, 0)
    cam = orbit_camera(256, 256, 40.0, 4.0, 0.0, 0.0)
    return s, cam, (0.0, 0.0, 0.0)


def config2():
    s = _scene(300_000, 1, -1.3, 1.3, -4.5, 0.5, 0.0, 1.5, 3)
    g = torch.Generator().manual_seed(101)
    az, el = (torch.rand(2, generator=g) * 90.0 - 30.0).tolist()
    return s, orbit_camera(800, 800, 39.6, 4.0, az, el), (1.0, 1.0, 1.0)


def config2_target(H=800, W=800, seed=1):
    """L1 target of config 2: U[0,1] per pixel, 5x5 box blurred."""
    g = torch.Generator().manual_seed(seed + 1000)
    t = torch.rand(1, 3, H, W, generator=g)
    t = torch.nn.functional.avg_pool2d(t, 5, stride=1, padding=2, count_include_pad=False)
    return t[0].permute(1, 2, 0).contiguous()


def config3_groups(n=1_000_000):
    """(name, floats per Gaussian, lr) of the config-3 / trainer Adam groups
    (train.py:167-191 with the configured rates)."""
    return [("means", 3, 1.6e-4), ("scales", 3, 5e-3), ("quats", 4, 1e-3), ("opac", 1, 5e-2),
            ("sh_dc", 3, 2.5e-3), ("sh_rest", 45, 1.25e-4)]


def config4(n=1_000_000, n_views=100):
    """(scene, cameras, targets-generator, background) of BASELINE configs[3]."""
    s = _scene(n, 3, -1.3, 1.3, -4.5, 0.5, 0.0, 1.5, 3)
    g = torch.Generator().manual_seed(303)
    cams = []
    for _ in range(n_views):
        v = torch.randn(3, generator=g)
        v = v / v.norm()
        az = math.degrees(math.atan2(float(v[1]), float(v[0])))
        el = math.degrees(math.asin(max(-1.0, min(1.0, float(v[2])))))
        cams.append(orbit_camera(800, 800, 39.6, 4.0, az, el))
    return s, cams, (0.0, 0.0, 0.0)


def config4_target(view: int, H=800, W=800):
    """Smooth target: an 8x8 U[0,1] grid per view, bilinearly upsampled."""
    g = torch.Generator().manual_seed(10_000 + view)
    grid = torch.rand(1, 3, 8, 8, generator=g)
    t = torch.nn.functional.interpolate(grid, size=(H, W), mode="bilinear", align_corners=False)
    return t[0].permute(1, 2, 0).contiguous()


def fps_scene(n, seed=7):
    """Forward-only render workload (the reference's bench/render_fps.py renders a
    loaded ply from one fixed view; this is a seeded stand-in of the same
    size): n Gaussians with SH 3 filling the view frustum of a camera at the
    origin looking down +z (identity world->camera), depths U[1.5, 6],
    log-scales N(-4.5, 0.5), opacity logits N(0, 1.5)."""
    g = torch.Generator().manual_seed(seed)
    z = torch.rand(n, generator=g) * 4.5 + 1.5
    xy = (torch.rand(n, 2, generator=g) * 2.0 - 1.0) * 0.45 * z[:, None]
    means = torch.cat([xy, z[:, None]], dim=1)
    log_scales = torch.randn(n, 3, generator=g) * 0.5 - 4.5
    quats = torch.randn(n, 4, generator=g)
    logit = torch.randn(n, generator=g) * 1.5
    dc = torch.randn(n, 1, 3, generator=g) * 0.3
    rest = torch.randn(n, 15, 3, generator=g) * 0.05
    return Scene(means, log_scales, quats, logit, dc, rest, 3)


def config5(n=3_000_000):
    s = _scene(n, 4, -2.0, 2.0, -5.0, 0.7, 0.5, 1.5, 3, heavy_tail=True)
    cam = Camera(intrinsics(1920, 1080, 60.0, horizontal=True),
                 look_at((2.0, 0.0, 0.0), (0.0, 0.0, 0.0)), 1920, 1080)
    return s, cam, (0.0, 0.0, 0.0)


def config5_crowded(n=3_000_000, n_cluster=600_000):
    """Config 5 with the stress its text names actually reached: the same
    scene and camera plus a cluster of ``n_cluster`` Gaussians uniform in a
    ball of radius 0.2 centred 1.0 in front of the camera (log-scales
    N(-5, 0.5), logits N(0.5, 1.5), SH as config 2), drawn from seed 44 after
    the base scene. At the defaults the lists hold about 39M intersections,
    over a thousand tiles hold more than 10k entries and the longest about
    23k."""
    s, cam, bg = config5(n)
    g = torch.Generator().manual_seed(44)
    d = torch.randn(n_cluster, 3, generator=g)
    d = d / d.norm(dim=1, keepdim=True)
    r = 0.2 * torch.rand(n_cluster, 1, generator=g) ** (1.0 / 3.0)
    means = torch.tensor([1.0, 0.0, 0.0]) + d * r
    log_scales = torch.randn(n_cluster, 3, generator=g) * 0.5 - 5.0
    quats = torch.randn(n_cluster, 4, generator=g)
    logit = torch.randn(n_cluster, generator=g) * 1.5 + 0.5
    dc = torch.randn(n_cluster, 1, 3, generator=g) * 0.3
    rest = torch.randn(n_cluster, 15, 3, generator=g) * 0.05
    cat = torch.cat
    return Scene(cat([s.means, means]), cat([s.log_scales, log_scales]), cat([s.quats, quats]),
                 cat([s.logit_opac, logit]), cat([s.sh_dc, dc]), cat([s.sh_rest, rest]),
                 3), cam, bg
