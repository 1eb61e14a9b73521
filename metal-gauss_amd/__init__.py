"""metal_gauss_amd: the differentiable 3D Gaussian splatting step of
nandometzger/metal-gauss, rebuilt as hand-written gfx950 HIP kernels.

Public surface (names of the reference's modules):
    render                 api.render with backend "hip" (alias "metal")
    backend                the metal_backend surface: render, build_tile_lists,
                           build_tile_lists_metal, antialias_scale, ...
    FusedAdam              fused_adam.FusedAdam
    SelectiveAdam          selective_adam.SelectiveAdam
    ssim, gaussian_kernel  the fused SSIM loss used by the training step
    compute_3d_filter,     mipfilter: Mip-Splatting's 3D filter (also folded
    apply_3d_filter        into render's projection kernel via filter_3d=)
    mcmc                   relocate / grow / add_noise / reset_adam_state
    io                     Splats, load_ply, save_ply, export_ply
    ext                    the reference's native-extension functions (backend._load())
    ListCapacity           tile-list sizing without a host read (render(list_capacity=))
"""

from .api import BACKENDS, render  # noqa: F401
from .fused_adam import FusedAdam  # noqa: F401
from .selective_adam import SelectiveAdam  # noqa: F401
from .ssim import gaussian_kernel, photometric_loss, ssim  # noqa: F401
from .mipfilter import apply_3d_filter, compute_3d_filter  # noqa: F401
from .backend import ListCapacity  # noqa: F401
from . import backend, ext  # noqa: F401

__version__ = "0.1.0"
