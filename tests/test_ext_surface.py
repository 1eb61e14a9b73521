"""The reference's extension surface (metal_gauss_amd.ext) on the CPU: the
thirteen functions exist with the reference's parameter names and order
(metal_gauss/csrc/rasterize.mm:79-533, bound at 518-533), and without a GPU
they raise instead of computing anything elsewhere."""

from __future__ import annotations

import inspect

import pytest
import torch

# Parameter lists of the reference's pybind functions, in order.
REFERENCE_SIGNATURES = {
    "init": ["src"],
    "rasterize_forward": ["uv", "conic", "opacity", "color", "gauss_ids", "tile_offsets", "W",
                          "H", "tile", "tiles_x"],
    "rasterize_backward": ["uv", "conic", "opacity", "color", "gauss_ids", "tile_offsets",
                           "final_T", "n_contrib", "grad_rgb", "grad_alpha", "W", "H", "tile",
                           "tiles_x", "want_absgrad"],
    "preprocess_forward": ["means", "quats", "scales", "sh", "sh_rest", "opacities", "viewmat",
                           "fx", "fy", "cx", "cy", "W", "H", "near", "far", "blur",
                           "max_radius", "cam_center", "sh_degree"],
    "preprocess_backward": ["means", "quats", "scales", "sh", "sh_rest", "d_uv", "d_conic",
                            "d_color", "valid", "viewmat", "fx", "fy", "cx", "cy", "W", "H",
                            "near", "far", "blur", "max_radius", "cam_center", "sh_degree"],
    "adam_step": ["p", "g", "m", "v", "lr", "b1", "b2", "eps", "step"],
    "ssim_tail_forward": ["b", "H", "W"],
    "ssim_tail_backward": ["b", "gout", "H", "W"],
    "ssim_stack_blur_h": ["x", "y", "w", "H", "W"],
    "ssim_blur15": ["src", "w", "dir", "H", "W"],
    "ssim_chain_backward": ["x", "y", "d_stack", "H", "W"],
    "bin_count": ["uv", "rxy", "conic", "opacity", "valid", "W", "H", "tile", "tiles_x",
                  "tiles_y"],
    "bin_write": ["uv", "rxy", "conic", "opacity", "valid", "depth", "offsets", "total", "W",
                  "H", "tile", "tiles_x", "tiles_y"],
}


def test_every_function_has_the_reference_parameters():
    from metal_gauss_amd import ext

    assert sorted(ext.__all__) == sorted(REFERENCE_SIGNATURES)
    for name, params in REFERENCE_SIGNATURES.items():
        got = list(inspect.signature(getattr(ext, name)).parameters)
        assert got == params, name


def test_without_a_gpu_the_extension_raises():
    from metal_gauss_amd import ext

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: the GPU tests cover the extension")
    z = torch.zeros(4, 2)
    with pytest.raises(RuntimeError):
        ext.bin_count(z, z, torch.zeros(4, 3), torch.zeros(4), torch.zeros(4, dtype=torch.int32),
                      8, 8, 16, 1, 1)
