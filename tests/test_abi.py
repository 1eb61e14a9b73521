"""The C ABI boundary: the library loads, exports exactly what include/mgauss.h
declares, and rejects bad arguments with the reference's messages before it
touches a GPU. CPU only: no entry point here reaches the HIP runtime."""

from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "mgauss.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_reference_surface():
    names = declared_symbols()
    # One native entry point per function of the reference's pybind module
    # (rasterize.mm:518-533), minus pack_intersections (uncalled there).
    for ref in ("init", "rasterize_forward", "rasterize_backward", "preprocess_forward",
                "preprocess_backward", "adam_step", "ssim_tail_forward", "ssim_tail_backward",
                "ssim_stack_blur_h", "ssim_blur15", "ssim_chain_backward", "bin_count",
                "bin_write"):
        assert f"mg_{ref}" in names, f"no C entry point replaces {ref}"


def test_library_exports_every_declared_symbol():
    from metal_gauss_amd import _lib

    lib = _lib.open_library()
    for name in declared_symbols():
        assert hasattr(lib, name), f"libmgauss.so does not export {name}"
    assert set(declared_symbols()) == set(_lib.EXPORTS), "ctypes table and header disagree"


def test_version_and_tile_limit():
    from metal_gauss_amd import _lib

    lib = _lib.open_library()
    assert lib.mg_version() >= 10000
    assert lib.mg_max_tile() == 32


def test_oversized_tile_is_refused_with_the_reference_message():
    """rasterize.mm:66-73 refuses a tile whose threadgroup exceeds the limit;
    tests/test_metal.py:205-213 pins the wording."""
    from metal_gauss_amd import _lib

    lib = _lib.open_library()
    rc = lib.mg_rasterize_forward(0, None, None, None, None, None, 1, 96, 64, 64, 2, 1e-4,
                                  None, 0, None, 0, 1, 1, 1, 1, None, None, None)
    assert rc == 1
    assert "threads per threadgroup" in lib.mg_last_error().decode()


def test_bad_arguments_fail_before_any_launch():
    from metal_gauss_amd import _lib

    lib = _lib.open_library()
    arr = (ctypes.c_void_p * 1)(None)
    n = (ctypes.c_int64 * 1)(1)
    assert lib.mg_adam_step_multi(99, arr, arr, arr, arr, n, (ctypes.c_double * 1)(1.0),
                                  n, 0.9, 0.999, 1e-15, 0, None) == 1
    assert "at most 32" in lib.mg_last_error().decode()
    # tiles that do not cover the image
    assert lib.mg_bin_count(10, 1, 1, 1, 1, 1, 100, 100, 16, 3, 7, 1, None) == 1
    assert "do not cover" in lib.mg_last_error().decode()
    # conic without opacity
    assert lib.mg_bin_count(10, 1, 1, 1, None, 1, 100, 100, 16, 7, 7, 1, None) == 1
    assert "together" in lib.mg_last_error().decode()
    # scan workspace too small
    assert lib.mg_exclusive_scan_i32(1, 5000, 1, 1, None, 1, 8, None) == 1
    assert "workspace" in lib.mg_last_error().decode()
    # sort bit range
    assert lib.mg_sort_pairs_u64(1, 1, 1, 1, 10, 0, 65, 1, 1 << 20, None) == 1
    assert "bit range" in lib.mg_last_error().decode()
    # tile counting sort: tile count and aliasing
    assert lib.mg_sort_pairs_by_tile(10, 1, 1, 5000, 1, 1, 1, 1 << 20, None) == 1
    assert "tiles" in lib.mg_last_error().decode()
    assert lib.mg_sort_pairs_by_tile(10, 1, 2, 16, 2, 1, 1, 1 << 20, None) == 1
    assert "alias" in lib.mg_last_error().decode()
    assert lib.mg_sort_pairs_by_tile(10, 1, 2, 16, 3, 1, 1, 1 << 20, None) == 1
    assert "16-byte aligned" in lib.mg_last_error().decode()
    assert lib.mg_sort_pairs_by_tile(10, 16, 2, 16, 3, 1, 1, 8, None) == 1
    assert "workspace" in lib.mg_last_error().decode()
    # SH layout
    vm = (ctypes.c_float * 16)(*([0.0] * 16))
    cc = (ctypes.c_float * 3)(0.0, 0.0, 0.0)
    rc = lib.mg_preprocess_forward(4, 1, 1, 1, 1, None, 0, 1, vm, 1.0, 1.0, 0.0, 0.0, 8, 8,
                                   0.01, 100.0, 0.3, 8.0, cc, 3, 1, 1, 1, 1, 1, None, 1, None)
    assert rc == 1
    assert "(N,16,3)" in lib.mg_last_error().decode()
    rc = lib.mg_preprocess_forward(4, 1, 1, 1, None, None, 1, 1, vm, 1.0, 1.0, 0.0, 0.0, 8, 8,
                                   0.01, 100.0, 0.3, 8.0, cc, 4, 1, 1, 1, 1, 1, None, None,
                                   None)
    assert rc == 1 and "sh_degree" in lib.mg_last_error().decode()
    # optimizer epilogue: its tensors must be the kernel's inputs, and the SH
    # must be 16-byte aligned (host pointers only; nothing is dereferenced)
    ins = [16, 32, 48, 96, 64, 80]     # means quats scales opacities sh sh_rest

    def bwd(epi, sh=64):
        return lib.mg_preprocess_backward_mip(
            4, 16, 32, 48, sh, 80, 0, 1, 1, 1, 10, 1, vm, 1.0, 1.0, 0.0, 0.0, 8, 8, 0.01,
            100.0, 0.3, 8.0, cc, 3, 96, None, 0, 3, 0.0, 0.0, 1, None, None, None, None,
            None, None, ctypes.byref(epi), None)

    epi = _lib.AdamEpilogue()
    for i, ptr in enumerate(ins):
        epi.p[i], epi.m[i], epi.v[i], epi.lr[i], epi.step[i] = ptr, 1 << 20, 2 << 20, 1e-3, 1
    epi.beta1, epi.beta2, epi.eps = 0.9, 0.999, 1e-15
    epi.p[3] = 112
    assert bwd(epi) == 1 and "tensor 3 is not the kernel's input" in lib.mg_last_error().decode()
    epi.p[3], epi.p[4] = 96, 68
    assert bwd(epi, sh=68) == 1 and "16-byte aligned" in lib.mg_last_error().decode()
    epi.p[4], epi.step[2] = 64, 0
    assert bwd(epi) == 1 and "step 0 < 1" in lib.mg_last_error().decode()


def test_workspace_size_queries_are_pure():
    from metal_gauss_amd import _lib

    lib = _lib.open_library()
    assert lib.mg_scan_workspace_bytes(0) > 0
    assert lib.mg_scan_workspace_bytes(1 << 20) >= 8 * ((1 << 20) // 2048)
    assert lib.mg_sort_workspace_bytes(3_500_000) >= 4 * 256 * (3_500_000 // 2048)
    assert lib.mg_ssim_fused_workspace_bytes(800, 800) == 2 * 4 * 25 * 50 * 3   # SSIM + L1 sums
    # tile sort: one count per (tile, chunk) plus the tile totals
    assert lib.mg_sort_pairs_by_tile_workspace_bytes(5_000_000, 2500) >= 4 * 2500 * 407
    assert lib.mg_bin_lists_finish_workspace_bytes(5_000_000) >= \
        lib.mg_sort_pairs_by_tile_workspace_bytes(5_000_000, 4096)


@pytest.mark.parametrize("missing", [True])
def test_missing_library_raises_instead_of_falling_back(tmp_path, monkeypatch, missing):
    from metal_gauss_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libmgauss.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="Refusing to silently substitute"):
        _lib.open_library()
