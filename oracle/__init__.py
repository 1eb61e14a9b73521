"""CPU oracle for the splatting hot path. TEST INFRASTRUCTURE ONLY.

Nothing in the product (metal-gauss_amd/) imports, links or runs anything in
this directory. Only tests/, __graft_entry__.smoke() and the cpu_baseline leg
of bench.py may use it, and only as the checker (or the timed CPU baseline),
never as a substitute for the HIP path.

Modules (each function cites the reference file:line it restates; paths are
relative to the nandometzger/metal-gauss repository):

  render_ref    PyTorch-CPU restatement of metal_gauss/torch_ref.py and
                metal_gauss/sh.py (projection, depth-slab compositing, render),
                plus the fused preprocess contract of preprocess.metal
                (SnugBox extents, validity, SH colour).
  binning_ref   numpy restatement of the tile binning (binning.metal,
                metal_backend.py:111-285): per-pair ellipse test, 64-bit
                (tile|depth) keys, stable order, tile ranges. Bit exact.
  raster_ref    the rasteriser's per-pixel contract (rasterize.metal:61-340):
                sequential front-to-back compositing with a per-pixel stop and
                its analytic back-to-front backward, in C (raster_seq.c, built
                by build.py) with a ctypes wrapper.
  adam_ref      numpy restatement of adam.metal / rasterize.mm:329-360 and of
                selective_adam.py.
  ssim_ref      PyTorch-CPU restatement of the SSIM expression the reference's
                tests use as oracle (tests/test_fused_ssim.py:19-30, ssim.py).

How each is pinned (so that the checker itself is checked) is listed in the
module docstrings and exercised by tests/test_oracle_*.py.
"""
