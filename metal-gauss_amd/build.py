"""Ahead-of-time build of libmgauss.so for gfx950.

The reference compiles its Metal source at first use (metal_backend.py:76-108);
here the HIP sources are compiled once with hipcc, in-tree, into
``metal-gauss_amd/libmgauss.so``. Each translation unit is compiled in
parallel to an object file under ``_build/`` and the objects are linked into
one shared library that exports the C ABI declared in include/mgauss.h.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmgauss.so"
ARCH = "gfx950"

SOURCES = ["runtime.hip", "adam.hip", "preprocess.hip", "mip.hip", "mcmc.hip", "binning.hip", "sort.hip",
           "rasterize.hip", "ssim.hip", "ply.hip"]

# -packed-fp32-ops keeps the compiler from emitting packed fp32 VALU forms;
# hardware float atomics are requested explicitly (the gradient buffers are
# ordinary coarse-grained device memory).
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
    f"-I{PKG.parent / 'include'}",
]


# Multiply-add fusion only within one source expression (as written) for the
# Adam update and the projection backward: the backward's gradient arithmetic
# is instantiated twice, writing gradients and feeding the optimizer epilogue,
# and hipcc's default cross-statement fusion may round the two differently;
# with this both instantiations, and the separate Adam kernel, round alike.
FILE_FLAGS = {
    "adam.hip": ["-ffp-contract=on"],
    "preprocess.hip": ["-ffp-contract=on"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: cannot build the gfx950 library")


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *CFLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{p.stdout}\n{p.stderr}")
    # hipcc's host pass reports the device-only target feature; keep the rest.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    warn = "\n".join(l for l in p.stderr.splitlines() if noise not in l)
    return obj, warn


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link libmgauss.so. Always rebuilds.

    Holds ``_build/lock`` while compiling; backend.stale_lock_message explains
    a lock that an interrupted build left behind.
    """
    BUILD.mkdir(exist_ok=True)
    lock = BUILD / "lock"
    try:
        fd = os.open(lock, os.O_CREAT | os.O_EXCL | os.O_WRONLY)
    except FileExistsError:
        import time
        age = time.time() - lock.stat().st_mtime
        raise RuntimeError(
            f"build lock {lock} exists ({age:.0f}s old): another build is running, or an "
            f"interrupted one left it behind (then delete it: rm {lock})") from None
    os.close(fd)
    try:
        return _build(verbose, jobs)
    finally:
        lock.unlink(missing_ok=True)


def _build(verbose: bool, jobs: int | None) -> Path:
    objs = []
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, CSRC / s, BUILD / (Path(s).stem + ".o")) for s in SOURCES]
        for f in futs:
            obj, warn = f.result()
            objs.append(obj)
            if verbose and warn.strip():
                print(warn, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
