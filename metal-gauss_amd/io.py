"""Load and save 3D Gaussian Splatting .ply files (metal_gauss/io.py,
train.export_ply at train.py:582-624).

The INRIA convention stores *parameterised* values: opacity as a logit,
scale as a log, an unnormalised wxyz quaternion; ``f_dc_{0,1,2}`` is the
degree-0 SH term per channel and ``f_rest_{0..3P-1}`` the higher bases stored
channel-major, ``f_rest_[c*P + (b-1)]``. Same functions and results as the
reference:

* ``Splats`` (means, quats, scales, opacities, sh, sh_degree; ``len``,
  ``to``, ``subset``);
* ``load_ply(path, device="cpu", dtype=torch.float32)`` de-parameterises;
* ``save_ply(splats, path)`` writes activated Splats back in that convention;
* ``export_ply(p, path, filter_3d=None)`` writes the trainer's parameter dict,
  with Mip-Splatting's 3D filter baked in when given.

The reference reads and writes through ``plyfile``; here the format is
parsed directly (PLY header, then the body as one numpy structured array,
memory-mapped for binary files; binary little- and big-endian and ascii are
read, binary little-endian float32 is written). On a ROCm device the raw
float32 records are uploaded once and one HIP kernel (``mg_ply_decode``)
writes every activated tensor, and ``export_ply`` encodes records on the GPU
(``mg_ply_encode``) before a single copy to the host; on the CPU the same
arithmetic runs in numpy.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib

_PLY_TYPES = {"char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1", "short": "i2",
              "int16": "i2", "ushort": "u2", "uint16": "u2", "int": "i4", "int32": "i4",
              "uint": "u4", "uint32": "u4", "float": "f4", "float32": "f4", "double": "f8",
              "float64": "f8"}


@dataclass
class Splats:
    means: torch.Tensor      # (N,3) world
    quats: torch.Tensor      # (N,4) wxyz, normalised
    scales: torch.Tensor     # (N,3) linear
    opacities: torch.Tensor  # (N,)  in [0,1]
    sh: torch.Tensor         # (N,B,3)
    sh_degree: int

    def __len__(self) -> int:
        return self.means.shape[0]

    def to(self, device) -> "Splats":
        return Splats(self.means.to(device), self.quats.to(device), self.scales.to(device),
                      self.opacities.to(device), self.sh.to(device), self.sh_degree)

    def subset(self, idx) -> "Splats":
        return Splats(self.means[idx], self.quats[idx], self.scales[idx],
                      self.opacities[idx], self.sh[idx], self.sh_degree)


# ------------------------------------------------------------------ format

def _read_header(f):
    """(format, [(element, count, [(property, numpy type)])], header bytes)."""
    if f.readline().strip() != b"ply":
        raise ValueError("not a PLY file (no 'ply' magic)")
    fmt = None
    elements = []
    while True:
        line = f.readline()
        if not line:
            raise ValueError("PLY header has no end_header")
        words = line.decode("ascii", errors="replace").split()
        if not words or words[0] in ("comment", "obj_info"):
            continue
        if words[0] == "end_header":
            break
        if words[0] == "format":
            fmt = words[1]
        elif words[0] == "element":
            elements.append((words[1], int(words[2]), []))
        elif words[0] == "property":
            if not elements:
                raise ValueError("PLY property before any element")
            if words[1] == "list":
                elements[-1][2].append((words[-1], None))
            else:
                if words[1] not in _PLY_TYPES:
                    raise ValueError(f"unknown PLY property type {words[1]!r}")
                elements[-1][2].append((words[2], _PLY_TYPES[words[1]]))
    if fmt not in ("binary_little_endian", "binary_big_endian", "ascii"):
        raise ValueError(f"unsupported PLY format {fmt!r}")
    return fmt, elements, f.tell()


def _vertex_array(path):
    """The vertex element as a numpy structured array (binary: memory-mapped)."""
    with open(path, "rb") as f:
        fmt, elements, off = _read_header(f)
    endian = {"binary_little_endian": "<", "binary_big_endian": ">", "ascii": "<"}[fmt]
    skip_bytes, skip_lines = 0, 0
    for name, count, props in elements:
        if any(t is None for _, t in props):
            if name == "vertex":
                raise ValueError("list properties in the vertex element are not supported")
            if fmt != "ascii":
                raise ValueError(f"cannot skip element {name!r} with list properties "
                                 "in a binary PLY")
        dt = np.dtype([(p, endian + t) for p, t in props if t is not None])
        if name == "vertex" and count == 0:
            return np.zeros(0, dtype=dt)
        if name == "vertex":
            if fmt == "ascii":
                with open(path, "rb") as f:
                    f.seek(off)
                    for _ in range(skip_lines):
                        f.readline()
                    rows = [f.readline().split() for _ in range(count)]
                vals = np.array(rows, dtype=np.float64).reshape(count, len(props))
                out = np.zeros(count, dtype=dt)
                for i, (p, _) in enumerate(props):
                    out[p] = vals[:, i]
                return out
            return np.memmap(path, dtype=dt, mode="r", offset=off + skip_bytes, shape=(count,))
        skip_bytes += dt.itemsize * count
        skip_lines += count
    raise ValueError(f"{path}: no vertex element")


def _write_ply(path, names, records: np.ndarray) -> None:
    """Binary little-endian float32 PLY with one vertex element."""
    n = records.shape[0]
    header = ["ply", "format binary_little_endian 1.0", f"element vertex {n}"]
    header += [f"property float {nm}" for nm in names]
    header.append("end_header")
    Path(path).parent.mkdir(parents=True, exist_ok=True)
    with open(path, "wb") as f:
        f.write(("\n".join(header) + "\n").encode("ascii"))
        np.ascontiguousarray(records, dtype="<f4").tofile(f)


def _sh_layout(names, path):
    """(bases per channel P, degree) from the f_rest_ count (io.py:100-110)."""
    n_rest = len([n for n in names if n.startswith("f_rest_")])
    # A count that is not a whole number per channel would otherwise silently
    # drop a column and shift the channel-major layout.
    if n_rest % 3:
        raise ValueError(f"{path}: {n_rest} f_rest coefficients is not a whole "
                         f"number per channel")
    per_channel = n_rest // 3
    n_bases = per_channel + 1
    degree = int(round(n_bases ** 0.5)) - 1
    if (degree + 1) ** 2 != n_bases:
        raise ValueError(f"{path}: {n_rest} f_rest coefficients is not a whole SH degree")
    return per_channel, degree


def _field_names(per_channel):
    return (["x", "y", "z"] + [f"rot_{i}" for i in range(4)] + [f"scale_{i}" for i in range(3)]
            + ["opacity"] + [f"f_dc_{i}" for i in range(3)]
            + [f"f_rest_{i}" for i in range(3 * per_channel)])


# The INRIA column order this module writes (train.py:591-593).
def _inria_names(per_channel):
    return (["x", "y", "z"] + [f"f_dc_{i}" for i in range(3)]
            + [f"f_rest_{i}" for i in range(3 * per_channel)] + ["opacity"]
            + [f"scale_{i}" for i in range(3)] + [f"rot_{i}" for i in range(4)])


# -------------------------------------------------------------------- load

def load_ply(path: str | Path, device: str = "cpu", dtype=torch.float32) -> Splats:
    """Read a 3DGS .ply and de-parameterise it (io.py:89-123)."""
    v = _vertex_array(str(path))
    names = list(v.dtype.names)
    per_channel, degree = _sh_layout(names, path)
    fields = _field_names(per_channel)
    missing = [f for f in fields if f not in names]
    if missing:
        raise ValueError(f"{path}: missing properties {missing[:4]}")
    dev = torch.device(device)
    n = v.shape[0]
    if dev.type == "cuda":
        return _load_on_gpu(v, names, fields, per_channel, degree, dev, dtype)

    def col(nm):
        return np.asarray(v[nm], dtype=np.float64)

    means = np.stack([col("x"), col("y"), col("z")], axis=1)
    quats = np.stack([col(f"rot_{i}") for i in range(4)], axis=1)
    scales = np.exp(np.stack([col(f"scale_{i}") for i in range(3)], axis=1))
    opac = 1.0 / (1.0 + np.exp(-col("opacity")))
    sh = np.zeros((n, per_channel + 1, 3), np.float64)
    for c in range(3):
        sh[:, 0, c] = col(f"f_dc_{c}")
        for b in range(per_channel):
            sh[:, b + 1, c] = col(f"f_rest_{c * per_channel + b}")
    quats = quats / np.linalg.norm(quats, axis=1, keepdims=True).clip(1e-12)

    def t(a):
        return torch.as_tensor(a, dtype=dtype, device=dev)

    return Splats(t(means), t(quats), t(scales), t(opac), t(sh), degree)


def _load_on_gpu(v, names, fields, per_channel, degree, dev, dtype):
    lib = _lib.load()
    n = v.shape[0]
    if all(v.dtype[nm] == np.dtype("<f4") for nm in names):
        # The records as they lie in the file: (n, properties) float32.
        rec_np = np.asarray(v).view(np.float32).reshape(n, len(names))
        stride = len(names)
        columns = [names.index(f) for f in fields]
    else:
        # Mixed or big-endian columns: gather the needed ones as float32 first.
        rec_np = np.stack([np.asarray(v[f], dtype=np.float32) for f in fields], axis=1)
        stride = len(fields)
        columns = list(range(len(fields)))
    # One host copy out of the memory map (writable, as torch requires), one
    # upload.
    rec = torch.from_numpy(np.array(rec_np, dtype=np.float32, order="C")).to(dev)
    means = torch.empty(n, 3, device=dev)
    quats = torch.empty(n, 4, device=dev)
    scales = torch.empty(n, 3, device=dev)
    opac = torch.empty(n, device=dev)
    sh = torch.empty(n, per_channel + 1, 3, device=dev)
    _lib.check(lib.mg_ply_decode(n, rec.data_ptr() if n else None, stride,
                                 _lib.i32_array(columns), per_channel, means.data_ptr(),
                                 quats.data_ptr(), scales.data_ptr(), opac.data_ptr(),
                                 sh.data_ptr(), _lib.stream(rec)))
    out = [means, quats, scales, opac, sh]
    if dtype != torch.float32:
        out = [x.to(dtype) for x in out]
    return Splats(*out, degree)


# ------------------------------------------------------------------- write

def save_ply(splats: Splats, path: str | Path) -> None:
    """Write activated Splats in the INRIA convention (io.py:45-86): scales
    back to logs and opacities back to logits, clamped so fully transparent
    or opaque splats stay finite."""
    n, bases = len(splats), int(splats.sh.shape[1])
    per_channel = bases - 1
    sh = splats.sh.detach().cpu().float()
    opac = splats.opacities.detach().cpu().float().clamp(1e-6, 1.0 - 1e-6)
    cols = [splats.means.detach().cpu().float(), sh[:, 0, :],
            sh[:, 1:, :].permute(0, 2, 1).reshape(n, 3 * per_channel),
            torch.log(opac / (1.0 - opac))[:, None],
            torch.log(splats.scales.detach().cpu().float().clamp_min(1e-12)),
            splats.quats.detach().cpu().float()]
    _write_ply(path, _inria_names(per_channel), torch.cat(cols, dim=1).numpy())


@torch.no_grad()
def export_ply(p: dict, path: str, filter_3d=None) -> None:
    """Write the trainer's parameters (train.py:582-624): pre-activation
    values as they are, SH from ``sh_dc`` + ``sh_rest`` (or ``sh``) at degree
    3 (45 f_rest), and with ``filter_3d`` Mip-Splatting's 3D filter baked into
    the written scales and opacities. On a ROCm device the records are built
    by one kernel and copied to the host once."""
    n = len(p["means"])
    per_channel = 15
    names = _inria_names(per_channel)
    dev = p["means"].device
    if dev.type == "cuda":
        lib = _lib.load()
        cols = [names.index(f) for f in _field_names(per_channel)]
        rec = torch.empty(n, len(names), device=dev)
        # Every operand on the parameters' device, contiguous float32: the
        # kernel takes raw device pointers.
        c = lambda t: t.detach().to(dev).contiguous().float()  # noqa: E731
        split = "sh_dc" in p
        sh = None if split else c(p["sh"])
        dc = c(p["sh_dc"]) if split else None
        rest = c(p["sh_rest"]) if split else None
        bases = (1 + rest.shape[1]) if split else sh.shape[1]
        if bases < 16:
            raise ValueError(f"export_ply writes degree 3: need 16 SH bases, have {bases}")
        f = None if filter_3d is None else c(filter_3d[:n])
        m, q, ls, lg = c(p["means"]), c(p["quats"]), c(p["log_scales"]), c(p["logit_opac"])
        _lib.check(lib.mg_ply_encode(
            n, m.data_ptr(), q.data_ptr(), ls.data_ptr(), lg.data_ptr(),
            None if dc is None else dc.data_ptr(), None if rest is None else rest.data_ptr(),
            None if sh is None else sh.data_ptr(), bases,
            None if f is None else f.data_ptr(), len(names), _lib.i32_array(cols), per_channel,
            rec.data_ptr(), _lib.stream(rec)))
        _write_ply(path, names, rec.cpu().numpy())
        return
    from .mipfilter import apply_3d_filter

    sh = (torch.cat([p["sh_dc"], p["sh_rest"]], dim=1) if "sh_dc" in p else p["sh"]).detach()
    logit = p["logit_opac"].detach()
    log_scales = p["log_scales"].detach()
    if filter_3d is not None:
        sc, op = apply_3d_filter(torch.exp(log_scales), torch.sigmoid(logit),
                                 filter_3d[:n].detach())
        log_scales = torch.log(sc.clamp_min(1e-12))
        op = op.clamp(1e-6, 1.0 - 1e-6)
        logit = torch.log(op / (1.0 - op))
    rec = torch.cat([p["means"].detach(), sh[:, 0, :],
                     sh[:, 1:16, :].permute(0, 2, 1).reshape(n, 45), logit[:, None],
                     log_scales, p["quats"].detach()], dim=1)
    _write_ply(path, names, rec.float().cpu().numpy())
