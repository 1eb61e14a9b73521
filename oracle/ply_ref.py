"""Restatement of the 3DGS .ply convention. TEST INFRASTRUCTURE ONLY.

* ``write_ply_bytes`` / ``read_ply_bytes`` build and parse PLY files value by
  value with ``struct``, from the PLY specification (an ascii header of
  ``element`` / ``property`` lines, then records in binary little-endian,
  binary big-endian or ascii). They share no code with the package's
  numpy-based reader and writer, so a layout mistake on either side shows.
* ``decode`` restates metal_gauss/io.py:89-123 (float64 numpy: exp, sigmoid,
  quaternion normalisation clamped at 1e-12, channel-major f_rest).
* ``encode_export`` restates train.export_ply (train.py:582-624) in float32
  torch, with the optional Mip 3D filter bake.

Pinned by tests/test_io.py: the reference's own known answers
(tests/test_io.py of the reference: logit and log de-parameterisation,
quaternion normalisation and the zero quaternion, channel-major f_rest,
degree inference, the whole-degree and whole-number-per-channel refusals,
header order independence) hold for ``decode`` on files from
``write_ply_bytes``, and ``read_ply_bytes`` reads back what it wrote in all
three formats.
"""

from __future__ import annotations

import struct

import numpy as np
import torch

_FMT = {"float": "f", "double": "d", "uchar": "B", "char": "b", "short": "h", "ushort": "H",
        "int": "i", "uint": "I"}


def write_ply_bytes(cols: dict, fmt: str = "binary_little_endian", types: dict | None = None,
                    extra_elements=()) -> bytes:
    """A PLY file with one vertex element holding ``cols`` (name -> 1-D values,
    in dict order). ``types`` maps a name to a PLY type (default float).
    ``extra_elements``: (name, count, [(prop, type)], rows) written before the
    vertex element, to check that a reader skips them."""
    types = types or {}
    names = list(cols)
    n = len(next(iter(cols.values()))) if cols else 0
    hdr = ["ply", f"format {fmt} 1.0", "comment written by oracle/ply_ref.py"]
    for name, count, props, _ in extra_elements:
        hdr.append(f"element {name} {count}")
        hdr += [f"property {t} {p}" for p, t in props]
    hdr.append(f"element vertex {n}")
    hdr += [f"property {types.get(nm, 'float')} {nm}" for nm in names]
    hdr.append("end_header")
    out = bytearray(("\n".join(hdr) + "\n").encode("ascii"))
    end = "<" if fmt == "binary_little_endian" else ">"

    def rows_bytes(props, rows):
        b = bytearray()
        for row in rows:
            if fmt == "ascii":
                b += (" ".join(repr(float(x)) if t in ("float", "double") else str(int(x))
                               for (_, t), x in zip(props, row)) + "\n").encode("ascii")
            else:
                for (_, t), x in zip(props, row):
                    b += struct.pack(end + _FMT[t], x)
        return b

    for _, _, props, rows in extra_elements:
        out += rows_bytes(props, rows)
    props = [(nm, types.get(nm, "float")) for nm in names]
    vrows = [[cols[nm][i] for nm in names] for i in range(n)]
    out += rows_bytes(props, vrows)
    return bytes(out)


def read_ply_bytes(data: bytes) -> dict:
    """Vertex columns (name -> float64 array) of a PLY file, value by value."""
    head, _, body = data.partition(b"end_header\n")
    lines = head.decode("ascii").splitlines()
    fmt = next(l.split()[1] for l in lines if l.startswith("format"))
    elements = []
    for l in lines:
        w = l.split()
        if w and w[0] == "element":
            elements.append([w[1], int(w[2]), []])
        elif w and w[0] == "property":
            elements[-1][2].append((w[2], w[1]))
    end = "<" if fmt == "binary_little_endian" else ">"
    pos = 0
    text = body.decode("ascii").splitlines() if fmt == "ascii" else None
    line = 0
    for name, count, props in elements:
        vals = {p: [] for p, _ in props}
        for _ in range(count):
            if fmt == "ascii":
                row = text[line].split()
                line += 1
                for (p, t), x in zip(props, row):
                    vals[p].append(float(x))
            else:
                for p, t in props:
                    (x,) = struct.unpack_from(end + _FMT[t], body, pos)
                    pos += struct.calcsize(_FMT[t])
                    vals[p].append(float(x))
        if name == "vertex":
            return {p: np.array(v, dtype=np.float64) for p, v in vals.items()}
    raise ValueError("no vertex element")


def decode(cols: dict):
    """io.py:89-123 on vertex columns -> (means, quats, scales, opac, sh, degree)."""
    def col(n):
        return np.asarray(cols[n], dtype=np.float64)

    n_rest = len([n for n in cols if n.startswith("f_rest_")])
    if n_rest % 3:
        raise ValueError(f"{n_rest} f_rest coefficients is not a whole number per channel")
    per_channel = n_rest // 3
    nb = per_channel + 1
    deg = int(round(nb ** 0.5)) - 1
    if (deg + 1) ** 2 != nb:
        raise ValueError(f"{n_rest} f_rest coefficients is not a whole SH degree")
    means = np.stack([col("x"), col("y"), col("z")], axis=1)
    quats = np.stack([col(f"rot_{i}") for i in range(4)], axis=1)
    scales = np.exp(np.stack([col(f"scale_{i}") for i in range(3)], axis=1))
    opac = 1.0 / (1.0 + np.exp(-col("opacity")))
    sh = np.zeros((len(means), nb, 3))
    for c in range(3):
        sh[:, 0, c] = col(f"f_dc_{c}")
        for b in range(per_channel):
            sh[:, b + 1, c] = col(f"f_rest_{c * per_channel + b}")
    quats = quats / np.linalg.norm(quats, axis=1, keepdims=True).clip(1e-12)
    return means, quats, scales, opac, sh, deg


def encode_export(p: dict, filter_3d=None) -> dict:
    """train.py:582-624 in float32 torch -> vertex columns (name -> float32)."""
    n = len(p["means"])
    sh = (torch.cat([p["sh_dc"], p["sh_rest"]], dim=1) if "sh_dc" in p else p["sh"]).float()
    logit = p["logit_opac"].float()
    log_scales = p["log_scales"].float()
    if filter_3d is not None:
        f2 = (filter_3d[:n].float() ** 2).unsqueeze(-1)
        s2 = torch.exp(log_scales) ** 2
        s2f = s2 + f2
        coef = torch.sqrt((s2.prod(dim=-1) / s2f.prod(dim=-1)).clamp(0.0, 1.0))
        sc, op = torch.sqrt(s2f), torch.sigmoid(logit) * coef
        log_scales = torch.log(sc.clamp_min(1e-12))
        op = op.clamp(1e-6, 1.0 - 1e-6)
        logit = torch.log(op / (1.0 - op))
    cols = {}
    m = p["means"].float()
    for i, nm in enumerate("xyz"):
        cols[nm] = m[:, i].numpy()
    for c in range(3):
        cols[f"f_dc_{c}"] = sh[:, 0, c].numpy()
    for c in range(3):
        for b in range(15):
            cols[f"f_rest_{c * 15 + b}"] = sh[:, b + 1, c].numpy()
    cols["opacity"] = logit.numpy()
    for i in range(3):
        cols[f"scale_{i}"] = log_scales[:, i].numpy()
    for i in range(4):
        cols[f"rot_{i}"] = p["quats"].float()[:, i].numpy()
    return cols
