"""PLY I/O of metal-gauss_amd/io.py on the CPU.

Every file here is assembled column by column by oracle/ply_ref.py, a
spec-level PLY writer that shares no code with the package. Columns hold
stored (parameterised) INRIA values; the decoded values the loader must
return are fixed in advance in DECODE_CASES below. Those known answers are
the ones the reference's own PLY tests rely on (tests/test_io.py of
nandometzger/metal-gauss): logit opacities, log scales, unnormalised and
zero quaternions, positions, the DC band and the channel-major f_rest
layout, the SH degree implied by the coefficient count and the two
refusals. Also ascii and big-endian bodies, elements before the vertex
element, property order, and the writer checked by the spec-level reader.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ply_ref

DECODED = ("means", "quats", "scales", "opacities", "sh")


def _stored(n, *, xyz=None, rot=None, log_scale=None, logit=None, dc=None, rest=None):
    """INRIA columns for n splats in stored space. Unset groups are benign:
    origin, identity rotation, unit scale, opacity 0.5, black DC, no f_rest.
    ``rest`` is (n, bands-1, 3) in (splat, band, channel) order and is laid
    out channel-major, f_rest_[c * per_channel + band - 1]."""
    f32 = np.float32
    xyz = np.zeros((n, 3), f32) if xyz is None else np.asarray(xyz, f32)
    rot = np.tile(f32([1, 0, 0, 0]), (n, 1)) if rot is None else np.asarray(rot, f32)
    log_scale = np.zeros((n, 3), f32) if log_scale is None else np.asarray(log_scale, f32)
    logit = np.zeros(n, f32) if logit is None else np.asarray(logit, f32)
    dc = np.zeros((n, 3), f32) if dc is None else np.asarray(dc, f32)
    cols = {a: xyz[:, i] for i, a in enumerate("xyz")}
    cols.update({f"f_dc_{c}": dc[:, c] for c in range(3)})
    if rest is not None:
        rest = np.asarray(rest, f32)
        per = rest.shape[1]
        cols.update({f"f_rest_{c * per + b}": rest[:, b, c]
                     for c in range(3) for b in range(per)})
    cols["opacity"] = logit
    cols.update({f"scale_{i}": log_scale[:, i] for i in range(3)})
    cols.update({f"rot_{i}": rot[:, i] for i in range(4)})
    return cols


def _file(tmp_path, name, cols, fmt="binary_little_endian", alphabetical=False, extra=()):
    if alphabetical:
        cols = dict(sorted(cols.items()))
    path = tmp_path / name
    path.write_bytes(ply_ref.write_ply_bytes(cols, fmt=fmt, extra_elements=extra))
    return path


def _read(path, **kw):
    from metal_gauss_amd.io import load_ply

    return load_ply(path, **kw)


def _tagged_rest(n, per):
    """f_rest values that name their own place: 1000 * splat + stored column
    index, so a transposed layout shows up as wrong numbers."""
    col = np.arange(per)[None, :, None] + per * np.arange(3)[None, None, :]
    return (1000.0 * np.arange(n)[:, None, None] + col).astype(np.float32)


# --------------------------------------------------------- known answers

_P = np.array([0.5, 0.9, 0.1])
_S = np.array([[0.01, 0.02, 0.03], [1.0, 1.0, 1.0], [0.5, 0.25, 0.125]])
_Q = np.array([[5.0, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0, 0.1], [1.0, 1.0, 1.0, 1.0]])
_M = np.array([[0.0, 1.0, 2.0], [-3.5, 4.25, 5.125], [1e3, -1e3, 0.0]])
_DC = np.array([[0.1, 0.2, 0.3], [1.0, 2.0, 3.0], [-1.0, -2.0, -3.0]])

# (id, stored columns, decoded field, expected value, relative tolerance)
DECODE_CASES = [
    ("opacity_from_logit", dict(logit=np.log(_P / (1 - _P))), "opacities", _P, 1e-6),
    ("scale_from_log", dict(log_scale=np.log(_S)), "scales", _S, 1e-6),
    ("quaternion_normalised", dict(rot=_Q), "quats",
     _Q / np.linalg.norm(_Q, axis=1, keepdims=True), 1e-6),
    ("position_as_stored", dict(xyz=_M), "means", _M, 0.0),
    ("dc_band_per_channel", dict(dc=_DC, rest=_tagged_rest(3, 15)), "sh[:, 0]", _DC, 0.0),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_decoded_value(tmp_path, case):
    name, stored, field, want, rel = case
    sp = _read(_file(tmp_path, f"{name}.ply", _stored(3, **stored)))
    got = sp.sh[:, 0].numpy() if field == "sh[:, 0]" else getattr(sp, field).numpy()
    assert got == pytest.approx(want.astype(np.float32), rel=rel, abs=0 if rel else 1e-12)


def test_opacities_stay_probabilities_for_extreme_logits(tmp_path):
    sp = _read(_file(tmp_path, "x.ply", _stored(3, logit=[-30.0, 0.0, 12.5])))
    op = sp.opacities
    assert torch.isfinite(op).all() and bool(((op > 0) & (op < 1)).all())
    assert float(op[1]) == 0.5


def test_decoded_scales_are_positive_and_quaternions_unit(tmp_path):
    sp = _read(_file(tmp_path, "u.ply", _stored(3, log_scale=np.log(_S), rot=_Q)))
    assert bool((sp.scales > 0).all())
    assert sp.quats.norm(dim=1).numpy() == pytest.approx(np.ones(3), rel=1e-6)


def test_an_all_zero_quaternion_decodes_finite(tmp_path):
    rot = np.array([[0.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0]])
    sp = _read(_file(tmp_path, "z.ply", _stored(2, rot=rot)))
    assert torch.isfinite(sp.quats).all()


def test_rest_coefficients_land_channel_major(tmp_path):
    sp = _read(_file(tmp_path, "r.ply", _stored(3, rest=_tagged_rest(3, 15))))
    assert tuple(sp.sh.shape) == (3, 16, 3)
    band = torch.arange(1, 16)[None, :, None]
    chan = torch.arange(3)[None, None, :]
    splat = torch.arange(3)[:, None, None]
    want = (1000 * splat + 15 * chan + band - 1).float()
    assert torch.equal(sp.sh[:, 1:, :], want)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_degree_from_the_number_of_rest_columns(tmp_path, degree):
    bands = (degree + 1) ** 2
    rest = None if degree == 0 else _tagged_rest(3, bands - 1)
    sp = _read(_file(tmp_path, f"g{degree}.ply", _stored(3, dc=_DC, rest=rest)))
    assert sp.sh_degree == degree and tuple(sp.sh.shape) == (3, bands, 3)
    assert sp.sh[:, 0].numpy() == pytest.approx(_DC.astype(np.float32))


@pytest.mark.parametrize("per_channel_cols,message", [
    (None, "whole SH degree"),          # 2 bands of rest per channel: 3 bands in all
    (46, "whole number per channel"),   # 46 rest columns do not split over 3 channels
])
def test_rest_counts_that_are_not_a_degree_are_refused(tmp_path, per_channel_cols, message):
    if per_channel_cols is None:
        cols = _stored(2, rest=np.zeros((2, 2, 3)))
    else:
        cols = _stored(2)
        cols.update({f"f_rest_{i}": np.zeros(2, np.float32) for i in range(per_channel_cols)})
    with pytest.raises(ValueError, match=message):
        _read(_file(tmp_path, "bad.ply", cols))


def _mixed(n=3, per=15):
    return dict(xyz=np.arange(3 * n, dtype=np.float32).reshape(n, 3) * 0.25,
                rot=np.arange(4 * n, dtype=np.float32).reshape(n, 4) + 1.0,
                log_scale=np.linspace(-4, 0, 3 * n, dtype=np.float32).reshape(n, 3),
                logit=np.linspace(-2, 2, n, dtype=np.float32),
                dc=np.full((n, 3), 0.1, np.float32), rest=_tagged_rest(n, per))


def test_header_order_does_not_change_the_result(tmp_path):
    a = _read(_file(tmp_path, "o.ply", _stored(3, **_mixed())))
    b = _read(_file(tmp_path, "s.ply", _stored(3, **_mixed()), alphabetical=True))
    assert a.sh_degree == b.sh_degree
    for f in DECODED:
        assert torch.equal(getattr(a, f), getattr(b, f)), f


@pytest.mark.parametrize("fmt", ["ascii", "binary_big_endian"])
def test_every_body_format_reads_alike(tmp_path, fmt):
    """The reference reads through plyfile, which takes all three formats."""
    cols = _stored(3, **_mixed(per=8))
    a = _read(_file(tmp_path, "le.ply", cols))
    b = _read(_file(tmp_path, "other.ply", cols, fmt=fmt))
    for f in DECODED:
        assert torch.allclose(getattr(a, f), getattr(b, f), rtol=1e-6, atol=0), f


def test_leading_non_vertex_elements_are_skipped(tmp_path):
    cams = [("camera", 2, [("fx", "float"), ("id", "uchar")], [[500.0, 1], [600.0, 2]])]
    logit = np.array([1.0, 2.0, 3.0])
    for fmt in ("binary_little_endian", "ascii"):
        sp = _read(_file(tmp_path, f"c_{fmt}.ply", _stored(3, xyz=np.ones((3, 3)), logit=logit),
                         fmt=fmt, extra=cams))
        assert sp.means.numpy() == pytest.approx(np.ones((3, 3)))
        want = np.array([1.0 / (1.0 + math.exp(-v)) for v in logit])
        assert sp.opacities.numpy() == pytest.approx(want, rel=1e-6)


def test_loader_agrees_with_the_spec_level_decode(tmp_path):
    """Random stored values through the package's reader and ply_ref.decode."""
    rng = np.random.default_rng(0)
    n = 200
    cols = _stored(n, xyz=rng.standard_normal((n, 3)), rot=rng.standard_normal((n, 4)),
                   log_scale=rng.standard_normal((n, 3)) - 3, logit=3 * rng.standard_normal(n),
                   dc=rng.standard_normal((n, 3)), rest=rng.standard_normal((n, 15, 3)))
    path = _file(tmp_path, "rand.ply", cols)
    sp = _read(path)
    want = ply_ref.decode(ply_ref.read_ply_bytes(path.read_bytes()))
    for f, w in zip(DECODED, want[:5]):
        assert np.array_equal(getattr(sp, f).numpy(), w.astype(np.float32)), f
    assert sp.sh_degree == want[5]


def test_splats_container_subset_len_and_to(tmp_path):
    from metal_gauss_amd.io import Splats

    sp = _read(_file(tmp_path, "c.ply", _stored(3, rest=_tagged_rest(3, 15))))
    pick = torch.tensor([2, 0])
    sub = sp.subset(pick)
    assert (len(sp), len(sub)) == (3, 2) and sub.sh_degree == sp.sh_degree
    for f in DECODED:
        assert torch.equal(getattr(sub, f), getattr(sp, f)[pick])
    moved = sp.to("cpu")
    assert isinstance(moved, Splats) and moved.sh_degree == sp.sh_degree


def test_requested_dtype_is_returned(tmp_path):
    sp = _read(_file(tmp_path, "d.ply", _stored(3, rest=_tagged_rest(3, 15))),
               dtype=torch.float64)
    assert all(getattr(sp, f).dtype is torch.float64 and getattr(sp, f).device.type == "cpu"
               for f in DECODED)


# --------------------------------------------------------------- writing

def _random_splats(n=32, degree=3, seed=0):
    from metal_gauss_amd.io import Splats

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, 4, generator=g)
    return Splats(means=torch.randn(n, 3, generator=g), quats=q / q.norm(dim=1, keepdim=True),
                  scales=torch.rand(n, 3, generator=g) * 0.1 + 1e-3,
                  opacities=torch.rand(n, generator=g),
                  sh=torch.randn(n, (degree + 1) ** 2, 3, generator=g), sh_degree=degree)


@pytest.mark.parametrize("degree", [0, 3])
def test_save_then_load_returns_the_splats(tmp_path, degree):
    from metal_gauss_amd.io import save_ply

    sp = _random_splats(degree=degree)
    save_ply(sp, tmp_path / "rt.ply")
    back = _read(tmp_path / "rt.ply")
    assert back.sh_degree == degree
    tol = dict(means=(0, 1e-6), quats=(0, 1e-6), scales=(1e-5, 1e-7), opacities=(0, 1e-5),
               sh=(0, 1e-6))
    for f, (rtol, atol) in tol.items():
        assert torch.allclose(getattr(back, f), getattr(sp, f), rtol=rtol, atol=atol), f


def test_opacities_of_exactly_zero_and_one_survive_a_save(tmp_path):
    from metal_gauss_amd.io import save_ply

    sp = _random_splats(n=2)
    sp.opacities[:] = torch.tensor([0.0, 1.0])
    save_ply(sp, tmp_path / "edge.ply")
    op = _read(tmp_path / "edge.ply").opacities
    assert torch.isfinite(op).all() and float(op[0]) < 1e-4 and float(op[1]) > 1.0 - 1e-4


def test_saved_columns_follow_the_inria_convention(tmp_path):
    """Names, stored values and the channel-major f_rest, as read by the
    spec-level reader."""
    from metal_gauss_amd.io import save_ply

    sp = _random_splats()
    save_ply(sp, tmp_path / "cols.ply")
    cols = ply_ref.read_ply_bytes((tmp_path / "cols.ply").read_bytes())
    need = ({"x", "y", "z", "opacity"} | {f"scale_{i}" for i in range(3)} |
            {f"rot_{i}" for i in range(4)} | {f"f_dc_{i}" for i in range(3)} |
            {f"f_rest_{i}" for i in range(45)})
    assert need <= set(cols)
    sh = sp.sh.numpy()
    # channel 1, band 2 is stored at column 1 * 15 + (2 - 1)
    assert np.array_equal(cols["f_rest_16"].astype(np.float32), sh[:, 2, 1])
    assert np.allclose(cols["scale_1"], np.log(sp.scales[:, 1].numpy()), atol=1e-6)


def test_export_from_trainer_parameters_matches_the_restated_export(tmp_path):
    """train.export_ply's columns (ply_ref.encode_export), with and without
    the baked 3D filter, read back by the spec-level reader."""
    from metal_gauss_amd.io import export_ply

    g = torch.Generator().manual_seed(3)
    n = 50
    p = {"means": torch.randn(n, 3, generator=g), "log_scales": torch.randn(n, 3, generator=g) - 4,
         "quats": torch.randn(n, 4, generator=g), "logit_opac": torch.randn(n, generator=g),
         "sh_dc": torch.randn(n, 1, 3, generator=g), "sh_rest": torch.randn(n, 15, 3, generator=g)}
    f3d = torch.rand(n, generator=g) * 0.02
    for filt in (None, f3d):
        export_ply(p, str(tmp_path / "exp.ply"), filter_3d=filt)
        got = ply_ref.read_ply_bytes((tmp_path / "exp.ply").read_bytes())
        want = ply_ref.encode_export(p, filt)
        for k, w in want.items():
            assert np.array_equal(got[k].astype(np.float32), w), k
