"""PLY I/O (metal-gauss_amd/io.py) on the CPU, in the style of the reference's
tests/test_io.py: every file is built value by value from the PLY
specification by oracle/ply_ref.py (no shared code with the package), in
stored (parameterised) space, and the de-parameterised values that must come
back are known in advance. Also ascii and big-endian bodies, skipped
elements, and the writer checked by the spec-level reader."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ply_ref

FIELDS = ("means", "quats", "scales", "opacities", "sh")


def write_ply(path, *, n=3, means=None, quats=None, log_scales=None, logit_opac=None,
              sh_dc=None, sh_rest=None, sort_properties=False, fmt="binary_little_endian",
              extra_elements=()):
    """tests/test_io.py:33-87 of the reference, with the spec-level writer."""
    means = np.zeros((n, 3), np.float32) if means is None else np.asarray(means, np.float32)
    quats = (np.tile([1.0, 0.0, 0.0, 0.0], (n, 1)).astype(np.float32) if quats is None
             else np.asarray(quats, np.float32))
    log_scales = (np.zeros((n, 3), np.float32) if log_scales is None
                  else np.asarray(log_scales, np.float32))
    logit_opac = (np.zeros(n, np.float32) if logit_opac is None
                  else np.asarray(logit_opac, np.float32))
    sh_dc = np.zeros((n, 3), np.float32) if sh_dc is None else np.asarray(sh_dc, np.float32)
    cols = {}
    for i, name in enumerate("xyz"):
        cols[name] = means[:, i]
    for c in range(3):
        cols[f"f_dc_{c}"] = sh_dc[:, c]
    if sh_rest is not None:
        sh_rest = np.asarray(sh_rest, np.float32)
        per = sh_rest.shape[1]
        for c in range(3):
            for b in range(per):
                cols[f"f_rest_{c * per + b}"] = sh_rest[:, b, c]
    cols["opacity"] = logit_opac
    for i in range(3):
        cols[f"scale_{i}"] = log_scales[:, i]
    for i in range(4):
        cols[f"rot_{i}"] = quats[:, i]
    if sort_properties:
        cols = {k: cols[k] for k in sorted(cols)}
    path.write_bytes(ply_ref.write_ply_bytes(cols, fmt=fmt, extra_elements=extra_elements))
    return path


def full_sh(n, per_channel):
    """Each coefficient encodes where it must land: 1000*splat + stored index."""
    idx = np.arange(per_channel)[None, :, None] + per_channel * np.arange(3)[None, None, :]
    return (1000.0 * np.arange(n)[:, None, None] + idx).astype(np.float32)


def load(path, **kw):
    from metal_gauss_amd.io import load_ply
    return load_ply(path, **kw)


def test_opacity_is_read_as_a_logit(tmp_path):
    want = np.array([0.5, 0.9, 0.1], np.float32)
    sp = load(write_ply(tmp_path / "o.ply", logit_opac=np.log(want / (1.0 - want))))
    assert sp.opacities.tolist() == pytest.approx(want.tolist(), rel=1e-6)


def test_opacity_is_always_a_probability(tmp_path):
    sp = load(write_ply(tmp_path / "o.ply", logit_opac=np.array([-30.0, 0.0, 12.5], np.float32)))
    assert (sp.opacities > 0).all() and (sp.opacities < 1).all()
    assert sp.opacities[1].item() == 0.5
    assert torch.isfinite(sp.opacities).all()


def test_scale_is_read_as_a_log(tmp_path):
    want = np.array([[0.01, 0.02, 0.03], [1.0, 1.0, 1.0], [0.5, 0.25, 0.125]], np.float32)
    sp = load(write_ply(tmp_path / "s.ply", log_scales=np.log(want)))
    assert sp.scales.numpy() == pytest.approx(want, rel=1e-6)
    assert (sp.scales > 0).all()


def test_quaternion_is_normalised(tmp_path):
    stored = np.array([[5.0, 0.0, 0.0, 0.0], [0.0, 0.0, 0.0, 0.1], [1.0, 1.0, 1.0, 1.0]],
                      np.float32)
    sp = load(write_ply(tmp_path / "q.ply", quats=stored))
    assert sp.quats.norm(dim=1).tolist() == pytest.approx([1.0, 1.0, 1.0], rel=1e-6)
    unit = stored / np.linalg.norm(stored, axis=1, keepdims=True)
    assert sp.quats.numpy() == pytest.approx(unit, rel=1e-6)


def test_zero_quaternion_does_not_become_nan(tmp_path):
    stored = np.array([[0.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0]], np.float32)
    sp = load(write_ply(tmp_path / "q0.ply", n=2, quats=stored))
    assert torch.isfinite(sp.quats).all()


def test_positions_pass_through_unchanged(tmp_path):
    means = np.array([[0.0, 1.0, 2.0], [-3.5, 4.25, 5.125], [1e3, -1e3, 0.0]], np.float32)
    sp = load(write_ply(tmp_path / "m.ply", means=means))
    assert sp.means.numpy() == pytest.approx(means)


def test_dc_band_is_the_degree_zero_term_per_channel(tmp_path):
    dc = np.array([[0.1, 0.2, 0.3], [1.0, 2.0, 3.0], [-1.0, -2.0, -3.0]], np.float32)
    sp = load(write_ply(tmp_path / "dc.ply", sh_dc=dc, sh_rest=full_sh(3, 15)))
    assert sp.sh[:, 0, :].numpy() == pytest.approx(dc)


def test_f_rest_is_channel_major(tmp_path):
    sp = load(write_ply(tmp_path / "r.ply", sh_rest=full_sh(3, 15)))
    assert sp.sh.shape == (3, 16, 3)
    for n in range(3):
        for c in range(3):
            for b in range(1, 16):
                assert sp.sh[n, b, c].item() == 1000.0 * n + c * 15 + (b - 1)
    assert sp.sh[0, 1, 1].item() == 15.0


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_sh_degree_follows_the_coefficient_count(tmp_path, degree):
    nb = (degree + 1) ** 2
    sp = load(write_ply(tmp_path / f"d{degree}.ply",
                        sh_rest=None if degree == 0 else full_sh(3, nb - 1)))
    assert sp.sh_degree == degree and sp.sh.shape == (3, nb, 3)


def test_degree_zero_ply_has_no_f_rest_at_all(tmp_path):
    dc = np.array([[0.1, 0.2, 0.3], [1.0, 2.0, 3.0], [-1.0, -2.0, -3.0]], np.float32)
    sp = load(write_ply(tmp_path / "d0.ply", sh_dc=dc))
    assert sp.sh_degree == 0 and sp.sh.shape == (3, 1, 3)
    assert sp.sh[:, 0, :].numpy() == pytest.approx(dc)


def test_non_square_f_rest_count_is_rejected(tmp_path):
    path = write_ply(tmp_path / "bad.ply", sh_rest=np.zeros((3, 2, 3), np.float32))
    with pytest.raises(ValueError, match="whole SH degree"):
        load(path)


def test_f_rest_count_must_be_divisible_by_three(tmp_path):
    cols = {nm: np.zeros(2, np.float32) for nm in
            ["x", "y", "z", "opacity"] + [f"scale_{i}" for i in range(3)]
            + [f"rot_{i}" for i in range(4)] + [f"f_dc_{i}" for i in range(3)]
            + [f"f_rest_{i}" for i in range(46)]}
    cols["rot_0"][:] = 1.0
    (tmp_path / "ragged.ply").write_bytes(ply_ref.write_ply_bytes(cols))
    with pytest.raises(ValueError, match="whole number per channel"):
        load(tmp_path / "ragged.ply")


def test_property_order_in_the_file_does_not_matter(tmp_path):
    kw = dict(means=np.arange(9, dtype=np.float32).reshape(3, 3),
              quats=np.arange(12, dtype=np.float32).reshape(3, 4) + 1.0,
              log_scales=np.linspace(-4, 0, 9, dtype=np.float32).reshape(3, 3),
              logit_opac=np.array([-2.0, 0.0, 2.0], np.float32),
              sh_dc=np.array([[0.1, 0.2, 0.3]] * 3, np.float32), sh_rest=full_sh(3, 15))
    ordered = load(write_ply(tmp_path / "ordered.ply", **kw))
    alpha = load(write_ply(tmp_path / "alpha.ply", sort_properties=True, **kw))
    assert alpha.sh_degree == ordered.sh_degree
    for f in FIELDS:
        assert torch.equal(getattr(ordered, f), getattr(alpha, f)), f


@pytest.mark.parametrize("fmt", ["ascii", "binary_big_endian"])
def test_ascii_and_big_endian_bodies_read_the_same(tmp_path, fmt):
    """plyfile (the reference's reader) reads all three PLY formats."""
    kw = dict(means=np.arange(9, dtype=np.float32).reshape(3, 3) * 0.25,
              quats=np.arange(12, dtype=np.float32).reshape(3, 4) + 1.0,
              log_scales=np.linspace(-4, 0, 9, dtype=np.float32).reshape(3, 3),
              logit_opac=np.array([-2.0, 0.0, 2.0], np.float32), sh_rest=full_sh(3, 8))
    a = load(write_ply(tmp_path / "le.ply", **kw))
    b = load(write_ply(tmp_path / "x.ply", fmt=fmt, **kw))
    for f in FIELDS:
        assert torch.allclose(getattr(a, f), getattr(b, f), rtol=1e-6, atol=0), f


def test_elements_before_the_vertex_element_are_skipped(tmp_path):
    extra = [("camera", 2, [("fx", "float"), ("id", "uchar")], [[500.0, 1], [600.0, 2]])]
    kw = dict(means=np.ones((3, 3), np.float32), logit_opac=np.array([1.0, 2.0, 3.0], np.float32))
    for fmt in ("binary_little_endian", "ascii"):
        sp = load(write_ply(tmp_path / f"e_{fmt}.ply", fmt=fmt, extra_elements=extra, **kw))
        assert sp.means.numpy() == pytest.approx(np.ones((3, 3)))
        assert sp.opacities.numpy() == pytest.approx(1.0 / (1.0 + np.exp(-np.array([1, 2, 3.0]))),
                                                     rel=1e-6)


def test_loader_equals_the_restated_decode(tmp_path):
    """Random fields through both: the package's reader and ply_ref.decode."""
    g = np.random.default_rng(0)
    n = 200
    kw = dict(n=n, means=g.standard_normal((n, 3)), quats=g.standard_normal((n, 4)),
              log_scales=g.standard_normal((n, 3)) - 3, logit_opac=g.standard_normal(n) * 3,
              sh_dc=g.standard_normal((n, 3)), sh_rest=g.standard_normal((n, 15, 3)))
    path = write_ply(tmp_path / "rand.ply", **kw)
    sp = load(path)
    want = ply_ref.decode(ply_ref.read_ply_bytes(path.read_bytes()))
    for got, w in zip((sp.means, sp.quats, sp.scales, sp.opacities, sp.sh), want[:5]):
        assert np.array_equal(got.numpy(), w.astype(np.float32))
    assert sp.sh_degree == want[5]


def test_subset_and_len_keep_the_degree(tmp_path):
    from metal_gauss_amd.io import Splats

    sp = load(write_ply(tmp_path / "sub.ply", n=3, sh_rest=full_sh(3, 15)))
    assert len(sp) == 3
    sub = sp.subset(torch.tensor([2, 0]))
    assert len(sub) == 2 and sub.sh_degree == sp.sh_degree
    for f in FIELDS:
        assert torch.equal(getattr(sub, f), getattr(sp, f)[torch.tensor([2, 0])])
    same = sp.to("cpu")
    assert isinstance(same, Splats) and same.sh_degree == sp.sh_degree


def test_dtype_and_device_are_honoured(tmp_path):
    sp = load(write_ply(tmp_path / "t.ply", sh_rest=full_sh(3, 15)), dtype=torch.float64)
    for f in FIELDS:
        t = getattr(sp, f)
        assert t.dtype is torch.float64 and t.device.type == "cpu"


def _synthetic_splats(n=32, degree=3, seed=0):
    from metal_gauss_amd.io import Splats

    g = torch.Generator().manual_seed(seed)
    return Splats(means=torch.randn(n, 3, generator=g),
                  quats=torch.nn.functional.normalize(torch.randn(n, 4, generator=g), dim=1),
                  scales=torch.rand(n, 3, generator=g) * 0.1 + 1e-3,
                  opacities=torch.rand(n, generator=g),
                  sh=torch.randn(n, (degree + 1) ** 2, 3, generator=g), sh_degree=degree)


@pytest.mark.parametrize("degree", [0, 3])
def test_a_written_file_reads_back_as_the_same_splats(tmp_path, degree):
    from metal_gauss_amd.io import save_ply

    sp = _synthetic_splats(degree=degree)
    save_ply(sp, tmp_path / "out.ply")
    back = load(tmp_path / "out.ply")
    assert back.sh_degree == degree
    assert torch.allclose(back.means, sp.means, atol=1e-6)
    assert torch.allclose(back.quats, sp.quats, atol=1e-6)
    assert torch.allclose(back.scales, sp.scales, rtol=1e-5, atol=1e-7)
    assert torch.allclose(back.opacities, sp.opacities, atol=1e-5)
    assert torch.allclose(back.sh, sp.sh, atol=1e-6)


def test_a_fully_opaque_splat_survives_the_logit(tmp_path):
    from metal_gauss_amd.io import save_ply

    sp = _synthetic_splats(n=2)
    sp.opacities[:] = torch.tensor([0.0, 1.0])
    save_ply(sp, tmp_path / "edge.ply")
    back = load(tmp_path / "edge.ply")
    assert torch.isfinite(back.opacities).all()
    assert float(back.opacities[0]) < 1e-4 and float(back.opacities[1]) > 1.0 - 1e-4


def test_a_written_file_carries_the_fields_the_renderer_reads(tmp_path):
    """Names, channel-major SH and stored values, read by the spec-level reader."""
    from metal_gauss_amd.io import save_ply

    sp = _synthetic_splats()
    save_ply(sp, tmp_path / "fields.ply")
    cols = ply_ref.read_ply_bytes((tmp_path / "fields.ply").read_bytes())
    names = set(cols)
    assert {"x", "y", "z", "opacity"} <= names
    assert {f"scale_{i}" for i in range(3)} <= names and {f"rot_{i}" for i in range(4)} <= names
    assert {f"f_dc_{i}" for i in range(3)} <= names and {f"f_rest_{i}" for i in range(45)} <= names
    sh = sp.sh.numpy()
    assert np.array_equal(cols["f_rest_16"].astype(np.float32), sh[:, 2, 1])   # c=1, b=2
    assert np.allclose(cols["scale_1"], np.log(sp.scales[:, 1].numpy()), atol=1e-6)


def test_export_ply_matches_the_trainer_on_the_cpu(tmp_path):
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
