"""PLY records decoded and encoded by the HIP kernels (mg_ply_decode /
mg_ply_encode) against the CPU path and the restated trainer export
(oracle/ply_ref.py). Decoding computes in double and rounds once on both
sides, so the tensors agree to the last bit but for an occasional 1-ulp
difference of a transcendental; the export without a filter is a layout
permutation and must be bit-identical."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ply_ref

pytestmark = pytest.mark.gpu


def random_cols(n, seed, per=15):
    g = np.random.default_rng(seed)
    cols = {}
    m = g.standard_normal((n, 3)).astype(np.float32)
    for i, nm in enumerate("xyz"):
        cols[nm] = m[:, i]
    for c in range(3):
        cols[f"f_dc_{c}"] = g.standard_normal(n).astype(np.float32)
    for i in range(3 * per):
        cols[f"f_rest_{i}"] = (g.standard_normal(n) * 0.1).astype(np.float32)
    cols["opacity"] = (g.standard_normal(n) * 3).astype(np.float32)
    for i in range(3):
        cols[f"scale_{i}"] = (g.standard_normal(n) - 4).astype(np.float32)
    q = g.standard_normal((n, 4)).astype(np.float32)
    q[::97] = 0.0                                   # dead splats with a zero rotation
    for i in range(4):
        cols[f"rot_{i}"] = q[:, i]
    return cols


def ulps(a, b):
    a = a.detach().cpu().numpy().astype(np.float32).view(np.int32).astype(np.int64)
    b = b.detach().cpu().numpy().astype(np.float32).view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max()) if a.size else 0


@pytest.mark.parametrize("case", ["le", "be", "double", "deg1", "reordered"])
def test_gpu_decode_matches_cpu(dev, tmp_path, case):
    from metal_gauss_amd.io import load_ply

    per = 3 if case == "deg1" else 15
    seed = {"le": 1, "be": 2, "double": 3, "deg1": 4, "reordered": 5}[case]
    cols = random_cols(3000, seed, per)
    types = None
    fmt = "binary_little_endian"
    if case == "be":
        fmt = "binary_big_endian"
    if case == "double":
        types = {k: "double" for k in cols if k.startswith("f_rest") or k == "opacity"}
    if case == "reordered":
        cols = {k: cols[k] for k in sorted(cols)}
    path = tmp_path / f"{case}.ply"
    path.write_bytes(ply_ref.write_ply_bytes(cols, fmt=fmt, types=types))
    cpu = load_ply(path)
    gpu = load_ply(path, device="cuda")
    assert gpu.sh_degree == cpu.sh_degree
    for f in ("means", "quats", "scales", "opacities", "sh"):
        a, b = getattr(gpu, f), getattr(cpu, f)
        assert a.device.type == "cuda" and a.shape == b.shape, f
        assert ulps(a, b) <= 1, (f, ulps(a, b))
    assert torch.isfinite(gpu.quats).all()


def trainer_params(n, seed, split=True):
    g = torch.Generator().manual_seed(seed)
    p = {"means": torch.randn(n, 3, generator=g), "log_scales": torch.randn(n, 3, generator=g) - 4,
         "quats": torch.randn(n, 4, generator=g), "logit_opac": torch.randn(n, generator=g) * 2}
    if split:
        p["sh_dc"] = torch.randn(n, 1, 3, generator=g)
        p["sh_rest"] = torch.randn(n, 15, 3, generator=g) * 0.1
    else:
        p["sh"] = torch.randn(n, 16, 3, generator=g)
    return p


@pytest.mark.parametrize("split", [True, False])
def test_gpu_export_matches_the_trainer(dev, tmp_path, split):
    from metal_gauss_amd.io import export_ply

    n = 5000
    p = trainer_params(n, 4, split)
    f3d = torch.rand(n, generator=torch.Generator().manual_seed(5)) * 0.02
    gp = {k: v.to(dev) for k, v in p.items()}
    # Without the filter: a permutation of the stored values, bit for bit.
    export_ply(gp, str(tmp_path / "a.ply"))
    got = ply_ref.read_ply_bytes((tmp_path / "a.ply").read_bytes())
    for k, w in ply_ref.encode_export(p).items():
        assert np.array_equal(got[k].astype(np.float32), w), k
    # With the baked 3D filter: float32 arithmetic on both sides. The logit
    # log(o / (1 - o)) amplifies one ulp of o by 1 / (1 - o) near o = 1, so
    # the opacity column is compared as an opacity.
    export_ply(gp, str(tmp_path / "b.ply"), filter_3d=f3d.to(dev))
    got = ply_ref.read_ply_bytes((tmp_path / "b.ply").read_bytes())
    for k, w in ply_ref.encode_export(p, f3d).items():
        if k == "opacity":
            sg = lambda x: 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))  # noqa: E731
            assert np.abs(sg(got[k]) - sg(w)).max() < 1e-6, k
        else:
            assert np.allclose(got[k], w, rtol=2e-6, atol=2e-6), (k, np.abs(got[k] - w).max())


def test_round_trip_at_a_million(dev, tmp_path):
    """Export the trainer's parameters from the GPU, load them back onto it:
    the activated values of the same parameters."""
    from metal_gauss_amd.io import export_ply, load_ply

    n = 1_000_000
    p = {k: v.to(dev) for k, v in trainer_params(n, 6).items()}
    path = tmp_path / "big.ply"
    export_ply(p, str(path))
    sp = load_ply(path, device="cuda")
    assert len(sp) == n and sp.sh_degree == 3
    assert torch.equal(sp.means, p["means"])
    assert torch.allclose(sp.scales, torch.exp(p["log_scales"]), rtol=1e-6)
    assert torch.allclose(sp.opacities, torch.sigmoid(p["logit_opac"]), rtol=1e-6, atol=1e-7)
    q = p["quats"] / p["quats"].norm(dim=1, keepdim=True).clamp_min(1e-12)
    assert torch.allclose(sp.quats, q, atol=1e-6)
    assert torch.equal(sp.sh, torch.cat([p["sh_dc"], p["sh_rest"]], dim=1))


# The GPU decode against the oracle rather than the CPU decode: the known
# answers of the reference's PLY tests, and the spec-level decode of
# oracle/ply_ref.py, both written independently of the package's reader.
from test_io import DECODE_CASES, _file, _stored, _tagged_rest  # noqa: E402


@pytest.mark.parametrize("case", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_gpu_decode_known_answers(dev, tmp_path, case):
    from metal_gauss_amd.io import load_ply

    name, stored, field, want, rel = case
    sp = load_ply(_file(tmp_path, f"{name}.ply", _stored(3, **stored)), device="cuda")
    got = (sp.sh[:, 0] if field == "sh[:, 0]" else getattr(sp, field)).cpu().numpy()
    assert got == pytest.approx(want.astype(np.float32), rel=rel, abs=0 if rel else 1e-12)


def test_gpu_decode_zero_quaternion_and_channel_major_rest(dev, tmp_path):
    from metal_gauss_amd.io import load_ply

    rot = np.array([[0.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0], [0.0, 2.0, 0.0, 0.0]])
    sp = load_ply(_file(tmp_path, "z.ply", _stored(3, rot=rot, rest=_tagged_rest(3, 15))),
                  device="cuda")
    assert torch.isfinite(sp.quats).all()
    band = torch.arange(1, 16)[None, :, None]
    chan = torch.arange(3)[None, None, :]
    splat = torch.arange(3)[:, None, None]
    assert torch.equal(sp.sh[:, 1:, :].cpu(), (1000 * splat + 15 * chan + band - 1).float())


def test_gpu_decode_matches_the_spec_level_decode(dev, tmp_path):
    from metal_gauss_amd.io import load_ply

    rng = np.random.default_rng(7)
    n = 500
    cols = _stored(n, xyz=rng.standard_normal((n, 3)), rot=rng.standard_normal((n, 4)),
                   log_scale=rng.standard_normal((n, 3)) - 3, logit=3 * rng.standard_normal(n),
                   dc=rng.standard_normal((n, 3)), rest=rng.standard_normal((n, 15, 3)))
    path = _file(tmp_path, "rand.ply", cols)
    sp = load_ply(path, device="cuda")
    want = ply_ref.decode(ply_ref.read_ply_bytes(path.read_bytes()))
    for f, w in zip(("means", "quats", "scales", "opacities", "sh"), want[:5]):
        assert ulps(getattr(sp, f), torch.from_numpy(w.astype(np.float32))) <= 1, f
    assert sp.sh_degree == want[5]
