"""GPU parity of PLY import/export (bh_ply_decode_rows,
bh_ply_decode_compressed, bh_ply_encode_rows through brush_amd.serde) with
the CPU restatement oracle/ply_oracle.py, whose behaviour is pinned by
tests/test_oracle_ply.py.

Every decoded value is compared bit for bit (both sides evaluate the same
float32 operations; inverse_sigmoid uses the same reproducible logf), as are
the exported bytes.  The min-scale fold runs in torch on the device and is
compared to the float32 restatement within 1e-5 relative.
"""
import os

import numpy as np
import pytest

from oracle import ply_oracle as P
from tests import ply_files as F
from tests.helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ply", "init.ply")


def compare(data, sub=None, gpu=None):
    from brush_amd import serde as S

    g = S.load_splat_from_ply(data, sub)
    o = P.load_splat_from_ply(data, sub)
    t, sh, op = o.data.with_defaults()
    assert_bits_equal("transforms", g.data.transforms.cpu().numpy(), t)
    assert_bits_equal("sh_coeffs", g.data.sh.cpu().numpy(), sh)
    assert_bits_equal("raw_opacities", g.data.opac.cpu().numpy(), op)
    assert g.meta.total_splats == o.meta.total_splats and g.meta.progress == o.meta.progress
    assert g.meta.up_axis == o.meta.up_axis
    for name in ("rotations", "log_scales", "sh_coeffs", "raw_opacities"):
        assert (getattr(g.data, name) is None) == (getattr(o.data, name) is None), name
    return g


STANDARD = [
    dict(n=1000, rest=45),
    dict(n=257, rest=0, color="rgb_u8", groups=()),
    dict(n=300, rest=9, color="rgb_u16", shuffle=True),
    dict(n=300, rest=24, color="rgb_f32", extra=(("normals", "f4"),)),
    dict(n=513, rest=72, groups=("rot",), extra=(("flag", "u1"), ("w", "f8"))),
    dict(n=64, rest=0, color="none", groups=("scale", "opacity"), extra=(("id", "i4"),)),
    dict(n=200, rest=9, shuffle=True, types={"x": "f8", "y": "i2", "z": "u1", "opacity": "i1", "rot_0": "u4",
                                            "scale_1": "i4", "f_rest_3": "u2"}),
    dict(n=129, rest=0, color="dc", groups=("rot", "scale", "opacity"), extra=(("k0", "u1"), ("k1", "u1"),
                                                                               ("k2", "u1"))),
]


@pytest.mark.parametrize("case", range(len(STANDARD)))
@pytest.mark.parametrize("fmt", ["binary_little_endian", "binary_big_endian", "ascii"])
def test_standard_ply_matches_oracle(gpu, case, fmt):
    spec = dict(STANDARD[case])
    print(f"[case] standard ply {case} {fmt} {spec}", flush=True)
    rng = np.random.default_rng(100 + case)
    n = spec.pop("n")
    arr = F.standard_rows(rng, n, **spec)
    data = F.write_ply(fmt, [("vertex", arr)], comments=("Vertical axis: 0 0 1",))
    compare(data)
    for sub in (2, 3, 7):
        compare(data, sub)


@pytest.mark.parametrize("rest,shuffle,sub", [(0, False, None), (9, False, None), (45, True, None), (72, False, 3),
                                              (24, True, 2)])
@pytest.mark.parametrize("fmt", ["binary_little_endian", "binary_big_endian"])
def test_compressed_ply_matches_oracle(gpu, rest, shuffle, sub, fmt):
    print(f"[case] compressed ply rest={rest} shuffle={shuffle} sub={sub} {fmt}", flush=True)
    rng = np.random.default_rng(rest + 7)
    n = 1500
    cm, vert, sh, _ = F.compressed_elements(rng, n, rest, shuffle)
    els = [("chunk", cm), ("vertex", vert)] + ([("sh", sh)] if sh is not None else [])
    compare(F.write_ply(fmt, els), sub)


def test_crate_fixtures_on_gpu(gpu):
    from brush_amd import serde as S

    g = compare(F.compressed_ply_with_sh())
    assert g.data.sh_coeffs.numel() == 12
    assert compare(F.ascii_ply(1, "1.0 2.0 3.0"), 2).data.means.tolist() == [1.0, 2.0, 3.0]
    assert compare(F.compressed_ply_one_vertex(), 2).data.num_splats() == 1
    m = S.load_splat_from_ply(F.ascii_ply(1, "1.0 2.0 3.0"))
    assert m.data.means.tolist() == [1.0, 2.0, 3.0] and m.meta.progress == 1.0


def test_init_ply_fixture(gpu):
    g = compare(open(GOLDEN, "rb").read())
    assert g.data.num_splats() == 100
    splats = g.data.into_splats()
    assert tuple(splats.sh_coeffs.shape) == (100, 1, 3) and tuple(splats.transforms.shape) == (100, 10)


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
def test_export_matches_oracle(gpu, degree):
    import torch

    from brush_amd import serde as S
    from brush_amd.render import Splats

    print(f"[case] export degree {degree}", flush=True)
    rng = np.random.default_rng(degree)
    n = 777
    c = (degree + 1) ** 2
    t = rng.standard_normal((n, 10)).astype(np.float32)
    t[5, 3:7] = 0.0
    sh = rng.standard_normal((n, c, 3)).astype(np.float32)
    o = rng.standard_normal(n).astype(np.float32)
    s = Splats(torch.from_numpy(t).to(gpu), torch.from_numpy(sh).to(gpu), torch.from_numpy(o).to(gpu), degree == 2)
    got = S.splat_to_ply(s, up_axis=(0.123, 0.456, -0.789) if degree == 1 else None)
    want = P.splat_to_ply(t, sh, o, render_mip=degree == 2, up_axis=(0.123, 0.456, -0.789) if degree == 1 else None)
    assert got == want
    # and back: the rows round-trip through the GPU decoder
    back = S.load_splat_from_ply(got)
    rows = P.export_rows(t, sh, o)
    assert_bits_equal("means", back.data.transforms[:, 0:3].cpu().numpy(), rows[:, 0:3])
    assert_bits_equal("rot", back.data.transforms[:, 3:7].cpu().numpy(), rows[:, 7:11])
    assert_bits_equal("sh", back.data.sh.cpu().numpy(), sh)
    assert back.meta.render_mode == (S.SplatRenderMode.Mip if degree == 2 else S.SplatRenderMode.Default)


def test_crate_roundtrip_tests_on_gpu(gpu):
    """export.rs:292-348 and import.rs:1082-1135 through the device path."""
    import torch

    from brush_amd import serde as S
    from brush_amd.render import Splats

    for degree in (0, 1, 2, 3):
        t, sh, o = F.create_test_splats(degree, 100)
        s = Splats(*(torch.from_numpy(a).to(gpu) for a in (t, sh, o)))
        m = S.load_splat_from_ply(S.splat_to_ply(s))
        imp = m.data.into_splats()
        assert imp.num_splats() == 100 and imp.sh_degree() == degree
        assert float((imp.sh_coeffs - s.sh_coeffs).abs().max()) < 1e-6
    t, sh, o = F.create_test_splats(0, 4)
    data = S.splat_to_ply(Splats(*(torch.from_numpy(a).to(gpu) for a in (t, sh, o))))
    assert S.load_splat_from_ply(data, 2).data.num_splats() == 2
    d = S.load_splat_from_ply(data).data.subsample(3)
    assert d.num_splats() == 2  # step ceil(4 / 3) = 2


def test_export_bakes_min_scale(gpu):
    import torch

    from brush_amd import serde as S
    from brush_amd.render import Splats

    rng = np.random.default_rng(12)
    n = 500
    t = rng.standard_normal((n, 10)).astype(np.float32)
    t[:, 7:10] = rng.uniform(-5, -1, (n, 3))
    sh = rng.standard_normal((n, 4, 3)).astype(np.float32)
    o = rng.standard_normal(n).astype(np.float32)
    f = rng.uniform(0.001, 0.05, n).astype(np.float32)
    s = Splats(*(torch.from_numpy(a).to(gpu) for a in (t, sh, o)), min_scale=torch.from_numpy(f).to(gpu))
    got = S.load_splat_from_ply(S.splat_to_ply(s)).data
    want = P.load_splat_from_ply(P.splat_to_ply(t, sh, o, min_scale=f)).data.with_defaults()
    for name, a, b in (("transforms", got.transforms, want[0]), ("raw_opac", got.opac, want[2])):
        a = a.cpu().numpy()
        assert np.allclose(a, b, rtol=1e-5, atol=1e-5), name


def test_full_size_roundtrip(gpu, tmp_path):
    """One million degree-3 splats: decode(export(x)) reproduces x with
    normalised quaternions, bit for bit, and the decoded file matches the
    restatement."""
    import torch

    from brush_amd import serde as S
    from brush_amd.render import Splats

    n = 1 << 20
    gen = torch.Generator(device=gpu).manual_seed(5)
    t = torch.randn((n, 10), device=gpu, generator=gen)
    sh = torch.randn((n, 16, 3), device=gpu, generator=gen)
    o = torch.randn((n,), device=gpu, generator=gen)
    data = S.splat_to_ply(Splats(t, sh, o))
    back = S.load_splat_from_ply(data).data
    rows = S.encode_rows(t, sh, o)
    assert torch.equal(back.transforms[:, 0:3], t[:, 0:3])
    assert torch.equal(back.transforms[:, 7:10], t[:, 7:10])
    assert torch.equal(back.transforms[:, 3:7], rows[:, 7:11])
    assert torch.equal(back.sh, sh) and torch.equal(back.opac, o)
    ref = P.load_splat_from_ply(data).data.with_defaults()
    assert_bits_equal("transforms", back.transforms.cpu().numpy(), ref[0])
    assert_bits_equal("sh", back.sh.cpu().numpy(), ref[1])
    # from a file: memory-mapped and streamed through the pinned staging buffers
    path = tmp_path / "full.ply"
    path.write_bytes(data)
    again = S.load_splat_from_ply(str(path)).data
    assert torch.equal(again.transforms, back.transforms) and torch.equal(again.sh, back.sh)
    assert torch.equal(again.opac, back.opac)
