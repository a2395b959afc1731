"""CPU tests of the PLY restatement (oracle/ply_oracle.py) and of the host
side of brush_amd.serde (header parsing and validation, which raise before
any device work).

The oracle is pinned by:
* the brush-serde crate's own tests (import.rs:915-1198, export.rs:244-348,
  quant.rs:72-112, ply_gaussian.rs:129-149), ported one for one;
* the reference's PLY fixture apps/brush-c/tests/data/test_dataset/init.ply
  (tests/golden/ply/init.ply) against an independent read of its bytes;
* what the mathematics fixes: rgb_to_sh at closed-form points, an
  independent SuperSplat encoder round trip for the quaternion and unorm
  packings, the Inria f_rest layout ([channel][coefficient]), byte order and
  ASCII equivalence, and the min-scale fold against float64 closed forms.
"""
import os

import numpy as np
import pytest

from oracle import ply_oracle as P
from tests import ply_files as F

f32 = np.float32
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ply", "init.ply")


def load(data, sub=None):
    return P.load_splat_from_ply(data, sub)


def error_of(data, sub=None):
    with pytest.raises(P.PlyError) as e:
        load(data, sub)
    return str(e.value)


# ---- import.rs tests ------------------------------------------------------------------------

@pytest.mark.parametrize("data", [F.truncated_binary_ply(), F.truncated_compressed_chunk_ply(),
                                  F.truncated_compressed_vertex_ply(), F.truncated_compressed_sh_ply()])
def test_truncated_returns_eof_error(data):
    assert "Unexpected EOF" in error_of(data)


def test_partial_ascii_token_returns_error():
    error_of(F.ascii_ply(1, "1.0 2.0 3e"))


def test_one_shot_compressed_import_drains_to_final_message():
    m = load(F.compressed_ply_with_sh())
    assert m.meta.progress == 1.0
    assert m.data.sh_coeffs.size == 12


def test_compressed_import_rejects_missing_chunk_metadata():
    assert "chunk rows" in error_of(F.compressed_ply_without_chunk_metadata())


def test_import_rejects_zero_subsample():
    assert "greater than zero" in error_of(F.ascii_ply(1, "1.0 2.0 3.0"), 0)


def test_regular_subsample_larger_than_input_keeps_first_row():
    m = load(F.ascii_ply(1, "1.0 2.0 3.0"), 2)
    assert m.data.means.tolist() == [1.0, 2.0, 3.0]
    assert m.meta.total_splats == 1


def test_compressed_subsample_larger_than_input_keeps_first_row():
    m = load(F.compressed_ply_one_vertex(), 2)
    assert m.data.num_splats() == 1 and m.meta.total_splats == 1


def test_regular_import_rejects_partial_rgb():
    assert "exactly one red, green, and blue" in error_of(F.ascii_ply_with_properties(["red"]))


def test_regular_import_rejects_oversized_sh_schema():
    props = ["f_dc_0", "f_dc_1", "f_dc_2"] + [f"f_rest_{i}" for i in range(75)]
    assert "Unsupported SH rest property count" in error_of(F.ascii_ply_with_properties(props))


def test_compressed_import_rejects_oversized_sh_schema():
    assert "Unsupported SH rest property count" in error_of(F.compressed_ply_with_oversized_sh_header())


def test_ascii_ply_accepts_final_token_without_newline():
    m = load(F.ascii_ply(1, "1.0 2.0 3.0"))
    assert m.data.means.tolist() == [1.0, 2.0, 3.0] and m.meta.progress == 1.0


def test_zero_row_plys_return_error():
    assert "no vertices" in error_of(F.ascii_ply(0, ""))
    assert "no vertices" in error_of(F.compressed_ply_header(0, 0))


def test_sh_schema_errors():
    assert "contiguous from f_rest_0" in error_of(F.ascii_ply_with_properties(["f_dc_0", "f_dc_1", "f_dc_2",
                                                                               "f_rest_1"]))
    assert "Invalid SH property name" in error_of(F.ascii_ply_with_properties(["f_rest_x"]))
    assert "require f_dc_0, f_dc_1, and f_dc_2" in error_of(F.ascii_ply_with_properties(["f_dc_0"]))
    rest = [f"f_rest_{i}" for i in range(9)]
    assert "require a complete DC or RGB color" in error_of(F.ascii_ply_with_properties(rest))
    assert "Unknown format" in error_of(b"ply\nformat ascii 1.0\nelement face 0\nend_header\n")


def test_import_basic_functionality():
    t, sh, o = F.create_test_splats(1)
    m = load(P.splat_to_ply(t, sh, o))
    assert m.data.num_splats() == 1 and m.meta.total_splats == 1
    for v in (m.data.rotations, m.data.log_scales, m.data.sh_coeffs, m.data.raw_opacities):
        assert v is not None


@pytest.mark.parametrize("degree", [0, 1, 2])
def test_import_different_sh_degrees(degree):
    t, sh, o = F.create_test_splats(degree)
    m = load(P.splat_to_ply(t, sh, o))
    assert m.data.sh_coeffs.size // m.data.num_splats() // 3 == (degree + 1) ** 2


def test_import_with_subsample():
    t, sh, o = F.create_test_splats(0, 4)
    data = P.splat_to_ply(t, sh, o)
    assert load(data).data.num_splats() == 4
    assert load(data, 2).data.num_splats() == 2


def test_splat_data_subsample():
    n = 10
    make = lambda stride: np.repeat(np.arange(n, dtype=f32), stride)
    d = P.SplatData(make(3), make(4), make(3), make(6), make(1))
    assert d.subsample(10).num_splats() == 10 and d.subsample(0).num_splats() == 10
    s = d.subsample(3)  # step ceil(10 / 3) = 4: rows 0, 4, 8
    assert s.num_splats() == 3
    assert s.means.tolist() == [0, 0, 0, 4, 4, 4, 8, 8, 8]
    assert s.rotations.tolist() == [0] * 4 + [4] * 4 + [8] * 4
    assert s.sh_coeffs.tolist()[6:12] == [4] * 6
    assert s.raw_opacities.tolist() == [0, 4, 8]


def test_import_custom_up_axis():
    t, sh, o = F.create_test_splats(1)
    m = load(P.splat_to_ply(t, sh, o, up_axis=(0.123, 0.456, -0.789)))
    assert np.allclose(m.meta.up_axis, (0.123, 0.456, -0.789), atol=1e-5)


@pytest.mark.parametrize("comment,expect", [
    ("Vertical axis: x", (1.0, 0.0, 0.0)), ("vertical axis: Y", (0.0, -1.0, 0.0)),
    ("Vertical axis: z", (0.0, 0.0, -1.0)), ("Vertical axis: [1, 2, 3]", (1.0, 2.0, 3.0)),
    ("Vertical axis: 1 2 foo 3", (1.0, 2.0, 3.0)), ("Vertical axis: 1 2", None),
])
def test_up_axis_comments(comment, expect):
    data = F.ascii_ply(1, "1 2 3").replace(b"format ascii 1.0\n", f"format ascii 1.0\ncomment {comment}\n".encode())
    assert load(data).meta.up_axis == expect


def test_render_mode_comment_last_wins():
    data = F.ascii_ply(1, "1 2 3").replace(
        b"format ascii 1.0\n", b"format ascii 1.0\ncomment SplatRenderMode: mip\ncomment SplatRenderMode: bogus\n")
    assert load(data).meta.render_mode == "mip"


# ---- export.rs tests ------------------------------------------------------------------------

@pytest.mark.parametrize("degree,rest", [(0, 0), (1, 9), (2, 24)])
def test_ply_field_count_matches_sh_degree(degree, rest):
    t, sh, o = F.create_test_splats(degree)
    text = P.splat_to_ply(t, sh, o).decode("latin-1")
    assert text.count("property float f_rest_") == rest
    assert "f_dc_0" in text
    if rest:
        assert "f_rest_0" in text and f"f_rest_{rest}" not in text
    else:
        assert "f_rest_0" not in text
    assert f"comment SH degree: {degree}" in text and "comment SplatRenderMode: default" in text
    assert "comment Vertical axis: y" in text and "comment Exported from Brush" in text


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
def test_export_roundtrip_multiple_splats(degree):
    t, sh, o = F.create_test_splats(degree, 100)
    m = load(P.splat_to_ply(t, sh, o))
    t2, sh2, o2 = m.data.with_defaults()
    assert m.data.num_splats() == 100
    assert sh2.shape == sh.shape and np.abs(sh2 - sh).max() < 1e-6
    assert np.array_equal(t2, t) and np.array_equal(o2, o)


# ---- quant.rs / ply_gaussian.rs tests ------------------------------------------------------------

def test_vector_decode():
    assert np.all(P.decode_vec_11_10_11([0]) == 0)
    full = (0x7FF << 21) | (0x3FF << 11) | 0x7FF
    assert np.allclose(P.decode_vec_11_10_11([full]), 1.0, atol=1e-6)
    assert np.all(P.decode_vec_8_8_8_8([0]) == 0)
    assert np.allclose(P.decode_vec_8_8_8_8([0xFFFFFFFF]), 1.0, atol=1e-6)
    vals = np.arange(100, dtype=np.uint64) * 42949673
    for arr in (P.decode_vec_11_10_11(vals.astype(np.uint32)), P.decode_vec_8_8_8_8(vals.astype(np.uint32))):
        assert arr.min() >= 0 and arr.max() <= 1


def test_decode_quat():
    q = P.decode_quat([(512 << 20) | (512 << 10) | 512])
    assert np.isfinite(q).all() and abs(np.linalg.norm(q) - 1.0) < 1e-5


def test_quantized_endpoints():
    assert P.dequant_color(np.array([0, 255], np.uint8), "u1").tolist() == [0.0, 1.0]
    assert P.dequant_color(np.array([0, 65535], np.uint16), "u2").tolist() == [0.0, 1.0]
    assert P.dequant_sh(np.array([0, 255], np.uint8)).tolist() == [-4.0, 4.0]


# ---- pins from the mathematics and the fixture -----------------------------------------------------

def test_rgb_to_sh_closed_forms():
    """SH_C0 = 1 / (2 sqrt(pi)): rgb 0.5 -> 0, rgb 1 -> sqrt(pi), rgb 0 -> -sqrt(pi)."""
    v = P.rgb_to_sh(np.array([0.5, 1.0, 0.0], f32))
    assert v[0] == 0.0
    assert abs(v[1] - np.sqrt(np.pi)) < 2e-7 and abs(v[2] + np.sqrt(np.pi)) < 2e-7


def test_init_ply_fixture():
    """The reference's own fixture: 100 float xyz with uchar rgba, read
    independently through a structured view of the bytes."""
    data = open(GOLDEN, "rb").read()
    m = load(data)
    body = data[data.index(b"end_header\n") + len(b"end_header\n"):]
    raw = np.frombuffer(body, np.dtype([("x", "<f4"), ("y", "<f4"), ("z", "<f4"), ("r", "u1"), ("g", "u1"),
                                        ("b", "u1"), ("a", "u1")]), 100)
    assert m.data.num_splats() == 100 and m.meta.total_splats == 100
    assert np.array_equal(m.data.means.reshape(100, 3), np.stack([raw["x"], raw["y"], raw["z"]], 1))
    rgb = np.stack([raw["r"], raw["g"], raw["b"]], 1).astype(np.float64) / 255.0
    assert np.allclose(m.data.sh_coeffs.reshape(100, 3), (rgb - 0.5) * 2.0 * np.sqrt(np.pi), atol=1e-6)
    assert m.data.rotations is None and m.data.log_scales is None and m.data.raw_opacities is None
    assert m.meta.up_axis is None and m.meta.render_mode is None


def test_quaternion_packing_roundtrip():
    """An independent smallest-three encoder (largest index in the top bits,
    sign made positive, v / sqrt(2) + 0.5 in 10 bits): decode recovers the
    unit quaternion up to sign within the 10-bit step."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal((5000, 4))
    dec = P.decode_quat(F.encode_quat(q)).astype(np.float64)
    qn = q / np.linalg.norm(q, axis=1, keepdims=True)
    err = np.minimum(np.abs(dec - qn).max(1), np.abs(dec + qn).max(1))
    assert err.max() < 2.5e-3
    assert np.abs(np.linalg.norm(dec, axis=1) - 1).max() < 1e-5


def test_unorm_packing_field_order():
    """x occupies the top 11 bits, y the middle 10, z the low 11; colour
    bytes run from the most significant."""
    assert P.decode_vec_11_10_11([0x7FF << 21]).tolist() == [[1.0, 0.0, 0.0]]
    assert P.decode_vec_11_10_11([0x3FF << 11]).tolist() == [[0.0, 1.0, 0.0]]
    assert P.decode_vec_11_10_11([0x7FF]).tolist() == [[0.0, 0.0, 1.0]]
    v = P.decode_vec_8_8_8_8([0x11223344])[0] * 255
    assert np.allclose(v, [0x11, 0x22, 0x33, 0x44])
    rng = np.random.default_rng(5)
    x = rng.uniform(0, 1, (1000, 3))
    dec = P.decode_vec_11_10_11(F.encode_unorm3(x))
    assert np.abs(dec - x).max() <= 0.5 / 1023 + 1e-7


def test_compressed_dequantisation_closed_form():
    """Positions, scales and colours are the chunk's [min, max] at the
    packed fraction; opacity is the logit of the alpha byte / 255."""
    rng = np.random.default_rng(11)
    cm, vert, _, _ = F.compressed_elements(rng, 700)
    m = load(F.write_ply("binary_little_endian", [("chunk", cm), ("vertex", vert)]))
    t, sh, o = m.data.with_defaults()
    c = np.arange(700) // 256
    frac = P.decode_vec_11_10_11(vert["packed_position"]).astype(np.float64)
    lo = np.stack([cm["min_x"][c], cm["min_y"][c], cm["min_z"][c]], 1).astype(np.float64)
    hi = np.stack([cm["max_x"][c], cm["max_y"][c], cm["max_z"][c]], 1).astype(np.float64)
    assert np.allclose(t[:, 0:3], lo + frac * (hi - lo), atol=1e-5)
    a = (vert["packed_color"] & 0xFF).astype(np.float64) / 255.0
    ok = (a > 0) & (a < 1)
    assert np.allclose(o[ok], np.log(a[ok] / (1 - a[ok])), atol=1e-5)
    assert sh.shape == (700, 1, 3)


def test_inria_rest_layout():
    """Files store f_rest as [channel][coefficient] (features_rest transposed
    and flattened); import yields sh[n, coefficient, channel]."""
    rng = np.random.default_rng(2)
    n, cpc = 50, 15
    feat = rng.standard_normal((n, cpc, 3)).astype(f32)
    arr = np.zeros(n, np.dtype([("x", "f4"), ("y", "f4"), ("z", "f4")] + [(f"f_dc_{k}", "f4") for k in range(3)] +
                               [(f"f_rest_{k}", "f4") for k in range(3 * cpc)]))
    flat = feat.transpose(0, 2, 1).reshape(n, -1)
    for k in range(3 * cpc):
        arr[f"f_rest_{k}"] = flat[:, k]
    m = load(F.write_ply("binary_little_endian", [("vertex", arr)]))
    sh = m.data.sh_coeffs.reshape(n, 16, 3)
    assert np.array_equal(sh[:, 1:, :], feat)


@pytest.mark.parametrize("fmt", ["ascii", "binary_big_endian"])
def test_formats_agree(fmt):
    rng = np.random.default_rng(4)
    arr = F.standard_rows(rng, 64, rest=9, extra=(("normals", "f4"),), shuffle=True)
    a = load(F.write_ply("binary_little_endian", [("vertex", arr)])).data.with_defaults()
    b = load(F.write_ply(fmt, [("vertex", arr)])).data.with_defaults()
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def _reorder(arr, rng):
    from numpy.lib import recfunctions as rfn

    names = list(arr.dtype.names)
    return rfn.repack_fields(arr[[names[i] for i in rng.permutation(len(names))]])


def test_property_order_does_not_matter():
    """Properties are read by name: permuting the declaration order of every
    element (standard and compressed, SH rows included) changes nothing."""
    rng = np.random.default_rng(21)
    arr = F.standard_rows(rng, 100, rest=24, color="rgb_u16")
    a = load(F.write_ply("binary_little_endian", [("vertex", arr)])).data.with_defaults()
    b = load(F.write_ply("binary_little_endian", [("vertex", _reorder(arr, rng))])).data.with_defaults()
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    cm, vert, sh, _ = F.compressed_elements(rng, 600, 45)
    a = load(F.write_ply("binary_little_endian", [("chunk", cm), ("vertex", vert), ("sh", sh)])).data.with_defaults()
    els = [("chunk", _reorder(cm, rng)), ("vertex", _reorder(vert, rng)), ("sh", _reorder(sh, rng))]
    b = load(F.write_ply("binary_little_endian", els)).data.with_defaults()
    for x, y in zip(a, b):
        assert np.array_equal(x, y, equal_nan=True)


def test_min_scale_fold_closed_form():
    """f = s (isotropic): scale sqrt(2) s, opacity sigma * (1/8)^(1/2); f = 0
    leaves the splat unchanged."""
    rng = np.random.default_rng(9)
    n = 200
    t = rng.standard_normal((n, 10)).astype(f32)
    ls = rng.uniform(-4, 0, n)
    t[:, 7:10] = ls[:, None]
    o = rng.uniform(-3, 3, n).astype(f32)
    t2, o2 = P.fold_min_scale(t, o, np.exp(ls).astype(f32))
    assert np.allclose(t2[:, 7:10], (ls + 0.5 * np.log(2.0))[:, None], atol=1e-5)
    sig = 1 / (1 + np.exp(-o.astype(np.float64))) * np.sqrt(1 / 8)
    assert np.allclose(o2, np.log(sig / (1 - sig)), atol=1e-4)
    t3, o3 = P.fold_min_scale(t, o, np.zeros(n, f32))
    assert np.allclose(t3, t, atol=1e-6) and np.allclose(o3, o, atol=1e-4)


def test_export_rows_normalise_quaternions():
    rng = np.random.default_rng(1)
    t = rng.standard_normal((100, 10)).astype(f32)
    t[0, 3:7] = 0.0  # |q| = 0: divided by 1e-12, stays 0
    rows = P.export_rows(t, rng.standard_normal((100, 4, 3)).astype(f32), rng.standard_normal(100).astype(f32))
    assert np.allclose(np.linalg.norm(rows[1:, 7:11], axis=1), 1.0, atol=1e-6)
    assert np.all(rows[0, 7:11] == 0.0)


# ---- host side of the product (errors raise before any device work) ---------------------------

@pytest.mark.parametrize("maker,needle", [
    (F.truncated_binary_ply, "Unexpected EOF"), (F.truncated_compressed_chunk_ply, "Unexpected EOF"),
    (F.truncated_compressed_vertex_ply, "Unexpected EOF"), (F.truncated_compressed_sh_ply, "Unexpected EOF"),
    (F.compressed_ply_without_chunk_metadata, "chunk rows"),
    (F.compressed_ply_with_oversized_sh_header, "Unsupported SH rest property count"),
    (lambda: F.ascii_ply_with_properties(["red"]), "exactly one red, green, and blue"),
    (lambda: F.ascii_ply(0, ""), "no vertices"), (lambda: F.compressed_ply_header(0, 0), "no vertices"),
    (lambda: F.ascii_ply(1, "1.0 2.0 3e"), ""),
])
def test_product_host_errors(maker, needle):
    from brush_amd import serde as S

    with pytest.raises(S.PlyError) as e:
        S.load_splat_from_ply(maker())
    assert needle in str(e.value)
    with pytest.raises(S.PlyError, match="greater than zero"):
        S.load_splat_from_ply(maker(), 0)


def test_product_header_metadata_matches_oracle():
    from brush_amd import serde as S

    for comment in ("Vertical axis: [1, 2, 3]", "vertical axis: z", "Vertical axis: 1 2 foo 3",
                    "SplatRenderMode: mip", "SplatRenderMode: default"):
        data = F.ascii_ply(1, "1 2 3").replace(b"format ascii 1.0\n",
                                               f"format ascii 1.0\ncomment {comment}\n".encode())
        up, mode = S.header_metadata(S.parse_header(data))
        ref = load(data).meta
        assert up == ref.up_axis
        assert (mode.name.lower() if mode is not None else None) == ref.render_mode
