"""CPU restatement of brush-serde's PLY import and export, in numpy.

TEST INFRASTRUCTURE ONLY: imported by tests/ and the ``cpu_baseline`` leg of
bench.py, as the checker.  The product package (brush_amd) never imports it.

Restates crates/brush-serde/src:
* ``load_splat_from_ply`` / ``stream_splat_from_ply`` (import.rs:167-296)
  for the standard 3DGS PLY (parse_ply, import.rs:341-502) in ascii and
  binary little- or big-endian, and for the SuperSplat compressed PLY
  (parse_compressed_ply, import.rs:504-720);
* ``SplatData`` (import.rs:26-91) with ``subsample`` and the into_splats
  defaults;
* ``splat_to_ply`` (export.rs:83-199) with ``bake_min_scale``
  (brush-render/src/gaussian_splats.rs:139-164, 294-307);
* the quantisation decoders of quant.rs:1-71 and the colour / SH
  dequantisers of ply_gaussian.rs:35-110.

Every value is computed in float32 by the reference's expressions: per row
where the reference works per row, here vectorised over the rows.
inverse_sigmoid takes the reproducible logf of the C restatement
(liboracle.so), the one the GPU kernels use; Rust's ``f32::ln`` agrees with it
to within 2 ulp.  ASCII values go through float64 on their way to float32
(Rust parses float32 directly; the two differ only when a decimal lies within
a float64 rounding of a float32 midpoint).
"""
from __future__ import annotations

import io
import os
from dataclasses import dataclass, field

import numpy as np

f32 = np.float32
SH_C0 = f32(0.28209479177387814)  # brush-render/src/shaders.rs SH_C0
SPLATS_PER_CHUNK = 256              # import.rs:513
SH_REST_COUNTS = (0, 9, 24, 45, 72)  # import.rs:325 (degrees 0..4)

_TYPES = {"char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1", "short": "i2", "int16": "i2",
          "ushort": "u2", "uint16": "u2", "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
          "float": "f4", "float32": "f4", "double": "f8", "float64": "f8"}


class PlyError(ValueError):
    """serde_ply::DeserializeError."""


# ---- small helpers (brush-render sh.rs, gaussian_splats.rs) ---------------------------------------

def rgb_to_sh(rgb: np.ndarray) -> np.ndarray:
    """sh.rs:20-31: (rgb - 0.5) / SH_C0, per channel, f32."""
    return (np.asarray(rgb, f32) - f32(0.5)) / SH_C0


def inverse_sigmoid(x: np.ndarray) -> np.ndarray:
    """gaussian_splats.rs:129-131: ln(x / (1 - x)), f32."""
    from oracle import oracle as _o

    x = np.asarray(x, f32)
    with np.errstate(divide="ignore", invalid="ignore"):
        return _o.logf(x / (f32(1.0) - x))


def sh_coeffs_for_degree(degree: int) -> int:
    return (degree + 1) ** 2


# ---- quantisation (quant.rs, ply_gaussian.rs) -------------------------------------------------------

def unpack_unorm(packed: np.ndarray, bits: int) -> np.ndarray:
    """quant.rs:4-7: an n-bit unsigned normalised integer to [0, 1]."""
    return np.asarray(packed, np.uint32).astype(f32) / f32((1 << bits) - 1)


def decode_vec_11_10_11(v) -> np.ndarray:
    """quant.rs:9-19 -> [n, 3]."""
    v = np.asarray(v, np.uint32)
    return np.stack([unpack_unorm((v >> 21) & 0x7FF, 11), unpack_unorm((v >> 11) & 0x3FF, 10),
                     unpack_unorm(v & 0x7FF, 11)], -1)


def decode_vec_8_8_8_8(v) -> np.ndarray:
    """quant.rs:20-35 -> [n, 4], the most significant byte first."""
    v = np.asarray(v, np.uint32)
    return np.stack([unpack_unorm((v >> s) & 0xFF, 8) for s in (24, 16, 8, 0)], -1)


def decode_quat(v) -> np.ndarray:
    """quant.rs:37-71 -> [n, 4] in (w, x, y, z): two bits name the largest
    component, three 10-bit fields hold the others scaled by 1/sqrt(2); the
    largest is recovered from the unit norm."""
    v = np.asarray(v, np.uint32).reshape(-1)
    largest = ((v >> 30) & 0x3).astype(np.int64)
    norm = f32(0.5) * f32(1.41421356237309504880)
    abc = [(unpack_unorm(x, 10) - f32(0.5)) / norm for x in ((v >> 20) & 0x3FF, (v >> 10) & 0x3FF, v & 0x3FF)]
    with np.errstate(invalid="ignore"):
        big = np.sqrt(f32(1.0) - (abc[0] * abc[0] + abc[1] * abc[1] + abc[2] * abc[2]))
    q = np.empty((v.size, 4), f32)
    for k in range(4):
        # quat[largest] = big; the other slots take a, b, c in order
        slot = np.clip(k - (largest < k).astype(np.int64), 0, 2)
        q[:, k] = np.where(largest == k, big, np.choose(slot, abc))
    return q


def dequant_color(values: np.ndarray, dtype: str) -> np.ndarray:
    """ply_gaussian.rs:35-56: u8 / 255, u16 / 65535, floats as they are."""
    if dtype == "u1":
        return values.astype(f32) / f32(255.0)
    if dtype == "u2":
        return values.astype(f32) / f32(65535.0)
    return values.astype(f32)


def dequant_sh(values: np.ndarray) -> np.ndarray:
    """ply_gaussian.rs:105-111: u8 to [-4, 4]: (v / 255 - 0.5) * 8."""
    return (values.astype(f32) / f32(255.0) - f32(0.5)) * f32(8.0)


# ---- parsed data (import.rs:19-98) --------------------------------------------------------------

@dataclass
class ParseMetadata:
    up_axis: tuple | None
    render_mode: str | None  # "default" | "mip" | None
    total_splats: int
    progress: float


@dataclass
class SplatData:
    """Raw splat arrays parsed from a PLY; only the means are guaranteed.
    sh_coeffs are coefficient-major ([n, coeffs, 3] flattened)."""
    means: np.ndarray
    rotations: np.ndarray | None = None
    log_scales: np.ndarray | None = None
    sh_coeffs: np.ndarray | None = None
    raw_opacities: np.ndarray | None = None

    def num_splats(self) -> int:
        return self.means.size // 3

    def subsample(self, max_splats: int) -> "SplatData":
        """import.rs:49-74: strided subsample to at most ``max_splats`` rows."""
        n = self.num_splats()
        if max_splats == 0 or n <= max_splats:
            return self
        step = -(-n // max_splats)

        def pick(v, stride):
            return None if v is None else np.ascontiguousarray(v.reshape(n, stride)[::step].reshape(-1))

        sh_stride = 0 if self.sh_coeffs is None else self.sh_coeffs.size // n
        return SplatData(pick(self.means, 3), pick(self.rotations, 4), pick(self.log_scales, 3),
                         pick(self.sh_coeffs, sh_stride), pick(self.raw_opacities, 1))

    def with_defaults(self):
        """import.rs:77-91 (into_splats): (transforms [n,10], sh [n,C,3],
        raw_opacities [n]) with identity rotation, log-scale -4, SH DC 0.5
        and opacity inverse_sigmoid(0.5) for missing fields."""
        n = self.num_splats()
        rot = self.rotations if self.rotations is not None else np.tile(np.array([1, 0, 0, 0], f32), n)
        scales = self.log_scales if self.log_scales is not None else np.full(n * 3, -4.0, f32)
        sh = self.sh_coeffs if self.sh_coeffs is not None else np.full(n * 3, 0.5, f32)
        opac = self.raw_opacities if self.raw_opacities is not None else np.full(n, inverse_sigmoid(f32(0.5)), f32)
        transforms = np.concatenate([self.means.reshape(n, 3), np.asarray(rot, f32).reshape(n, 4),
                                     np.asarray(scales, f32).reshape(n, 3)], 1).astype(f32)
        return transforms, np.asarray(sh, f32).reshape(n, -1, 3), np.asarray(opac, f32).reshape(n)


@dataclass
class SplatMessage:
    meta: ParseMetadata
    data: SplatData


# ---- header -------------------------------------------------------------------------------------

@dataclass
class PlyProperty:
    name: str
    dtype: str                   # numpy code of a scalar property
    list_types: tuple | None = None  # (count dtype, item dtype) of a list property


@dataclass
class PlyElement:
    name: str
    count: int
    properties: list = field(default_factory=list)

    def has_property(self, name: str) -> bool:
        return any(p.name == name for p in self.properties)

    def dtype(self, endian: str) -> np.dtype:
        if any(p.list_types for p in self.properties):
            raise PlyError(f"list properties are not supported in element '{self.name}'")
        return np.dtype([(p.name, endian + p.dtype) for p in self.properties])


@dataclass
class PlyHeader:
    format: str
    comments: list
    elements: list
    data_offset: int

    def get_element(self, name: str):
        return next((e for e in self.elements if e.name == name), None)


def parse_header(buf: bytes) -> PlyHeader:
    end = buf.find(b"end_header")
    if not buf.startswith(b"ply") or end < 0:
        if not buf:
            raise PlyError("Unexpected EOF while reading PLY data")
        raise PlyError("missing PLY header")
    nl = buf.find(b"\n", end)
    if nl < 0:
        raise PlyError("missing PLY header")
    lines = buf[:end].decode("ascii", errors="replace").replace("\r", "").split("\n")
    fmt, comments, elements = None, [], []
    for line in lines[1:]:
        parts = line.split()
        if not parts:
            continue
        key = parts[0]
        if key == "format":
            fmt = parts[1]
        elif key in ("comment", "obj_info"):
            comments.append(line.split(None, 1)[1] if len(parts) > 1 else "")
        elif key == "element":
            elements.append(PlyElement(parts[1], int(parts[2])))
        elif key == "property":
            if not elements:
                raise PlyError("property before any element")
            if parts[1] == "list":
                elements[-1].properties.append(PlyProperty(parts[4], "", (_TYPES[parts[2]], _TYPES[parts[3]])))
            else:
                if parts[1] not in _TYPES:
                    raise PlyError(f"unknown property type {parts[1]}")
                elements[-1].properties.append(PlyProperty(parts[2], _TYPES[parts[1]]))
    if fmt not in ("ascii", "binary_little_endian", "binary_big_endian"):
        raise PlyError(f"unknown PLY format {fmt}")
    return PlyHeader(fmt, comments, elements, nl + 1)


def _header_metadata(header: PlyHeader):
    """import.rs:206-248: the last 'vertical axis' and 'SplatRenderMode'
    comments.  x maps to +X, y to -Y and z to -Z; three numbers are taken as
    the axis itself."""
    up, mode = None, None
    for c in header.comments:
        s = c.lower()
        if s.startswith("vertical axis: "):
            suffix = s[len("vertical axis: "):].strip()
            named = {"x": (1.0, 0.0, 0.0), "y": (0.0, -1.0, 0.0), "z": (0.0, 0.0, -1.0)}
            if suffix in named:
                up = named[suffix]
            else:
                toks = suffix.replace(",", " ").replace("[", " ").replace("]", " ").split()
                vals = []
                for tok in toks:  # filter_map(parse::<f32>().ok()): unparseable tokens are dropped
                    try:
                        if "_" not in tok:
                            vals.append(float(f32(float(tok))))
                    except ValueError:
                        pass
                if len(vals) == 3:
                    up = tuple(vals)
        if s.startswith("splatrendermode: "):
            m = s[len("splatrendermode: "):].strip()
            if m in ("mip", "default"):
                mode = m
    return up, mode


# ---- element readers ------------------------------------------------------------------------------

class _Body:
    """Reads the elements of a PLY body in order."""

    def __init__(self, buf: bytes, header: PlyHeader):
        self.buf = buf
        self.header = header
        self.pos = header.data_offset
        self.tokens = None
        if header.format == "ascii":
            self.tokens = buf[header.data_offset:].split()
            self.tpos = 0

    def read(self, el: PlyElement) -> np.ndarray:
        if self.header.format == "ascii":
            return self._read_ascii(el)
        endian = "<" if self.header.format == "binary_little_endian" else ">"
        if any(p.list_types for p in el.properties):
            return self._skip_binary_lists(el, endian)
        dt = el.dtype(endian)
        need = dt.itemsize * el.count
        if len(self.buf) - self.pos < need:
            raise PlyError("Unexpected EOF while reading PLY data")
        rows = np.frombuffer(self.buf, dt, el.count, self.pos)
        self.pos += need
        return rows

    def _skip_binary_lists(self, el, endian):
        for _ in range(el.count):
            for p in el.properties:
                if p.list_types:
                    ct = np.dtype(endian + p.list_types[0])
                    if len(self.buf) - self.pos < ct.itemsize:
                        raise PlyError("Unexpected EOF while reading PLY data")
                    n = int(np.frombuffer(self.buf, ct, 1, self.pos)[0])
                    self.pos += ct.itemsize + n * np.dtype(p.list_types[1]).itemsize
                else:
                    self.pos += np.dtype(p.dtype).itemsize
        if self.pos > len(self.buf):
            raise PlyError("Unexpected EOF while reading PLY data")
        return None

    def _read_ascii(self, el):
        if any(p.list_types for p in el.properties):
            for _ in range(el.count):
                for p in el.properties:
                    if self.tpos >= len(self.tokens):
                        raise PlyError("Unexpected EOF while reading PLY data")
                    if p.list_types:
                        self.tpos += 1 + int(self.tokens[self.tpos])
                    else:
                        self.tpos += 1
            return None
        k = len(el.properties)
        need = k * el.count
        if len(self.tokens) - self.tpos < need:
            raise PlyError("Unexpected EOF while reading PLY data")
        toks = self.tokens[self.tpos:self.tpos + need]
        self.tpos += need
        rows = np.empty(el.count, el.dtype("<"))
        try:
            vals = np.array([float(t) for t in toks], np.float64).reshape(el.count, k)
        except ValueError as e:
            raise PlyError(f"invalid ASCII PLY value: {e}") from None
        for j, p in enumerate(el.properties):
            rows[p.name] = vals[:, j].astype(p.dtype)
        return rows


def _validate_sh_rest(names) -> int:
    """import.rs:306-333."""
    idx = []
    for name in names:
        suffix = name[len("f_rest_"):] if name.startswith("f_rest_") else ""
        if not suffix.isdigit():
            raise PlyError(f"Invalid SH property name: {name}")
        idx.append(int(suffix))
    idx.sort()
    if idx != list(range(len(idx))):
        raise PlyError("SH rest properties must be contiguous from f_rest_0")
    if len(idx) not in SH_REST_COUNTS:
        raise PlyError(f"Unsupported SH rest property count: {len(idx)}")
    return len(idx)


def _interleave(dc: np.ndarray, rest: np.ndarray) -> np.ndarray:
    """import.rs:133-144: DC then the rest coefficients, which the file stores
    channel-major (all red, then green, then blue), as [coeff][channel]."""
    n = dc.shape[0]
    cpc = rest.shape[1] // 3
    out = np.empty((n, 1 + cpc, 3), f32)
    out[:, 0, :] = dc
    if cpc:
        out[:, 1:, :] = rest.reshape(n, 3, cpc).transpose(0, 2, 1)
    return out.reshape(n, -1)


def _column(rows, name) -> np.ndarray:
    return rows[name].astype(f32)


def _parse_ply(header: PlyHeader, body: _Body, subsample: int):
    """import.rs:341-502 for the standard layout."""
    vertex = header.get_element("vertex")
    total = vertex.count
    if total == 0:
        raise PlyError("PLY contains no vertices")
    props = vertex.properties
    rest_names = [p.name for p in props if p.name.startswith("f_rest_")]
    rest_count = _validate_sh_rest(rest_names)
    dc_count = sum(p.name in ("f_dc_0", "f_dc_1", "f_dc_2") for p in props)
    chan = lambda a, b: sum(p.name in (a, b) for p in props)
    rgb_channels = [chan("r", "red"), chan("g", "green"), chan("b", "blue")]
    has_rgb = all(c == 1 for c in rgb_channels)
    if dc_count not in (0, 3):
        raise PlyError("PLY SH colors require f_dc_0, f_dc_1, and f_dc_2")
    if any(rgb_channels) and not has_rgb:
        raise PlyError("PLY RGB colors require exactly one red, green, and blue property")
    has_color = dc_count == 3 or has_rgb
    if rest_count > 0 and not has_color:
        raise PlyError("PLY SH rest properties require a complete DC or RGB color")
    for name in ("x", "y", "z"):
        if not vertex.has_property(name):
            raise PlyError(f"missing field `{name}`")
    # the vertex element is read where it lies; elements before it are skipped
    rows = None
    for el in header.elements:
        r = body.read(el)
        if el is vertex:
            rows = r
            break
    rows = rows[::subsample]
    n = rows.shape[0]
    means = np.stack([_column(rows, k) for k in ("x", "y", "z")], 1).reshape(-1)
    get = lambda name: _column(rows, name) if vertex.has_property(name) else np.zeros(n, f32)
    data = SplatData(np.ascontiguousarray(means))
    if vertex.has_property("rot_0"):
        data.rotations = np.stack([get(f"rot_{i}") for i in range(4)], 1).reshape(-1)
    if vertex.has_property("scale_0"):
        data.log_scales = np.stack([get(f"scale_{i}") for i in range(3)], 1).reshape(-1)
    if vertex.has_property("opacity"):
        data.raw_opacities = get("opacity")
    if has_color:
        if has_rgb:
            names = [next(p for p in props if p.name in pair) for pair in (("r", "red"), ("g", "green"),
                                                                             ("b", "blue"))]
            rgb = np.stack([dequant_color(rows[p.name], p.dtype) for p in names], 1)
            dc = rgb_to_sh(rgb)  # import.rs:445-452: RGB overrides the DC terms
        else:
            dc = np.stack([get(f"f_dc_{i}") for i in range(3)], 1)
        rest = np.stack([get(f"f_rest_{i}") for i in range(rest_count)], 1) if rest_count else np.zeros((n, 0), f32)
        data.sh_coeffs = _interleave(dc, rest).reshape(-1)
    return data, -(-total // subsample)


def _parse_compressed(header: PlyHeader, body: _Body, subsample: int):
    """import.rs:504-720: the SuperSplat compressed layout."""
    chunk = header.elements[0]
    metas = body.read(chunk)
    vertex = header.elements[1] if len(header.elements) > 1 else None
    if vertex is None or vertex.name != "vertex":
        raise PlyError("Unknown format")
    total = vertex.count
    if total == 0:
        raise PlyError("PLY contains no vertices")
    required = -(-total // SPLATS_PER_CHUNK)
    if chunk.count < required:
        raise PlyError(f"Compressed PLY has {chunk.count} chunk rows but needs at least {required} for "
                       f"{total} vertices")
    sh_el = header.elements[2] if len(header.elements) > 2 else None
    if sh_el is not None:
        if sh_el.name != "sh" or sh_el.count != total:
            raise PlyError(f"Invalid compressed PLY SH element: expected {total} rows")
        _validate_sh_rest([p.name for p in sh_el.properties])
    rows = body.read(vertex)
    keep = np.arange(0, total, subsample)
    rows = rows[::subsample]
    c = keep // SPLATS_PER_CHUNK

    def lerp(raw, lo, hi):
        mn = np.stack([metas[k][c].astype(f32) for k in lo], 1)
        mx = np.stack([metas[k][c].astype(f32) for k in hi], 1)
        return raw * (mx - mn) + mn

    means = lerp(decode_vec_11_10_11(rows["packed_position"]), ("min_x", "min_y", "min_z"),
                 ("max_x", "max_y", "max_z"))
    log_scales = lerp(decode_vec_11_10_11(rows["packed_scale"]), ("min_scale_x", "min_scale_y", "min_scale_z"),
                      ("max_scale_x", "max_scale_y", "max_scale_z"))
    rot = decode_quat(rows["packed_rotation"])
    rgba = decode_vec_8_8_8_8(rows["packed_color"])
    color = lerp(rgba[:, :3], ("min_r", "min_g", "min_b"), ("max_r", "max_g", "max_b"))
    dc = rgb_to_sh(color)
    opacity = inverse_sigmoid(rgba[:, 3])
    data = SplatData(means.reshape(-1), rot.reshape(-1), log_scales.reshape(-1), dc.reshape(-1), opacity)
    if sh_el is not None:
        sh_rows = body.read(sh_el)[::subsample]
        # QuantSh reads its fields by name: f_rest_0, f_rest_1, ... whatever the file order
        rest = np.stack([dequant_sh(sh_rows[f"f_rest_{k}"]) for k in range(len(sh_el.properties))], 1)
        data.sh_coeffs = _interleave(dc, rest).reshape(-1)
    return data, -(-total // subsample)


def _read_all(source) -> bytes:
    if isinstance(source, (bytes, bytearray, memoryview)):
        return bytes(source)
    if isinstance(source, (str, os.PathLike)):
        with open(source, "rb") as f:
            return f.read()
    return source.read()


def stream_splat_from_ply(source, subsample_points: int | None = None, streaming: bool = False):
    """import.rs:180-296: yields the complete SplatMessage (the reference's
    timed partial messages are a display aid and carry prefixes of it)."""
    if subsample_points == 0:
        raise PlyError("subsample_points must be greater than zero")
    subsample = subsample_points or 1
    buf = _read_all(source)
    if not buf:
        raise PlyError("Unexpected EOF while reading PLY data")
    header = parse_header(buf)
    up, mode = _header_metadata(header)
    has_vertex = header.get_element("vertex") is not None
    body = _Body(buf, header)
    if has_vertex and header.elements[0].name == "chunk":
        data, total = _parse_compressed(header, body, subsample)
    elif has_vertex:
        data, total = _parse_ply(header, body, subsample)
    else:
        raise PlyError("Unknown format")
    yield SplatMessage(ParseMetadata(up, mode, total, 1.0), data)


def load_splat_from_ply(source, subsample_points: int | None = None) -> SplatMessage:
    """import.rs:167-178: the final message of the stream."""
    last = None
    for msg in stream_splat_from_ply(source, subsample_points, False):
        last = msg
    if last is None:
        raise PlyError("Couldn't load single splat from ply")
    return last


# ---- export (export.rs) ---------------------------------------------------------------------------

def _fmt_f32(v) -> str:
    """Rust's Display for f32: shortest round-trip digits, positional."""
    return np.format_float_positional(f32(v), trim="-")


def fold_min_scale(transforms: np.ndarray, raw_opac: np.ndarray, f: np.ndarray):
    """gaussian_splats.rs:139-164 in float32: scales sqrt(s^2 + f^2), opacity
    scaled by sqrt(det(s^2) / det(s^2 + f^2)) and clamped to [1e-6, 1 - 1e-6]."""
    t = np.array(transforms, f32).reshape(-1, 10)
    n = t.shape[0]
    f = np.asarray(f, f32).reshape(n, 1)
    s2 = np.exp(t[:, 7:10] * f32(2.0))
    s2f = s2 + f * f
    t[:, 7:10] = np.log(s2f) * f32(0.5)
    det = lambda a: a[:, 0] * a[:, 1] * a[:, 2]
    coef = np.sqrt(det(s2) / det(s2f))
    sig = f32(1.0) / (f32(1.0) + np.exp(-np.asarray(raw_opac, f32)))
    opac = np.clip(sig * coef, f32(1e-6), f32(1.0 - 1e-6))
    return t, np.log(opac / (f32(1.0) - opac))


def export_rows(transforms: np.ndarray, sh_coeffs: np.ndarray, raw_opac: np.ndarray) -> np.ndarray:
    """export.rs:83-178: [n, 11 + 3C] float32 rows x y z, scale_0..2,
    opacity, rot_0..3 / max(|q|, 1e-12), f_dc_0..2, then the rest
    coefficients channel-major (sh permuted to [n, channel, coeff])."""
    t = np.asarray(transforms, f32).reshape(-1, 10)
    sh = np.asarray(sh_coeffs, f32)
    n, c = t.shape[0], sh.shape[1]
    q = t[:, 3:7]
    # ((q0 q0 + q1 q1) + q2 q2) + q3 q3 in f32; Rust's f32::max drops a NaN like fmax
    rn = np.fmax(np.sqrt(q[:, 0] * q[:, 0] + q[:, 1] * q[:, 1] + q[:, 2] * q[:, 2] + q[:, 3] * q[:, 3]),
                 f32(1e-12))
    cols = np.empty((n, 11 + 3 * c), f32)
    cols[:, 0:3] = t[:, 0:3]
    cols[:, 3:6] = t[:, 7:10]
    cols[:, 6] = np.asarray(raw_opac, f32).reshape(n)
    cols[:, 7:11] = q / rn[:, None]
    cols[:, 11:14] = sh[:, 0, :]
    if c > 1:
        cols[:, 14:] = sh[:, 1:, :].transpose(0, 2, 1).reshape(n, -1)
    return cols


def export_property_names(num_coeffs: int) -> list:
    return ["x", "y", "z", "scale_0", "scale_1", "scale_2", "opacity", "rot_0", "rot_1", "rot_2", "rot_3",
            "f_dc_0", "f_dc_1", "f_dc_2"] + [f"f_rest_{i}" for i in range(3 * (num_coeffs - 1))]


def splat_to_ply(transforms, sh_coeffs, raw_opac, render_mip: bool = False, up_axis=None,
                 min_scale=None) -> bytes:
    """export.rs:180-199: bake the min-scale floor, then one binary
    little-endian vertex element with the reference's comments."""
    if min_scale is not None:
        transforms, raw_opac = fold_min_scale(transforms, raw_opac, min_scale)
    sh = np.asarray(sh_coeffs, f32)
    c = sh.shape[1]
    rows = export_rows(transforms, sh, raw_opac)
    degree = {1: 0, 4: 1, 9: 2, 16: 3, 25: 4}[c]
    comments = ["Exported from Brush"]
    if up_axis is not None:
        comments.append("Vertical axis: " + " ".join(_fmt_f32(v) for v in up_axis))
    else:
        comments.append("Vertical axis: y")
    comments.append(f"SH degree: {degree}")
    comments.append(f"SplatRenderMode: {'mip' if render_mip else 'default'}")
    head = ["ply", "format binary_little_endian 1.0"] + [f"comment {x}" for x in comments]
    head += [f"element vertex {rows.shape[0]}"] + [f"property float {k}" for k in export_property_names(c)]
    head += ["end_header"]
    return ("\n".join(head) + "\n").encode("ascii") + rows.astype("<f4").tobytes()
