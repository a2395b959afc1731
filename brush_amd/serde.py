"""PLY import and export of splats (crates/brush-serde) on the gfx950 library.

Mirrors, with the same names, argument meaning and error messages:

* ``load_splat_from_ply`` / ``stream_splat_from_ply`` (import.rs:167-296):
  the standard 3DGS PLY (ascii, binary little- or big-endian) and the
  SuperSplat compressed PLY, returning ``SplatMessage(meta, data)``;
* ``SplatData`` (import.rs:26-91) with ``num_splats``, ``subsample`` and
  ``into_splats``;
* ``splat_to_ply`` (export.rs:180-199).

The header is parsed and validated on the host exactly where the reference
does it (metadata comments, format detection, SH schema checks, chunk
counts).  The element bytes then go to the device in one copy and one kernel
per element decodes them straight into the splat layout (bh_ply_decode_rows,
bh_ply_decode_compressed); export encodes the rows on the device
(bh_ply_encode_rows) and copies them back behind the header.  ``SplatData``
therefore holds device tensors: transforms [n,10], sh_coeffs [n,C,3] and
raw_opacities [n], already filled with into_splats' defaults where the file
has no such property, plus which groups the file held.  There is no CPU
fallback: without libbrush_hip.so every call raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from ._lib import PlyColumn, PlyCompressedLayout, context, lib, ptr
from .render import SplatRenderMode, Splats

f32 = np.float32
SPLATS_PER_CHUNK = 256               # import.rs:513
SH_REST_COUNTS = (0, 9, 24, 45, 72)  # import.rs:325
CHUNK_FIELDS = ("min_x", "max_x", "min_y", "max_y", "min_z", "max_z", "min_scale_x", "max_scale_x",
                "min_scale_y", "max_scale_y", "min_scale_z", "max_scale_z", "min_r", "max_r", "min_g", "max_g",
                "min_b", "max_b")  # QuantMeta, import.rs:515-534

_TYPES = {"char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1", "short": "i2", "int16": "i2",
          "ushort": "u2", "uint16": "u2", "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
          "float": "f4", "float32": "f4", "double": "f8", "float64": "f8"}
_TYPE_CODES = {"i1": _lib.PLY_I8, "u1": _lib.PLY_U8, "i2": _lib.PLY_I16, "u2": _lib.PLY_U16, "i4": _lib.PLY_I32,
               "u4": _lib.PLY_U32, "f4": _lib.PLY_F32, "f8": _lib.PLY_F64}


class PlyError(ValueError):
    """serde_ply::DeserializeError: the reference's import errors."""


# ---- header --------------------------------------------------------------------------------------

@dataclass
class PlyProperty:
    name: str
    dtype: str                       # numpy code of a scalar property
    list_types: tuple | None = None  # (count dtype, item dtype) of a list property


@dataclass
class PlyElement:
    name: str
    count: int
    properties: list = field(default_factory=list)

    def has_property(self, name: str) -> bool:
        return any(p.name == name for p in self.properties)

    def has_lists(self) -> bool:
        return any(p.list_types for p in self.properties)

    def dtype(self, endian: str = "<") -> np.dtype:
        """Packed row dtype (no padding), in file order."""
        if self.has_lists():
            raise PlyError(f"list properties are not supported in element '{self.name}'")
        return np.dtype([(p.name, endian + p.dtype) for p in self.properties])

    def offsets(self) -> dict:
        d = self.dtype()
        return {name: d.fields[name][1] for name in d.names}


@dataclass
class PlyHeader:
    format: str
    comments: list
    elements: list
    data_offset: int

    def get_element(self, name: str):
        return next((e for e in self.elements if e.name == name), None)

    @property
    def endian(self) -> str:
        return ">" if self.format == "binary_big_endian" else "<"


def parse_header(buf) -> PlyHeader:
    end = buf.find(b"end_header")
    if not bytes(buf[:3]) == b"ply" or end < 0:
        raise PlyError("missing PLY header")
    nl = buf.find(b"\n", end)
    if nl < 0:
        raise PlyError("missing PLY header")
    lines = bytes(buf[:end]).decode("ascii", errors="replace").replace("\r", "").split("\n")
    fmt, comments, elements = None, [], []
    for line in lines[1:]:
        parts = line.split()
        if not parts:
            continue
        key = parts[0]
        try:
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
                    elements[-1].properties.append(PlyProperty(parts[2], _TYPES[parts[1]]))
        except (IndexError, KeyError, ValueError):
            raise PlyError(f"invalid PLY header line: {line!r}") from None
    if fmt not in ("ascii", "binary_little_endian", "binary_big_endian"):
        raise PlyError(f"unknown PLY format {fmt}")
    return PlyHeader(fmt, comments, elements, nl + 1)


def _parse_f32(tok: str):
    """Rust's str::parse::<f32>, or None where it fails."""
    if "_" in tok:
        return None
    try:
        return float(f32(float(tok)))
    except ValueError:
        return None


def header_metadata(header: PlyHeader):
    """import.rs:206-248: the last parseable 'vertical axis' comment (x maps
    to +X, y to -Y, z to -Z; otherwise three numbers split on commas,
    whitespace and brackets, unparseable tokens dropped) and the last
    'SplatRenderMode' comment."""
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
                vals = [v for v in (_parse_f32(t) for t in toks) if v is not None]
                if len(vals) == 3:
                    up = tuple(vals)
        if s.startswith("splatrendermode: "):
            m = s[len("splatrendermode: "):].strip()
            if m == "mip":
                mode = SplatRenderMode.Mip
            elif m == "default":
                mode = SplatRenderMode.Default
    return up, mode


def validate_sh_rest_properties(names) -> int:
    """import.rs:306-333."""
    idx = []
    for name in names:
        suffix = name[len("f_rest_"):] if name.startswith("f_rest_") else ""
        if not (suffix.isascii() and suffix.isdigit()):
            raise PlyError(f"Invalid SH property name: {name}")
        idx.append(int(suffix))
    idx.sort()
    if idx != list(range(len(idx))):
        raise PlyError("SH rest properties must be contiguous from f_rest_0")
    if len(idx) not in SH_REST_COUNTS:
        raise PlyError(f"Unsupported SH rest property count: {len(idx)}")
    return len(idx)


# ---- element bytes -------------------------------------------------------------------------------

def _unexpected_eof():
    return PlyError("Unexpected EOF while reading PLY data")


class _Body:
    """The element bodies in file order.  Binary elements are located in
    place; an ASCII body is tokenised once and each element converted to
    packed little-endian rows."""

    def __init__(self, buf: np.ndarray, length: int, header: PlyHeader):
        self.buf = buf
        self.length = length
        self.header = header
        self.pos = header.data_offset
        if header.format == "ascii":
            self.tokens = bytes(buf[header.data_offset:length]).split()
            self.tpos = 0

    def element(self, el: PlyElement):
        """(host uint8 array holding the rows, byte start, little-endian?) of
        the next element, after checking that all its rows are present."""
        if self.header.format == "ascii":
            return self._ascii(el)
        if el.has_lists():
            self._skip_binary_lists(el)
            return None
        need = el.dtype().itemsize * el.count
        if self.length - self.pos < need:
            raise _unexpected_eof()
        start = self.pos
        self.pos += need
        return self.buf, start, self.header.format == "binary_little_endian"

    def rows(self, el: PlyElement) -> np.ndarray:
        """Structured numpy rows of a small element (chunk metadata)."""
        loc = self.element(el)
        buf, start, little = loc
        return np.frombuffer(buf, el.dtype("<" if little else ">"), el.count, start)

    def _skip_binary_lists(self, el):
        endian = self.header.endian
        for _ in range(el.count):
            for p in el.properties:
                if p.list_types:
                    ct = np.dtype(endian + p.list_types[0])
                    if self.length - self.pos < ct.itemsize:
                        raise _unexpected_eof()
                    n = int(np.frombuffer(self.buf, ct, 1, self.pos)[0])
                    self.pos += ct.itemsize + n * np.dtype(p.list_types[1]).itemsize
                else:
                    self.pos += np.dtype(p.dtype).itemsize
        if self.pos > self.length:
            raise _unexpected_eof()

    def _ascii(self, el):
        if el.has_lists():
            for _ in range(el.count):
                for p in el.properties:
                    if self.tpos >= len(self.tokens):
                        raise _unexpected_eof()
                    self.tpos += 1 + int(self.tokens[self.tpos]) if p.list_types else 1
            return None
        k = len(el.properties)
        need = k * el.count
        if len(self.tokens) - self.tpos < need:
            raise _unexpected_eof()
        toks = self.tokens[self.tpos:self.tpos + need]
        self.tpos += need
        try:
            vals = np.array(toks, dtype=np.float64).reshape(el.count, k) if need else np.zeros((el.count, k))
        except ValueError as e:
            raise PlyError(f"invalid ASCII PLY value: {e}") from None
        rows = np.empty(el.count, el.dtype("<"))
        for j, p in enumerate(el.properties):
            rows[p.name] = vals[:, j].astype(p.dtype)
        raw = np.zeros(rows.nbytes + 8, np.uint8)
        raw[:rows.nbytes] = rows.view(np.uint8).reshape(-1)
        return raw, 0, True


_STAGING_BYTES = 32 << 20
_staging: dict = {}


def _staging_buffers(device: torch.device):
    """Two pinned host buffers per device, kept for the process, each with
    the event of the last copy out of it."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    bufs = _staging.get(key)
    if bufs is None:
        bufs = [(torch.empty(_STAGING_BYTES, dtype=torch.uint8, pin_memory=True), torch.cuda.Event())
                for _ in range(2)]
        _staging[key] = bufs
    return bufs


def _to_device(loc, nbytes: int, device) -> torch.Tensor:
    """The element's bytes in a fresh device buffer of nbytes rounded up to
    4, plus 4 zero bytes.  Large elements stream through the pinned staging
    buffers (host copy of one chunk overlapping the DMA of the other); the
    copies are ordered on the current stream before the decode kernel."""
    buf, start, _ = loc
    padded = (nbytes + 3) // 4 * 4 + 4
    dev = torch.empty(padded, dtype=torch.uint8, device=device)
    dev[nbytes:].zero_()
    src = buf[start:start + nbytes]
    if nbytes <= (1 << 20):
        dev[:nbytes].copy_(torch.from_numpy(np.array(src)))
        return dev
    bufs = _staging_buffers(dev.device)
    stream = torch.cuda.current_stream(dev.device)
    for k, off in enumerate(range(0, nbytes, _STAGING_BYTES)):
        n = min(_STAGING_BYTES, nbytes - off)
        pin, ev = bufs[k % 2]
        ev.synchronize()  # the copy that last read this buffer has finished
        pin.numpy()[:n] = src[off:off + n]
        dev[off:off + n].copy_(pin[:n], non_blocking=True)
        ev.record(stream)
    return dev


def _header_bytes(buf: np.ndarray, length: int) -> bytes:
    """The leading bytes that hold the header (all of them if needed)."""
    head = bytes(buf[:min(length, 1 << 16)])
    if b"end_header" in head or length <= (1 << 16):
        return head
    return bytes(buf[:length])


def _read_source(source):
    """(read-only uint8 view of the whole file, length): a path is
    memory-mapped, bytes-like data is viewed in place."""
    if isinstance(source, (str, os.PathLike)):
        size = os.path.getsize(source)
        if size == 0:
            return np.zeros(0, np.uint8), 0
        return np.memmap(source, dtype=np.uint8, mode="r"), size
    data = source if isinstance(source, (bytes, bytearray, memoryview)) else source.read()
    view = np.frombuffer(data, np.uint8)
    return view, view.size


# ---- parsed data ---------------------------------------------------------------------------------

@dataclass
class ParseMetadata:
    """import.rs:19-24"""
    up_axis: tuple | None
    render_mode: SplatRenderMode | None
    total_splats: int
    progress: float


class SplatData:
    """import.rs:26-91.  Holds the decoded splats on the device in the
    layout Splats uses; ``means`` / ``rotations`` / ``log_scales`` /
    ``sh_coeffs`` / ``raw_opacities`` return the reference's flat vectors
    (device tensors), or None for a group the file does not hold."""

    def __init__(self, transforms: torch.Tensor, sh_coeffs: torch.Tensor, raw_opacities: torch.Tensor,
                 has_rotations: bool, has_log_scales: bool, has_sh_coeffs: bool, has_raw_opacities: bool):
        self.transforms = transforms
        self.sh = sh_coeffs
        self.opac = raw_opacities
        self.has_rotations = has_rotations
        self.has_log_scales = has_log_scales
        self.has_sh_coeffs = has_sh_coeffs
        self.has_raw_opacities = has_raw_opacities

    @property
    def means(self) -> torch.Tensor:
        return self.transforms[:, 0:3].reshape(-1)

    @property
    def rotations(self):
        return self.transforms[:, 3:7].reshape(-1) if self.has_rotations else None

    @property
    def log_scales(self):
        return self.transforms[:, 7:10].reshape(-1) if self.has_log_scales else None

    @property
    def sh_coeffs(self):
        return self.sh.reshape(-1) if self.has_sh_coeffs else None

    @property
    def raw_opacities(self):
        return self.opac if self.has_raw_opacities else None

    def num_splats(self) -> int:
        return int(self.transforms.shape[0])

    def subsample(self, max_splats: int) -> "SplatData":
        """import.rs:49-74: keep every ceil(n / max_splats)-th splat."""
        n = self.num_splats()
        if max_splats == 0 or n <= max_splats:
            return self
        step = -(-n // max_splats)
        return SplatData(self.transforms[::step].contiguous(), self.sh[::step].contiguous(),
                         self.opac[::step].contiguous(), self.has_rotations, self.has_log_scales,
                         self.has_sh_coeffs, self.has_raw_opacities)

    def into_splats(self, mode: SplatRenderMode = SplatRenderMode.Default) -> Splats:
        """import.rs:77-91; the defaults are already in place."""
        return Splats(self.transforms, self.sh, self.opac, mode is SplatRenderMode.Mip)


@dataclass
class SplatMessage:
    meta: ParseMetadata
    data: SplatData


# ---- decoding ------------------------------------------------------------------------------------

def _column(prop: PlyProperty | None, offset: int, op: int = _lib.PLY_OP_PLAIN, konst: float = 0.0) -> PlyColumn:
    if prop is None:
        return PlyColumn(0, _lib.PLY_CONST, 0, konst)
    return PlyColumn(offset, _TYPE_CODES[prop.dtype], op, 0.0)


def _outputs(n: int, num_coeffs: int, device):
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("PLY rows are decoded on the GPU (libbrush_hip.so); no ROCm device is visible")
        device = torch.device("cuda", torch.cuda.current_device())
    return (torch.empty((n, 10), dtype=torch.float32, device=device),
            torch.empty((n, num_coeffs, 3), dtype=torch.float32, device=device),
            torch.empty((n,), dtype=torch.float32, device=device))


@dataclass
class VertexLayout:
    """A standard vertex element resolved into the decoder's column table."""
    columns: list
    num_coeffs: int
    row_bytes: int
    has_rotations: bool
    has_log_scales: bool
    has_sh_coeffs: bool
    has_raw_opacities: bool


def vertex_layout(vertex: PlyElement) -> VertexLayout:
    """import.rs:357-403: the schema checks of parse_ply, then one column per
    output value (x y z rot_0..3 scale_0..2 | opacity | sh[c][channel])."""
    props = {p.name: p for p in vertex.properties}
    rest_count = validate_sh_rest_properties(p.name for p in vertex.properties if p.name.startswith("f_rest_"))
    dc_count = sum(p.name in ("f_dc_0", "f_dc_1", "f_dc_2") for p in vertex.properties)
    chan = lambda a, b: sum(p.name in (a, b) for p in vertex.properties)
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
        if name not in props:
            raise PlyError(f"missing field `{name}`")
    if vertex.has_lists():
        raise PlyError("list properties are not supported in element 'vertex'")
    off = vertex.offsets()
    col = lambda name, konst=0.0: _column(props.get(name), off.get(name, 0), konst=konst)
    has_rot, has_scale, has_opac = "rot_0" in props, "scale_0" in props, "opacity" in props
    cols = [col("x"), col("y"), col("z")]
    # PlyGaussian's serde defaults are 0 for a missing member of a present
    # group; a missing group takes into_splats' default
    cols += [col(f"rot_{k}") for k in range(4)] if has_rot else [_column(None, 0, konst=v) for v in (1, 0, 0, 0)]
    cols += [col(f"scale_{k}") for k in range(3)] if has_scale else [_column(None, 0, konst=-4.0)] * 3
    cols.append(col("opacity"))  # inverse_sigmoid(0.5) = ln(1) = 0
    if has_color:
        cpc = rest_count // 3
        num_coeffs = 1 + cpc
        if has_rgb:  # import.rs:445-452: RGB overrides the DC terms
            for a, b in (("r", "red"), ("g", "green"), ("b", "blue")):
                p = props.get(a) or props.get(b)
                if p.dtype not in ("u1", "u2", "f4"):
                    raise PlyError(f"invalid type for colour property {p.name}: expected u8, u16 or float")
                cols.append(_column(p, off[p.name], _lib.PLY_OP_COLOR))
        else:
            cols += [col(f"f_dc_{k}") for k in range(3)]
        # import.rs:133-144: coefficient c of channel ch is f_rest_{ch * cpc + c - 1}
        for c in range(1, num_coeffs):
            cols += [col(f"f_rest_{ch * cpc + c - 1}") for ch in range(3)]
    else:
        num_coeffs = 1
        cols += [_column(None, 0, konst=0.5)] * 3
    return VertexLayout(cols, num_coeffs, vertex.dtype().itemsize, has_rot, has_scale, has_color, has_opac)


def decode_rows(rows: torch.Tensor, layout: VertexLayout, num_rows: int, subsample: int = 1,
                big_endian: bool = False, out=None) -> SplatData:
    """bh_ply_decode_rows over a device byte buffer holding ``num_rows`` rows
    (its length a multiple of 4 at least num_rows * row_bytes).  ``out``:
    optional (transforms, sh, raw_opac) tensors to write into."""
    n = -(-num_rows // subsample)
    t, sh, o = out if out is not None else _outputs(n, layout.num_coeffs, rows.device)
    with torch.cuda.device(rows.device):
        table = (PlyColumn * len(layout.columns))(*layout.columns)
        ctx = context()
        flags = _lib.PLY_BIG_ENDIAN if big_endian else 0
        ctx.check(lib().bh_ply_decode_rows(ctx.handle, ptr(rows), rows.numel(), layout.row_bytes, num_rows, subsample,
                                           flags, table, layout.num_coeffs, ptr(t), ptr(sh), ptr(o)),
                  "ply_decode_rows")
    return SplatData(t, sh, o, layout.has_rotations, layout.has_log_scales, layout.has_sh_coeffs,
                     layout.has_raw_opacities)


def _parse_ply(header: PlyHeader, body: _Body, subsample: int, device):
    """import.rs:341-502: schema checks on the host, rows on the device."""
    vertex = header.get_element("vertex")
    total = vertex.count
    max_splats = -(-total // subsample)
    if total == 0:
        raise PlyError("PLY contains no vertices")
    layout = vertex_layout(vertex)
    # the vertex element's bytes (elements before it are skipped)
    loc = None
    for el in header.elements:
        got = body.element(el)
        if el is vertex:
            loc = got
            break
    out = _outputs(max_splats, layout.num_coeffs, device)
    with torch.cuda.device(out[0].device):
        rows = _to_device(loc, layout.row_bytes * total, out[0].device)
    return decode_rows(rows, layout, total, subsample, not loc[2], out), max_splats


def _parse_compressed(header: PlyHeader, body: _Body, subsample: int, device):
    """import.rs:504-720."""
    chunk = header.elements[0]
    metas = body.rows(chunk) if chunk.count else None
    vertex = header.elements[1] if len(header.elements) > 1 else None
    if vertex is None or vertex.name != "vertex":
        raise PlyError("Unknown format")
    total = vertex.count
    max_splats = -(-total // subsample)
    if total == 0:
        raise PlyError("PLY contains no vertices")
    required = -(-total // SPLATS_PER_CHUNK)
    if chunk.count < required:
        raise PlyError(f"Compressed PLY has {chunk.count} chunk rows but needs at least {required} for "
                       f"{total} vertices")
    sh_el = header.elements[2] if len(header.elements) > 2 else None
    rest_count = 0
    if sh_el is not None:
        if sh_el.name != "sh" or sh_el.count != total:
            raise PlyError(f"Invalid compressed PLY SH element: expected {total} rows")
        rest_count = validate_sh_rest_properties(p.name for p in sh_el.properties)
    # QuantMeta rows: every field must be present (import.rs:515-534)
    chunk_arr = np.empty((chunk.count, 18), f32)
    for k, name in enumerate(CHUNK_FIELDS):
        if not chunk.has_property(name):
            raise PlyError(f"missing field `{name}`")
        chunk_arr[:, k] = metas[name].astype(f32)
    layout = PlyCompressedLayout()
    if vertex.has_lists():
        raise PlyError("list properties are not supported in element 'vertex'")
    voff = vertex.offsets()
    for name in ("packed_position", "packed_scale", "packed_rotation", "packed_color"):
        p = next((q for q in vertex.properties if q.name == name), None)
        if p is None:
            raise PlyError(f"missing field `{name}`")
        if p.dtype not in ("u4", "i4"):
            raise PlyError(f"invalid type for {name}: expected a 32-bit integer")
        setattr(layout, name.replace("packed_", "") + "_offset", voff[name])
    layout.vertex_row_bytes = vertex.dtype().itemsize
    vloc = body.element(vertex)
    sloc = None
    if sh_el is not None:
        if any(p.dtype != "u1" for p in sh_el.properties):
            raise PlyError("compressed SH properties must be uchar")
        soff = sh_el.offsets()
        for p in sh_el.properties:
            layout.sh_offsets[int(p.name[len("f_rest_"):])] = soff[p.name]
        layout.sh_row_bytes = sh_el.dtype().itemsize
        layout.sh_rest_count = rest_count
        sloc = body.element(sh_el)
    num_coeffs = 1 + rest_count // 3
    t, sh, o = _outputs(max_splats, num_coeffs, device)
    device = t.device
    with torch.cuda.device(device):
        chunks_dev = torch.from_numpy(chunk_arr).to(device)
        vrows = _to_device(vloc, layout.vertex_row_bytes * total, device)
        srows = _to_device(sloc, layout.sh_row_bytes * total, device) if sloc is not None else None
        ctx = context()
        flags = 0 if vloc[2] else _lib.PLY_BIG_ENDIAN
        ctx.check(lib().bh_ply_decode_compressed(ctx.handle, ptr(chunks_dev), chunk.count, ptr(vrows), vrows.numel(),
                                                 ptr(srows), 0 if srows is None else srows.numel(), total, subsample,
                                                 flags, ctypes.byref(layout), ptr(t), ptr(sh), ptr(o)),
                  "ply_decode_compressed")
    return SplatData(t, sh, o, True, True, True, True), max_splats


def stream_splat_from_ply(source, subsample_points: int | None = None, streaming: bool = False, device=None):
    """import.rs:180-296.  Yields SplatMessage values; the last is complete.
    The reference's timed partial messages exist to show a file while its
    rows are still being parsed; decoding a whole element here is one kernel,
    so the stream yields the complete message only."""
    if subsample_points == 0:
        raise PlyError("subsample_points must be greater than zero")
    subsample = subsample_points or 1
    buf, length = _read_source(source)
    if length == 0:
        raise _unexpected_eof()
    header = parse_header(_header_bytes(buf, length))
    up, mode = header_metadata(header)
    has_vertex = header.get_element("vertex") is not None
    body = _Body(buf, length, header)
    dev = torch.device(device) if device is not None else None
    if has_vertex and header.elements[0].name == "chunk":
        data, total = _parse_compressed(header, body, subsample, dev)
    elif has_vertex:
        data, total = _parse_ply(header, body, subsample, dev)
    else:
        raise PlyError("Unknown format")
    yield SplatMessage(ParseMetadata(up, mode, total, 1.0), data)


def load_splat_from_ply(source, subsample_points: int | None = None, device=None) -> SplatMessage:
    """import.rs:167-178: the final message of the stream."""
    last = None
    for msg in stream_splat_from_ply(source, subsample_points, False, device):
        last = msg
    if last is None:
        raise PlyError("Couldn't load single splat from ply")
    return last


# ---- export --------------------------------------------------------------------------------------

def _fmt_f32(v) -> str:
    """Rust's Display for f32: the shortest digits that round-trip, positional."""
    return np.format_float_positional(f32(v), trim="-")


def export_property_names(num_coeffs: int) -> list:
    """DynamicPlyGaussian's fields in serialisation order (export.rs:42-76)."""
    return ["x", "y", "z", "scale_0", "scale_1", "scale_2", "opacity", "rot_0", "rot_1", "rot_2", "rot_3",
            "f_dc_0", "f_dc_1", "f_dc_2"] + [f"f_rest_{i}" for i in range(3 * (num_coeffs - 1))]


def encode_rows(transforms: torch.Tensor, sh_coeffs: torch.Tensor, raw_opac: torch.Tensor) -> torch.Tensor:
    """The export rows on the device: f32 [n, 11 + 3C] (bh_ply_encode_rows)."""
    n, c = int(transforms.shape[0]), int(sh_coeffs.shape[1])
    if transforms.dtype != torch.float32 or sh_coeffs.dtype != torch.float32 or raw_opac.dtype != torch.float32:
        raise ValueError("splat tensors must be float32")
    rows = torch.empty((n, 11 + 3 * c), dtype=torch.float32, device=transforms.device)
    with torch.cuda.device(transforms.device):
        ctx = context()
        ctx.check(lib().bh_ply_encode_rows(ctx.handle, ptr(transforms.contiguous()), ptr(sh_coeffs.contiguous()),
                                           ptr(raw_opac.contiguous()), n, c, ptr(rows)), "ply_encode_rows")
    return rows


def splat_to_ply(splats: Splats, up_axis=None) -> bytes:
    """export.rs:180-199: bake the min-scale floor, encode the rows on the
    device and write them as one binary little-endian vertex element behind
    the reference's header comments."""
    splats = splats.bake_min_scale()
    c = int(splats.sh_coeffs.shape[1])
    degree = {1: 0, 4: 1, 9: 2, 16: 3, 25: 4}.get(c)
    if degree is None:
        raise ValueError(f"Invalid nr. of sh bases {c}")
    rows = encode_rows(splats.transforms.detach(), splats.sh_coeffs.detach(), splats.raw_opacities.detach())
    comments = ["Exported from Brush"]
    if up_axis is not None:
        comments.append("Vertical axis: " + " ".join(_fmt_f32(v) for v in up_axis))
    else:
        comments.append("Vertical axis: y")
    comments.append(f"SH degree: {degree}")
    comments.append(f"SplatRenderMode: {'mip' if splats.render_mip else 'default'}")
    head = ["ply", "format binary_little_endian 1.0"] + [f"comment {x}" for x in comments]
    head += [f"element vertex {rows.shape[0]}"] + [f"property float {k}" for k in export_property_names(c)]
    head += ["end_header"]
    body = rows.cpu().numpy().astype("<f4", copy=False).tobytes()
    return ("\n".join(head) + "\n").encode("ascii") + body
