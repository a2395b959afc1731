"""PLY files for the serde tests: the brush-serde crate's own test fixtures
(crates/brush-serde/src/import.rs:760-897, lib.rs:26-71) rebuilt as bytes,
and seeded generators of standard and compressed files with independent
encoders (the SuperSplat packing written from its published format)."""
from __future__ import annotations

import struct

import numpy as np

f32 = np.float32

# ---- the crate's fixtures (import.rs:760-897) ------------------------------------------------

def truncated_binary_ply() -> bytes:
    data = b"ply\nformat binary_little_endian 1.0\nelement vertex 2\nproperty float x\nproperty float y\n" \
           b"property float z\nend_header\n"
    data += struct.pack("<3f", 1.0, 2.0, 3.0)
    return data + struct.pack("<f", 4.0)  # only the first property of the second vertex


def ascii_ply(vertex_count: int, rows: str) -> bytes:
    return (f"ply\nformat ascii 1.0\nelement vertex {vertex_count}\nproperty float x\nproperty float y\n"
            f"property float z\nend_header\n{rows}").encode()


def ascii_ply_with_properties(properties) -> bytes:
    data = b"ply\nformat ascii 1.0\nelement vertex 1\nproperty float x\nproperty float y\nproperty float z\n"
    for p in properties:
        data += f"property float {p}\n".encode()
    return data + b"end_header\n"


CHUNK_PROPS = ["min_x", "max_x", "min_y", "max_y", "min_z", "max_z", "min_scale_x", "max_scale_x", "min_scale_y",
               "max_scale_y", "min_scale_z", "max_scale_z", "min_r", "max_r", "min_g", "max_g", "min_b", "max_b"]


def compressed_ply_header(chunk_count: int, vertex_count: int, sh=None, fmt="binary_little_endian") -> bytes:
    h = f"ply\nformat {fmt} 1.0\nelement chunk {chunk_count}\n"
    h += "".join(f"property float {p}\n" for p in CHUNK_PROPS)
    h += f"element vertex {vertex_count}\nproperty uint packed_position\nproperty uint packed_scale\n" \
         f"property uint packed_rotation\nproperty uint packed_color\n"
    if sh is not None:
        sh_count, prop_count = sh
        h += f"element sh {sh_count}\n" + "".join(f"property uchar f_rest_{i}\n" for i in range(prop_count))
    return (h + "end_header\n").encode()


def truncated_compressed_chunk_ply() -> bytes:
    return compressed_ply_header(1, 1) + struct.pack("<f", 0.0)


def truncated_compressed_vertex_ply() -> bytes:
    return compressed_ply_header(1, 1) + bytes(18 * 4) + struct.pack("<I", 0)


def truncated_compressed_sh_ply() -> bytes:
    return compressed_ply_header(1, 1, (1, 9)) + bytes(18 * 4) + bytes(4 * 4)


def compressed_ply_with_sh() -> bytes:
    return compressed_ply_header(1, 1, (1, 9)) + bytes(18 * 4) + bytes(4 * 4) + bytes([0, 32, 64, 96, 127, 160,
                                                                                         192, 224, 255])


def compressed_ply_one_vertex() -> bytes:
    return compressed_ply_header(1, 1) + bytes(18 * 4) + bytes(4 * 4)


def compressed_ply_with_oversized_sh_header() -> bytes:
    return compressed_ply_header(1, 1, (1, 75)) + bytes(18 * 4)


def compressed_ply_without_chunk_metadata() -> bytes:
    return compressed_ply_header(0, 1) + bytes(4 * 4)


def create_test_splats(sh_degree: int, num_splats: int = 1):
    """lib.rs:26-71 (create_test_splats_with_count): transforms [n,10],
    sh [n,C,3], raw opacities [n] as float32 arrays."""
    c = (sh_degree + 1) ** 2
    means, rots, scales, sh, opac = [], [], [], [], []
    for i in range(num_splats):
        o = f32(i)
        means += [o, o + f32(1.0), o + f32(2.0)]
        rots += [1.0, 0.0, 0.0, 0.0]
        scales += [f32(-0.1) + o * f32(0.05), f32(0.2) + o * f32(0.05), f32(-0.3) + o * f32(0.05)]
        for _ in range(3):
            sh.append(f32(0.5) + o * f32(0.1))
            for j in range(1, c):
                sh.append(f32(j) * f32(0.1) + o * f32(0.01))
        opac.append(f32(0.8) - o * f32(0.1))
    n = num_splats
    t = np.concatenate([np.array(means, f32).reshape(n, 3), np.array(rots, f32).reshape(n, 4),
                        np.array(scales, f32).reshape(n, 3)], 1)
    return t, np.array(sh, f32).reshape(n, c, 3), np.array(opac, f32)


# ---- generators -------------------------------------------------------------------------------

def write_ply(fmt: str, elements, comments=()) -> bytes:
    """elements: [(name, structured array)] written in the given format."""
    names = {"i1": "char", "u1": "uchar", "i2": "short", "u2": "ushort", "i4": "int", "u4": "uint",
             "f4": "float", "f8": "double"}
    h = ["ply", f"format {fmt} 1.0"] + [f"comment {c}" for c in comments]
    for name, arr in elements:
        h.append(f"element {name} {arr.shape[0]}")
        for fld in arr.dtype.names:
            h.append(f"property {names[arr.dtype[fld].str[1:]]} {fld}")
    out = ("\n".join(h + ["end_header"]) + "\n").encode()
    for _, arr in elements:
        if fmt == "ascii":
            lines = []
            for row in arr:
                vals = []
                for fld in arr.dtype.names:
                    v = row[fld]
                    vals.append(repr(float(v)) if arr.dtype[fld].kind == "f" else str(int(v)))
                lines.append(" ".join(vals))
            out += ("\n".join(lines) + "\n").encode()
        else:
            endian = "<" if fmt == "binary_little_endian" else ">"
            out += arr.astype(arr.dtype.newbyteorder(endian)).tobytes()
    return out


def standard_rows(rng, n: int, rest: int = 45, color: str = "dc", groups=("rot", "scale", "opacity"),
                  extra=(), shuffle: bool = False, types=None) -> np.ndarray:
    """A structured vertex array: x y z, optional groups, colour as f_dc or
    red/green/blue of the named kind, ``rest`` f_rest properties and extra
    properties (name, dtype)."""
    fields = [("x", "f4"), ("y", "f4"), ("z", "f4")]
    if "normals" in extra:
        fields += [("nx", "f4"), ("ny", "f4"), ("nz", "f4")]
    if color == "dc":
        fields += [(f"f_dc_{k}", "f4") for k in range(3)]
    elif color != "none":
        kind = {"rgb_u8": "u1", "rgb_u16": "u2", "rgb_f32": "f4"}[color]
        fields += [(c, kind) for c in ("red", "green", "blue")]
    fields += [(f"f_rest_{k}", "f4") for k in range(rest)]
    if "opacity" in groups:
        fields.append(("opacity", "f4"))
    if "scale" in groups:
        fields += [(f"scale_{k}", "f4") for k in range(3)]
    if "rot" in groups:
        fields += [(f"rot_{k}", "f4") for k in range(4)]
    for name, dt in extra:
        if name != "normals":
            fields.append((name, dt))
    if types:
        fields = [(nm, types.get(nm, dt)) for nm, dt in fields]
    if shuffle:
        order = rng.permutation(len(fields))
        fields = [fields[i] for i in order]
    arr = np.zeros(n, np.dtype(fields))
    for nm, dt in fields:
        k = np.dtype(dt).kind
        if k == "f":
            arr[nm] = rng.standard_normal(n).astype(dt)
        else:
            info = np.iinfo(np.dtype(dt))
            arr[nm] = rng.integers(info.min, int(info.max) + 1, n, dtype=np.int64).astype(dt)
    return arr


def encode_quat(q: np.ndarray) -> np.ndarray:
    """SuperSplat's smallest-three packing: the largest |component| index in
    the top two bits, the quaternion's sign chosen so that it is positive,
    the other three (in w x y z order) as v / sqrt(2) + 0.5 in 10-bit
    unorms."""
    q = np.asarray(q, np.float64)
    q = q / np.linalg.norm(q, axis=1, keepdims=True)
    largest = np.argmax(np.abs(q), axis=1)
    q = q * np.where(q[np.arange(len(q)), largest] < 0, -1.0, 1.0)[:, None]
    out = (largest.astype(np.uint32) << 30)
    shift = [20, 10, 0]
    for i in range(len(q)):
        others = [q[i, k] for k in range(4) if k != largest[i]]
        for s, v in zip(shift, others):
            u = int(np.clip(np.round((v / np.sqrt(2.0) + 0.5) * 1023.0), 0, 1023))
            out[i] |= np.uint32(u << s)
    return out


def encode_unorm3(v: np.ndarray, bits=(11, 10, 11)) -> np.ndarray:
    """Three values in [0, 1] packed x | y | z from the most significant bit."""
    v = np.clip(np.asarray(v, np.float64), 0.0, 1.0)
    a = np.round(v[:, 0] * ((1 << bits[0]) - 1)).astype(np.uint32)
    b = np.round(v[:, 1] * ((1 << bits[1]) - 1)).astype(np.uint32)
    c = np.round(v[:, 2] * ((1 << bits[2]) - 1)).astype(np.uint32)
    return (a << (bits[1] + bits[2])) | (b << bits[2]) | c


def compressed_elements(rng, n: int, rest: int = 0, shuffle: bool = False):
    """(chunk rows, vertex rows, sh rows or None, the float64 values they encode)."""
    chunks = -(-n // 256)
    cm = np.zeros(chunks, np.dtype([(p, "f4") for p in CHUNK_PROPS]))
    for axis in ("x", "y", "z"):
        lo = rng.uniform(-5, 0, chunks).astype(f32)
        cm[f"min_{axis}"], cm[f"max_{axis}"] = lo, lo + rng.uniform(0.5, 5, chunks).astype(f32)
        lo = rng.uniform(-8, -3, chunks).astype(f32)
        cm[f"min_scale_{axis}"], cm[f"max_scale_{axis}"] = lo, lo + rng.uniform(0.5, 4, chunks).astype(f32)
    for c in ("r", "g", "b"):
        lo = rng.uniform(-0.5, 0.3, chunks).astype(f32)
        cm[f"min_{c}"], cm[f"max_{c}"] = lo, lo + rng.uniform(0.2, 1.5, chunks).astype(f32)
    q = rng.standard_normal((n, 4))
    vfields = [("packed_position", "u4"), ("packed_scale", "u4"), ("packed_rotation", "u4"), ("packed_color", "u4")]
    if shuffle:
        vfields = [vfields[i] for i in rng.permutation(4)] + [("pad", "u1")]
    vert = np.zeros(n, np.dtype(vfields))
    vert["packed_position"] = encode_unorm3(rng.uniform(0, 1, (n, 3)))
    vert["packed_scale"] = encode_unorm3(rng.uniform(0, 1, (n, 3)))
    vert["packed_rotation"] = encode_quat(q)
    vert["packed_color"] = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    sh = None
    if rest:
        names = [f"f_rest_{k}" for k in range(rest)]
        if shuffle:
            names = [names[i] for i in rng.permutation(rest)]
        sh = np.zeros(n, np.dtype([(nm, "u1") for nm in names]))
        for nm in names:
            sh[nm] = rng.integers(0, 256, n, dtype=np.int64).astype(np.uint8)
    return cm, vert, sh, q
