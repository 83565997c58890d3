"""CPU restatement of the scene file format — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker of
``gaussian_splats_hip.splats.ply`` (host parse, GPU record split and pack).

Restates src/gaussian_splats/splats/ply.py: ``save_ply`` (ply.py:12-52) writes
one binary little-endian PLY ``vertex`` element of float32 properties x y z nx
ny nz f_dc_0..2 f_rest_0..3(K-1)-1 opacity scale_0..2 rot_0..3 with
f_rest_{c (K-1) + k - 1} = color[k][c] (``color[:, 1:].transpose(0, 2, 1)``,
ply.py:36); ``load_ply`` (ply.py:55-89) reads the properties by name, so
property order, extra properties and other elements do not matter, and
missing normals read as zeros.  The third-party reader the reference uses
(plyfile, absent here) is replaced by the PLY format itself (Greg Turk's
specification: an ASCII header, then each element's rows in the declared
property order and types, ``binary_little_endian``, ``binary_big_endian`` or
``ascii``).  Written with ``struct`` and Python loops value by value, for small
files only.  Pinned by tests/test_ply_host.py: hand-assembled bytes of a
two-Gaussian file (the header text and each value's position written out),
and files of other layouts built value by value.
"""

from __future__ import annotations

import math
import struct

_TYPES = {
    "char": "b", "int8": "b", "uchar": "B", "uint8": "B",
    "short": "h", "int16": "h", "ushort": "H", "uint16": "H",
    "int": "i", "int32": "i", "uint": "I", "uint32": "I",
    "float": "f", "float32": "f", "double": "d", "float64": "d",
}


def save_fields(k: int) -> list[str]:
    """Property names of save_ply for K SH coefficients (ply.py:23-30)."""
    return (
        ["x", "y", "z", "nx", "ny", "nz"]
        + [f"f_dc_{i}" for i in range(3)]
        + [f"f_rest_{i}" for i in range((k - 1) * 3)]
        + ["opacity"]
        + [f"scale_{i}" for i in range(3)]
        + [f"rot_{i}" for i in range(4)]
    )


def save_ply_bytes(state: dict) -> bytes:
    """The file save_ply writes for ``state`` (nested lists or arrays of
    floats: mean [N][3], rotation [N][4], scale [N][3], opacity [N][1],
    color [N][K][3], optional normals [N][3])."""
    mean, rotation, scale = state["mean"], state["rotation"], state["scale"]
    opacity, color = state["opacity"], state["color"]
    n = len(mean)
    normals = state.get("normals")
    if normals is None:
        normals = [[0.0, 0.0, 0.0] for _ in range(n)]
    k = len(color[0]) if n else 1
    fields = save_fields(k)
    header = ["ply", "format binary_little_endian 1.0", f"element vertex {n}"]
    header += [f"property float {f}" for f in fields]
    header += ["end_header"]
    out = bytearray(("\n".join(header) + "\n").encode("ascii"))
    for g in range(n):
        row = list(mean[g]) + list(normals[g]) + [color[g][0][c] for c in range(3)]
        for c in range(3):  # channel-major higher bands
            for kk in range(1, k):
                row.append(color[g][kk][c])
        row += [opacity[g][0]] + list(scale[g]) + list(rotation[g])
        for v in row:
            out += struct.pack("<f", float(v))
    return bytes(out)


def parse_header(data: bytes) -> tuple[str, list[dict], int]:
    """(format, elements, data offset); each element is {name, count,
    properties: [(name, type) or (name, ("list", count type, item type))]}."""
    end = data.index(b"end_header")
    stop = data.index(b"\n", end) + 1
    lines = data[:stop].decode("ascii").splitlines()
    assert lines[0].strip() == "ply", "not a PLY file"
    fmt = None
    elements: list[dict] = []
    for line in lines[1:]:
        words = line.split()
        if not words:
            continue
        if words[0] == "format":
            fmt = words[1]
        elif words[0] == "element":
            elements.append({"name": words[1], "count": int(words[2]), "properties": []})
        elif words[0] == "property":
            if words[1] == "list":
                elements[-1]["properties"].append((words[4], ("list", words[2], words[3])))
            else:
                elements[-1]["properties"].append((words[2], words[1]))
    return fmt, elements, stop


def read_elements(data: bytes) -> dict[str, list[dict]]:
    """Every element's rows as {property: value (or list)}."""
    fmt, elements, pos = parse_header(data)
    out: dict[str, list[dict]] = {}
    if fmt == "ascii":
        tokens = data[pos:].decode("ascii").split()
        t = 0
        for el in elements:
            rows = []
            for _ in range(el["count"]):
                row = {}
                for name, typ in el["properties"]:
                    if isinstance(typ, tuple):
                        m = int(tokens[t])
                        t += 1
                        conv = float if _TYPES[typ[2]] in "fd" else int
                        row[name] = [conv(tokens[t + i]) for i in range(m)]
                        t += m
                    else:
                        conv = float if _TYPES[typ] in "fd" else int
                        value = conv(tokens[t])
                        if _TYPES[typ] == "f":  # the value a float32 property holds
                            value = struct.unpack("<f", struct.pack("<f", value))[0]
                        row[name] = value
                        t += 1
                rows.append(row)
            out[el["name"]] = rows
        return out
    order = "<" if fmt == "binary_little_endian" else ">"
    for el in elements:
        rows = []
        for _ in range(el["count"]):
            row = {}
            for name, typ in el["properties"]:
                if isinstance(typ, tuple):
                    code = _TYPES[typ[1]]
                    (m,) = struct.unpack_from(order + code, data, pos)
                    pos += struct.calcsize(code)
                    item = _TYPES[typ[2]]
                    row[name] = list(struct.unpack_from(order + item * m, data, pos))
                    pos += struct.calcsize(item) * m
                else:
                    code = _TYPES[typ]
                    (row[name],) = struct.unpack_from(order + code, data, pos)
                    pos += struct.calcsize(code)
            rows.append(row)
        out[el["name"]] = rows
    return out


def load_ply_values(data: bytes) -> dict[str, list]:
    """load_ply's dictionary (ply.py:55-89) as nested lists of Python floats:
    mean, normals (zeros when nx/ny/nz are absent), rotation, scale,
    opacity [N][1], color [N][K][3] with K - 1 = (number of f_rest) / 3."""
    rows = read_elements(data)["vertex"]
    _, elements, _ = parse_header(data)
    vertex = next(e for e in elements if e["name"] == "vertex")
    names = {p for p, _ in vertex["properties"]}
    d = sum(1 for p in names if p.startswith("f_rest_"))
    assert d % 3 == 0, "f_rest count must be a multiple of 3"
    has_normals = all(p in names for p in ("nx", "ny", "nz"))
    out = {k: [] for k in ("mean", "normals", "rotation", "scale", "opacity", "color")}
    for r in rows:
        out["mean"].append([r["x"], r["y"], r["z"]])
        out["normals"].append([r["nx"], r["ny"], r["nz"]] if has_normals else [0.0, 0.0, 0.0])
        out["rotation"].append([r[f"rot_{i}"] for i in range(4)])
        out["scale"].append([r[f"scale_{i}"] for i in range(3)])
        out["opacity"].append([r["opacity"]])
        color = [[r[f"f_dc_{c}"] for c in range(3)]]
        for kk in range(1, d // 3 + 1):
            color.append([r[f"f_rest_{c * (d // 3) + kk - 1}"] for c in range(3)])
        out["color"].append(color)
    return out


def float32(value: float) -> float:
    """The float32 nearest ``value`` (what a float property stores)."""
    if math.isnan(value):
        return value
    return struct.unpack("<f", struct.pack("<f", value))[0]
