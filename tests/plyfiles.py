"""PLY files of several layouts for the scene-file tests, assembled value by
value with ``struct`` from the PLY format (header lines, then each element's
rows in the declared property order and types)."""

from __future__ import annotations

import struct

import numpy as np

CODES = {"char": "b", "uchar": "B", "short": "h", "ushort": "H", "int": "i", "uint": "I",
         "float": "f", "double": "d"}


def random_state(n: int, k: int, seed: int = 0, normals: bool = True) -> dict[str, np.ndarray]:
    rng = np.random.default_rng(seed)
    state = {
        "mean": rng.normal(size=(n, 3)).astype(np.float32),
        "rotation": rng.normal(size=(n, 4)).astype(np.float32),
        "scale": rng.normal(-3, 1, size=(n, 3)).astype(np.float32),
        "opacity": rng.normal(size=(n, 1)).astype(np.float32),
        "color": rng.normal(size=(n, k, 3)).astype(np.float32),
    }
    if normals:
        state["normals"] = rng.normal(size=(n, 3)).astype(np.float32)
    return state


def vertex_columns(state: dict[str, np.ndarray], normals: bool = True) -> dict[str, np.ndarray]:
    """Property name -> column, named as the reference's files name them."""
    n, k, _ = state["color"].shape
    cols = {"x": state["mean"][:, 0], "y": state["mean"][:, 1], "z": state["mean"][:, 2]}
    if normals:
        for i, name in enumerate(("nx", "ny", "nz")):
            cols[name] = state["normals"][:, i]
    for c in range(3):
        cols[f"f_dc_{c}"] = state["color"][:, 0, c]
    for c in range(3):
        for kk in range(1, k):
            cols[f"f_rest_{c * (k - 1) + kk - 1}"] = state["color"][:, kk, c]
    cols["opacity"] = state["opacity"][:, 0]
    for i in range(3):
        cols[f"scale_{i}"] = state["scale"][:, i]
    for i in range(4):
        cols[f"rot_{i}"] = state["rotation"][:, i]
    return cols


def write(path, elements, fmt: str = "binary_little_endian", newline: str = "\n") -> None:
    """``elements``: list of (name, [(property, type)], rows) where a list
    property's type is ("list", count type, item type) and rows is a list of
    tuples of values (a list for a list property)."""
    lines = ["ply", f"format {fmt} 1.0", "comment written by the scene-file tests"]
    for name, props, rows in elements:
        lines.append(f"element {name} {len(rows)}")
        for pname, ptype in props:
            if isinstance(ptype, tuple):
                lines.append(f"property list {ptype[1]} {ptype[2]} {pname}")
            else:
                lines.append(f"property {ptype} {pname}")
    lines.append("end_header")
    out = bytearray((newline.join(lines) + newline).encode("ascii"))
    order = ">" if fmt == "binary_big_endian" else "<"
    for _, props, rows in elements:
        for row in rows:
            if fmt == "ascii":
                words = []
                for (pname, ptype), v in zip(props, row):
                    if isinstance(ptype, tuple):
                        words.append(str(len(v)))
                        words.extend(repr(float(x)) if ptype[2] in ("float", "double") else str(int(x)) for x in v)
                    elif ptype in ("float", "double"):
                        words.append(repr(float(v)))
                    else:
                        words.append(str(int(v)))
                out += (" ".join(words) + newline).encode("ascii")
                continue
            for (pname, ptype), v in zip(props, row):
                if isinstance(ptype, tuple):
                    out += struct.pack(order + CODES[ptype[1]], len(v))
                    out += struct.pack(order + CODES[ptype[2]] * len(v), *v)
                else:
                    out += struct.pack(order + CODES[ptype], v)
    with open(path, "wb") as f:
        f.write(bytes(out))


def vertex_element(state, order=None, types=None, extras=(), normals=True):
    """('vertex', props, rows) with the properties in ``order`` (default: the
    reference's, then the extras), per-property ``types`` (default float)
    and extra (name, type, column) properties, which ``order`` may place
    anywhere."""
    cols = vertex_columns(state, normals)
    types = dict(types or {})
    for name, typ, column in extras:
        cols[name] = column
        types[name] = typ
    names = list(order) if order is not None else list(cols)
    props = [(name, types.get(name, "float")) for name in names]
    columns = [cols[name] for name in names]
    n = len(state["mean"])
    rows = []
    for g in range(n):
        row = []
        for (name, typ), col in zip(props, columns):
            v = col[g]
            row.append(float(v) if typ in ("float", "double") else int(v))
        rows.append(tuple(row))
    return ("vertex", props, rows)
