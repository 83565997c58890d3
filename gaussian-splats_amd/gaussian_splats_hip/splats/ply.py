"""Scene files: Gaussian-splat PLY load and save (reference:
src/gaussian_splats/splats/ply.py:12-89).

``save_ply(state, path)`` writes one binary little-endian ``vertex`` element
of float32 properties ``x y z nx ny nz f_dc_0..2 f_rest_0.. opacity
scale_0..2 rot_0..3`` (``f_rest_{c (K-1) + k - 1} = color[k][c]``);
``load_ply(path)`` reads those properties by name from any PLY file (any
property order, extra properties and elements, either binary byte order or
ascii, missing normals read as zeros) and returns the reference's dictionary
of CPU tensors.

The reference parses with plyfile; here the header is parsed directly and
the vertex block is read with numpy.  With ``device`` set to a ROCm GPU
(``load_ply(path, device="cuda")``), or for state tensors that live on one
(``save_ply``), the records are split or assembled on the GPU by the
library's ``gs_ply_unpack`` / ``gs_ply_pack`` kernels: the file's vertex
block is uploaded unchanged through pinned staging buffers, chunk by chunk,
and one kernel writes the six parameter tensors (and the reverse for a save),
so a scene reaches HBM without per-property host passes.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

_NUMPY_TYPES = {
    "char": "i1", "int8": "i1", "uchar": "u1", "uint8": "u1",
    "short": "i2", "int16": "i2", "ushort": "u2", "uint16": "u2",
    "int": "i4", "int32": "i4", "uint": "u4", "uint32": "u4",
    "float": "f4", "float32": "f4", "double": "f8", "float64": "f8",
}
_FORMATS = {"ascii": None, "binary_little_endian": "<", "binary_big_endian": ">"}
_MAX_HEADER = 1 << 20
_CHUNK = 32 << 20  # bytes per pinned staging buffer


@dataclass
class _Element:
    name: str
    count: int
    properties: list[tuple[str, str | tuple[str, str]]] = field(default_factory=list)

    def has_lists(self) -> bool:
        return any(isinstance(t, tuple) for _, t in self.properties)


def _parse_header(f) -> tuple[str, list[_Element], int]:
    """(format, elements, byte offset of the body)."""
    if f.readline().strip() != b"ply":
        raise ValueError("not a PLY file (missing 'ply' magic)")
    fmt = None
    elements: list[_Element] = []
    read = 0
    while True:
        line = f.readline()
        read += len(line)
        if not line or read > _MAX_HEADER:
            raise ValueError("PLY header has no end_header line")
        words = line.decode("ascii", errors="replace").split()
        if not words:
            continue
        key = words[0]
        if key == "end_header":
            break
        if key == "format":
            if words[1] not in _FORMATS:
                raise ValueError(f"unsupported PLY format {words[1]!r}")
            fmt = words[1]
        elif key == "element":
            elements.append(_Element(words[1], int(words[2])))
        elif key == "property":
            if not elements:
                raise ValueError("PLY property before any element")
            if words[1] == "list":
                elements[-1].properties.append((words[4], (words[2], words[3])))
            else:
                if words[1] not in _NUMPY_TYPES:
                    raise ValueError(f"unknown PLY property type {words[1]!r}")
                elements[-1].properties.append((words[2], words[1]))
    if fmt is None:
        raise ValueError("PLY header has no format line")
    return fmt, elements, f.tell()


def _vertex_dtype(vertex: _Element, order: str) -> np.dtype:
    if vertex.has_lists():
        raise ValueError("list properties in the vertex element are not supported")
    return np.dtype([(name, order + _NUMPY_TYPES[t]) for name, t in vertex.properties])


def _fields(names: list[str]) -> tuple[int, list[str]]:
    """(K, the property of each canonical output float): mean 3, normals 3
    (None when absent), rotation 4, scale 3, opacity 1, color 3K
    coefficient-major (ply.py:62-80)."""
    d = sum(1 for name in names if name.startswith("f_rest_"))
    if d % 3:
        raise ValueError(f"the number of f_rest properties ({d}) is not a multiple of 3")
    k = d // 3 + 1
    normals = ["nx", "ny", "nz"] if all(n in names for n in ("nx", "ny", "nz")) else [None] * 3
    color = []
    for kk in range(k):
        for c in range(3):
            color.append(f"f_dc_{c}" if kk == 0 else f"f_rest_{c * (k - 1) + kk - 1}")
    fields = (
        ["x", "y", "z"] + normals + [f"rot_{i}" for i in range(4)]
        + [f"scale_{i}" for i in range(3)] + ["opacity"] + color
    )
    present = set(names)
    for name in fields:
        if name is not None and name not in present:
            raise ValueError(f"no field of name {name}")
    return k, fields


_WIDTHS = (("mean", 3), ("normals", 3), ("rotation", 4), ("scale", 3), ("opacity", 1))


def _read_vertex(path: Path) -> tuple[str, _Element, int, int]:
    """(format, vertex element, byte offset of its block (binary) or line
    index of its first row (ascii), header size)."""
    with open(path, "rb") as f:
        fmt, elements, body = _parse_header(f)
        order = _FORMATS[fmt]
        skip = 0
        for el in elements:
            if el.name == "vertex":
                return fmt, el, (body + skip) if order else skip, body
            if order is None:
                skip += el.count
            elif el.has_lists():
                raise ValueError(
                    f"element {el.name!r} with list properties precedes the vertex element")
            else:
                skip += el.count * _vertex_dtype(el, order).itemsize
    raise ValueError("PLY file has no vertex element")


def _host_records(path: Path, fmt: str, vertex: _Element, where: int, body: int) -> np.ndarray:
    """The vertex rows as a structured array of native byte order."""
    order = _FORMATS[fmt]
    if order is not None:
        dtype = _vertex_dtype(vertex, order)
        rows = np.fromfile(path, dtype=dtype, count=vertex.count, offset=where)
        if len(rows) != vertex.count:
            raise ValueError(f"PLY file ends after {len(rows)} of {vertex.count} vertices")
        return rows.astype(dtype.newbyteorder("="))
    dtype = _vertex_dtype(vertex, "=")
    with open(path, "rb") as f:
        f.seek(body)
        for _ in range(where):
            f.readline()
        lines = [f.readline() for _ in range(vertex.count)]
    if vertex.count and not lines[-1].strip():
        raise ValueError("PLY file ends before the last vertex")
    values = np.array(b" ".join(lines).split(), dtype=np.float64)
    if values.size != vertex.count * len(vertex.properties):
        raise ValueError("ascii vertex rows do not match the declared properties")
    values = values.reshape(vertex.count, len(vertex.properties))
    rows = np.empty(vertex.count, dtype=dtype)
    for i, (name, _) in enumerate(vertex.properties):
        rows[name] = values[:, i]
    return rows


def _stack(rows: np.ndarray, names: list[str]) -> np.ndarray:
    return np.stack([rows[name] for name in names], axis=1)  # ply.py:8-9


def load_ply(path: str | Path, device: torch.device | str | None = None) -> dict[str, torch.Tensor]:
    """The parameters stored in a PLY file (ply.py:55-89): ``mean``,
    ``normals`` (zeros when absent), ``rotation``, ``scale``, ``opacity``
    [N, 1] and ``color`` [N, K, 3].  Without ``device`` the tensors are on
    the CPU with the properties' numpy dtype, as the reference returns them;
    with a ROCm ``device`` they are float32 tensors there, split on the GPU."""
    assert Path(path).suffix.lower() == ".ply", f"Only .ply files are supported. Got {Path(path)}"
    path = Path(path)
    fmt, vertex, where, body = _read_vertex(path)
    names = [name for name, _ in vertex.properties]
    k, fields = _fields(names)
    if device is not None and torch.device(device).type == "cuda":
        return _load_device(path, fmt, vertex, where, body, k, fields, torch.device(device))
    rows = _host_records(path, fmt, vertex, where, body)
    mean = _stack(rows, ["x", "y", "z"])
    normals = _stack(rows, ["nx", "ny", "nz"]) if fields[3] is not None else np.zeros_like(mean)
    d = 3 * (k - 1)
    dc = _stack(rows, [f"f_dc_{i}" for i in range(3)])
    if d:
        rest = _stack(rows, [f"f_rest_{i}" for i in range(d)]).reshape(len(rows), 3, k - 1)
        rest = rest.transpose(0, 2, 1)
    else:
        rest = np.empty((len(rows), 0, 3), dtype=dc.dtype)
    out = {
        "mean": mean,
        "normals": normals,
        "rotation": _stack(rows, [f"rot_{i}" for i in range(4)]),
        "scale": _stack(rows, [f"scale_{i}" for i in range(3)]),
        "opacity": rows["opacity"][:, None],
        "color": np.concatenate((dc[:, None], rest), axis=1),
    }
    out = {key: torch.as_tensor(np.ascontiguousarray(v)) for key, v in out.items()}
    if device is not None:
        out = {key: v.to(device) for key, v in out.items()}
    return out


def _upload(path: Path, offset: int, nbytes: int, device: torch.device) -> torch.Tensor:
    """The file's bytes [offset, offset + nbytes) in device memory (16-byte
    aligned), read through two pinned staging buffers so that the disk read
    of one chunk overlaps the upload of the previous one."""
    dst = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
    chunk = min(_CHUNK, max(nbytes, 1))
    staging = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    done = [None, None]
    stream = torch.cuda.current_stream(device)
    with open(path, "rb") as f:
        f.seek(offset)
        pos = 0
        i = 0
        while pos < nbytes:
            size = min(chunk, nbytes - pos)
            if done[i] is not None:
                done[i].synchronize()
            view = memoryview(staging[i].numpy())[:size]
            got = 0
            while got < size:
                r = f.readinto(view[got:])
                if not r:
                    raise ValueError(f"PLY file ends {nbytes - pos - got} bytes early")
                got += r
            dst[pos:pos + size].copy_(staging[i][:size], non_blocking=True)
            done[i] = torch.cuda.Event()
            done[i].record(stream)
            pos += size
            i ^= 1
    for ev in done:
        if ev is not None:
            ev.synchronize()
    return dst


def _load_device(path, fmt, vertex, where, body, k, fields, device) -> dict[str, torch.Tensor]:
    from ..kernels.rasterize import _native as nat

    if 14 + 3 * k > nat.PLY_MAX_FIELDS:
        raise NotImplementedError(f"{k} SH coefficients exceed the GPU loader's limit")
    n = vertex.count
    order = _FORMATS[fmt]
    types = dict(vertex.properties)
    raw = order is not None and all(f is None or types[f] in ("float", "float32") for f in fields)
    if raw:
        # The records as stored: each output float's byte offset in a row.
        offsets, pos = {}, 0
        for name, t in vertex.properties:
            offsets[name] = pos
            pos += np.dtype(_NUMPY_TYPES[t]).itemsize
        record_bytes = pos
        table = [-1 if f is None else offsets[f] for f in fields]
        records = _upload(path, where, n * record_bytes, device)
        big = order == ">"
    else:
        # Other property types or ascii: the host converts the needed
        # properties to a float32 matrix in canonical order.
        rows = _host_records(path, fmt, vertex, where, body)
        matrix = np.zeros((n, len(fields)), dtype=np.float32)
        for j, f in enumerate(fields):
            if f is not None:
                matrix[:, j] = rows[f]
        record_bytes = 4 * len(fields)
        table = [4 * j for j in range(len(fields))]
        records = torch.empty(max(n * record_bytes, 16), dtype=torch.uint8, device=device)
        records[: n * record_bytes].copy_(torch.from_numpy(matrix.reshape(-1).view(np.uint8)))
        big = False
    parts = [torch.empty((n, w), dtype=torch.float32, device=device) for _, w in _WIDTHS]
    color = torch.empty((n, k, 3), dtype=torch.float32, device=device)
    lib = nat.library()
    offsets_arr = (ctypes.c_int32 * len(table))(*table)
    nat.check(
        nat.launch("ply_unpack", lambda: lib.gs_ply_unpack(
            nat.ptr(records), n, record_bytes, ctypes.cast(offsets_arr, ctypes.c_void_p), int(big),
            k, *(nat.ptr(p) for p in parts), nat.ptr(color), nat.stream(device))),
        "ply_unpack",
    )
    torch.cuda.current_stream(device).synchronize()  # the records buffer is freed on return
    result = {key: p for (key, _), p in zip(_WIDTHS, parts)}
    result["color"] = color
    return result


def _header(n: int, k: int) -> bytes:
    fields = (
        ["x", "y", "z", "nx", "ny", "nz"]
        + [f"f_dc_{i}" for i in range(3)]
        + [f"f_rest_{i}" for i in range((k - 1) * 3)]
        + ["opacity"]
        + [f"scale_{i}" for i in range(3)]
        + [f"rot_{i}" for i in range(4)]
    )
    lines = ["ply", "format binary_little_endian 1.0", f"element vertex {n}"]
    lines += [f"property float {name}" for name in fields] + ["end_header"]
    return ("\n".join(lines) + "\n").encode("ascii")


def save_ply(state: dict[str, torch.Tensor], path: str | Path) -> None:
    """Writes ``state`` (a GaussianSplat state dict, or any mapping with
    mean, rotation, scale, opacity, color and optionally normals) as a
    binary PLY file (ply.py:12-52).  Tensors on a ROCm GPU are packed into
    records there and downloaded in chunks that overlap the file writes."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    tensors = [state[key].detach() for key in ("mean", "rotation", "scale", "opacity", "color")]
    mean, rotation, scale, opacity, color = tensors
    normals = state.get("normals")
    normals = torch.zeros_like(mean) if normals is None else normals.detach()
    n, d, c = color.shape
    if c != 3 or int(d**0.5) ** 2 != d:
        raise ValueError(f"Invalid color shape {color.shape}. Expected [N, (degree + 1) ** 2, 3]")
    if mean.is_cuda:
        records = _pack_device(mean, normals, rotation, scale, opacity, color)
        with open(path, "wb") as f:
            f.write(_header(n, d))
            _download(records.view(torch.uint8).reshape(-1), f)
        return
    values = np.concatenate(
        (
            mean.cpu().numpy(),
            normals.cpu().numpy(),
            color[:, 0].cpu().numpy(),
            color[:, 1:].cpu().numpy().transpose(0, 2, 1).reshape(n, (d - 1) * 3),
            opacity.cpu().numpy().reshape(n, 1),
            scale.cpu().numpy(),
            rotation.cpu().numpy(),
        ),
        axis=1,
    )
    with open(path, "wb") as f:
        f.write(_header(n, d))
        f.write(memoryview(np.ascontiguousarray(values.astype("<f4")).reshape(-1).view(np.uint8)))


def _download(src: torch.Tensor, f) -> None:
    """Writes the device bytes ``src`` to ``f`` through two pinned staging
    buffers: the download of one chunk overlaps the file write of the
    previous one."""
    nbytes = src.numel()
    if nbytes == 0:
        return
    chunk = min(_CHUNK, nbytes)
    staging = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    stream = torch.cuda.current_stream(src.device)
    pending = None  # (event, buffer index, size) of the chunk in flight
    i = 0
    for pos in range(0, nbytes, chunk):
        size = min(chunk, nbytes - pos)
        staging[i][:size].copy_(src[pos:pos + size], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        if pending is not None:
            pending[0].synchronize()
            f.write(memoryview(staging[pending[1]].numpy())[: pending[2]])
        pending = (ev, i, size)
        i ^= 1
    pending[0].synchronize()
    f.write(memoryview(staging[pending[1]].numpy())[: pending[2]])


def _pack_device(mean, normals, rotation, scale, opacity, color) -> torch.Tensor:
    from ..kernels.rasterize import _native as nat

    device = mean.device
    n, k, _ = color.shape
    if 14 + 3 * k > nat.PLY_MAX_FIELDS:
        raise NotImplementedError(f"{k} SH coefficients exceed the GPU writer's limit")
    ins = [
        nat.prepare(t.to(device=device, dtype=torch.float32))
        for t in (mean, normals, rotation, scale, opacity, color)
    ]
    records = torch.empty((n, 14 + 3 * k), dtype=torch.float32, device=device)
    nat.check(
        nat.launch("ply_pack", lambda: nat.library().gs_ply_pack(
            *(nat.ptr(t) for t in ins), n, k, nat.ptr(records), nat.stream(device))),
        "ply_pack",
    )
    return records
