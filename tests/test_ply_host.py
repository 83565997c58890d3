"""Scene files on the CPU: the oracle pinned by a hand-assembled file, the
product's load_ply / save_ply (ply.py:12-89 semantics) against the oracle on
files of many layouts, the reference's error behaviour and the conversion
commands.  No GPU."""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from gaussian_splats_hip.splats import GaussianSplat
from gaussian_splats_hip.splats.ply import load_ply, save_ply
from oracle import ply as oply
from tests import plyfiles

KNOWN_HEADER = """ply
format binary_little_endian 1.0
element vertex 2
property float x
property float y
property float z
property float nx
property float ny
property float nz
property float f_dc_0
property float f_dc_1
property float f_dc_2
property float f_rest_0
property float f_rest_1
property float f_rest_2
property float f_rest_3
property float f_rest_4
property float f_rest_5
property float f_rest_6
property float f_rest_7
property float f_rest_8
property float opacity
property float scale_0
property float scale_1
property float scale_2
property float rot_0
property float rot_1
property float rot_2
property float rot_3
end_header
"""

# Record of Gaussian n of the known-answer state below, in file order: the
# higher SH bands are channel-major (f_rest_{c*3 + k-1} = color[k][c]).
KNOWN_RECORDS = [
    [0.5, 0.25, 0.125, 1, 2, 3, 0, 1, 2, 10, 20, 30, 11, 21, 31, 12, 22, 32,
     -0.5, -1, -2, -3, 0.75, 1.5, 2.5, 3.5],
    [1.5, 1.25, 1.125, 2, 3, 4, 1000, 1001, 1002, 1010, 1020, 1030, 1011, 1021, 1031, 1012,
     1022, 1032, 0.5, 0, -1, -2, 1.75, 2.5, 3.5, 4.5],
]


def known_state():
    n, k = 2, 4
    return {
        "mean": [[g + 0.5, g + 0.25, g + 0.125] for g in range(n)],
        "normals": [[g + 1.0, g + 2.0, g + 3.0] for g in range(n)],
        "color": [[[g * 1000 + kk * 10 + c for c in range(3)] for kk in range(k)] for g in range(n)],
        "opacity": [[g - 0.5] for g in range(n)],
        "scale": [[g - 1.0, g - 2.0, g - 3.0] for g in range(n)],
        "rotation": [[g + 0.75, g + 1.5, g + 2.5, g + 3.5] for g in range(n)],
    }


def known_bytes() -> bytes:
    body = b"".join(struct.pack("<26f", *r) for r in KNOWN_RECORDS)
    return KNOWN_HEADER.encode("ascii") + body


def as_tensors(state):
    return {k: torch.tensor(np.asarray(v, dtype=np.float32)) for k, v in state.items()}


def test_oracle_writes_the_known_file():
    assert oply.save_ply_bytes(known_state()) == known_bytes()


def test_oracle_reads_the_known_file():
    values = oply.load_ply_values(known_bytes())
    expected = known_state()
    for key in expected:
        assert values[key] == expected[key], key


def test_oracle_transposition_is_pinned():
    """A writer that keeps the coefficient-major order (the plausible
    mistake) produces other bytes."""
    state = known_state()
    wrong = dict(state)
    wrong["color"] = [[[c[kk][ch] for ch in range(3)] for kk in (0, 2, 1, 3)] for c in state["color"]]
    assert oply.save_ply_bytes(wrong) != known_bytes()


def test_save_ply_writes_the_known_file(tmp_path):
    path = tmp_path / "known.ply"
    save_ply(as_tensors(known_state()), path)
    assert path.read_bytes() == known_bytes()


def test_load_ply_reads_the_known_file(tmp_path):
    path = tmp_path / "known.ply"
    path.write_bytes(known_bytes())
    out = load_ply(path)
    for key, value in as_tensors(known_state()).items():
        assert out[key].dtype == torch.float32
        assert torch.equal(out[key], value), key


@pytest.mark.parametrize("n,k", [(0, 1), (1, 1), (37, 4), (20, 9), (50, 16)])
def test_save_ply_matches_oracle(tmp_path, n, k):
    state = plyfiles.random_state(n, k, seed=n + k)
    path = tmp_path / "s.ply"
    save_ply({key: torch.from_numpy(v) for key, v in state.items()}, path)
    assert path.read_bytes() == oply.save_ply_bytes(state)


def test_save_ply_without_normals_writes_zeros(tmp_path):
    state = plyfiles.random_state(5, 4, normals=False)
    path = tmp_path / "s.ply"
    save_ply({key: torch.from_numpy(v) for key, v in state.items()}, path)
    assert path.read_bytes() == oply.save_ply_bytes(state)
    assert torch.equal(load_ply(path)["normals"], torch.zeros(5, 3))


def test_save_ply_rounds_float64_to_float32(tmp_path):
    state = plyfiles.random_state(7, 4)
    wide = {key: torch.from_numpy(v.astype(np.float64) * (1 + 1e-9)) for key, v in state.items()}
    path = tmp_path / "s.ply"
    save_ply(wide, path)
    rounded = {key: v.numpy().astype(np.float32) for key, v in wide.items()}
    assert path.read_bytes() == oply.save_ply_bytes(rounded)


def _layouts(state):
    """(name, elements, format, newline) of files holding ``state``."""
    n = len(state["mean"])
    cols = plyfiles.vertex_columns(state)
    names = list(cols)
    rng = np.random.default_rng(1)
    shuffled = [names[i] for i in rng.permutation(len(names))]
    extras = [("red", "uchar", np.arange(n) % 256), ("confidence", "double", np.linspace(0, 1, n))]
    odd = ["red"] + shuffled[:5] + ["confidence"] + shuffled[5:]
    doubles = {name: "double" for name in names[::2]}
    face = ("face", [("vertex_indices", ("list", "uchar", "int"))], [([0, 1, 2],), ([2, 1],)])
    camera = ("camera", [("id", "int"), ("f", "float")], [(1, 2.5), (2, 3.5)])
    return [
        ("reference", [plyfiles.vertex_element(state)], "binary_little_endian", "\n"),
        ("shuffled", [plyfiles.vertex_element(state, order=shuffled)], "binary_little_endian", "\n"),
        ("odd_record", [plyfiles.vertex_element(state, order=odd, extras=extras)],
         "binary_little_endian", "\n"),
        ("big_endian", [plyfiles.vertex_element(state, order=shuffled)], "binary_big_endian", "\n"),
        ("big_endian_odd", [plyfiles.vertex_element(state, order=odd, extras=extras)],
         "binary_big_endian", "\n"),
        ("doubles", [plyfiles.vertex_element(state, types=doubles)], "binary_little_endian", "\n"),
        ("ascii", [plyfiles.vertex_element(state, order=shuffled)], "ascii", "\n"),
        ("crlf", [plyfiles.vertex_element(state)], "binary_little_endian", "\r\n"),
        ("no_normals", [plyfiles.vertex_element(state, normals=False)], "binary_little_endian", "\n"),
        ("other_elements", [camera, plyfiles.vertex_element(state), face], "binary_little_endian",
         "\n"),
        ("ascii_other_elements", [camera, plyfiles.vertex_element(state), face], "ascii", "\n"),
    ]


LAYOUTS = [name for name, *_ in _layouts(plyfiles.random_state(1, 1))]


def write_layout(tmp_path, name, n=29, k=9):
    state = plyfiles.random_state(n, k, seed=3)
    elements, fmt, newline = next((e, f, nl) for nm, e, f, nl in _layouts(state) if nm == name)
    path = tmp_path / f"{name}.ply"
    plyfiles.write(path, elements, fmt, newline)
    return path, state


@pytest.mark.parametrize("layout", LAYOUTS)
def test_load_ply_matches_oracle(tmp_path, layout):
    path, _ = write_layout(tmp_path, layout)
    out = load_ply(path)
    expected = oply.load_ply_values(path.read_bytes())
    for key, value in expected.items():
        got = out[key].double().numpy()
        want = np.asarray(value, dtype=np.float64).reshape(got.shape)
        assert np.array_equal(got, want), (layout, key)


def test_load_ply_keeps_the_property_dtype(tmp_path):
    """As np.stack in the reference: float64 properties give float64 tensors."""
    path, _ = write_layout(tmp_path, "doubles")
    out = load_ply(path)
    assert out["mean"].dtype == torch.float64  # x and z are double, y float
    path, _ = write_layout(tmp_path, "reference")
    assert all(v.dtype == torch.float32 for v in load_ply(path).values())


def test_load_ply_empty(tmp_path):
    path = tmp_path / "empty.ply"
    save_ply({key: torch.from_numpy(v) for key, v in plyfiles.random_state(0, 16).items()}, path)
    out = load_ply(path)
    assert out["mean"].shape == (0, 3) and out["color"].shape == (0, 16, 3)


def test_load_ply_errors(tmp_path):
    with pytest.raises(AssertionError, match="Only .ply files"):
        load_ply(tmp_path / "scene.pt")
    path = tmp_path / "bad.ply"
    path.write_bytes(b"not a ply\n")
    with pytest.raises(ValueError):
        load_ply(path)
    state = plyfiles.random_state(3, 4)
    cols = [c for c in plyfiles.vertex_columns(state) if c != "rot_2"]
    plyfiles.write(path, [plyfiles.vertex_element(state, order=cols)])
    with pytest.raises(ValueError, match="rot_2"):
        load_ply(path)
    cols = [c for c in plyfiles.vertex_columns(state) if c != "f_rest_8"]
    plyfiles.write(path, [plyfiles.vertex_element(state, order=cols)])
    with pytest.raises(ValueError, match="multiple of 3"):
        load_ply(path)
    face = ("face", [("vertex_indices", ("list", "uchar", "int"))], [([0, 1, 2],)])
    plyfiles.write(path, [face, plyfiles.vertex_element(state)])
    with pytest.raises(ValueError, match="list properties"):
        load_ply(path)
    data = plyfiles.vertex_element(state)
    plyfiles.write(path, [data])
    path.write_bytes(path.read_bytes()[:-5])
    with pytest.raises(ValueError, match="ends"):
        load_ply(path)


def test_save_ply_rejects_bad_color_shape(tmp_path):
    state = {key: torch.from_numpy(v) for key, v in plyfiles.random_state(3, 4).items()}
    state["color"] = torch.zeros(3, 5, 3)
    with pytest.raises(ValueError, match="Invalid color shape"):
        save_ply(state, tmp_path / "x.ply")
    state["color"] = torch.zeros(3, 4, 4)
    with pytest.raises(ValueError, match="Invalid color shape"):
        save_ply(state, tmp_path / "x.ply")


def test_splat_round_trip_and_convert_commands(tmp_path):
    from typer.testing import CliRunner

    from gaussian_splats_hip.splats.convert import app

    torch.manual_seed(0)
    splats = GaussianSplat(41, sh_degree=2)
    with torch.no_grad():
        splats.normals.normal_()
    ckpt = tmp_path / "scene.pt"
    splats.save_checkpoint(ckpt)
    runner = CliRunner()
    result = runner.invoke(app, ["pt-to-ply", str(ckpt)])
    assert result.exit_code == 0, result.output
    assert (tmp_path / "scene.ply").exists()
    result = runner.invoke(app, ["ply-to-pt", str(tmp_path / "scene.ply"), "-o", str(tmp_path / "back.pt")])
    assert result.exit_code == 0, result.output
    back = GaussianSplat.from_checkpoint(tmp_path / "back.pt")
    assert back.sh_degree == 2
    for key, value in splats.state_dict().items():
        assert torch.equal(back.state_dict()[key], value), key


def test_ply_kernels_host_checks():
    """The C ABI validates sizes, offsets and alignment before any launch."""
    import ctypes

    from gaussian_splats_hip.kernels.rasterize import _native as nat

    lib = nat.library()
    fake = ctypes.c_void_p(256)
    outs = [fake] * 6
    null = ctypes.c_void_p(0)
    good = (ctypes.c_int32 * 62)(*[4 * j for j in range(62)])
    bad = (ctypes.c_int32 * 62)(*([4 * j for j in range(61)] + [248]))
    table = ctypes.cast(good, ctypes.c_void_p)
    assert lib.gs_ply_unpack(fake, 10, 248, table, 0, 26, *outs, null) == nat.GS_ERR_UNSUPPORTED
    assert lib.gs_ply_unpack(fake, 10, 2, table, 0, 16, *outs, null) == nat.GS_ERR_UNSUPPORTED
    assert lib.gs_ply_unpack(fake, 10, 248, null, 0, 16, *outs, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ply_unpack(fake, 10, 248, ctypes.cast(bad, ctypes.c_void_p), 0, 16, *outs,
                             null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ply_unpack(ctypes.c_void_p(260), 10, 248, table, 0, 16, *outs,
                             null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ply_unpack(fake, 10, 248, table, 0, 16, fake, null, fake, fake, fake, fake,
                             null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ply_unpack(null, 0, 248, table, 0, 16, *([null] * 6), null) == nat.GS_OK
    assert lib.gs_ply_pack(*([fake] * 6), 10, 0, fake, null) == nat.GS_ERR_UNSUPPORTED
    assert lib.gs_ply_pack(fake, null, fake, fake, fake, fake, 10, 16, null,
                           null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ply_pack(*([null] * 6), 0, 16, null, null) == nat.GS_OK
