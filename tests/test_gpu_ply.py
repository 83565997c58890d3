"""Scene files on the GPU: ``load_ply(path, device=cuda)`` (records split by
gs_ply_unpack) and ``save_ply`` of GPU tensors (records assembled by
gs_ply_pack) against the host path, itself pinned to the oracle
(tests/test_ply_host.py).  Bit-exact: the kernels only move bytes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splats_hip.splats.ply import load_ply, save_ply
from oracle import ply as oply
from tests import plyfiles
from tests.test_ply_host import LAYOUTS, write_layout

pytestmark = pytest.mark.gpu


def _equal(gpu: dict, cpu: dict):
    for key, value in cpu.items():
        got = gpu[key]
        assert got.is_cuda and got.dtype == torch.float32, key
        assert torch.equal(got.cpu(), value.float()), key


@pytest.mark.parametrize("layout", LAYOUTS)
def test_load_ply_device_equals_host(tmp_path, device, layout):
    path, _ = write_layout(tmp_path, layout, n=301, k=16)
    print(f"load_ply device layout={layout}", flush=True)
    _equal(load_ply(path, device=device), load_ply(path))


@pytest.mark.parametrize("n", [1, 131, 132, 133, 1000])
@pytest.mark.parametrize("k", [1, 4, 16, 25])
def test_group_boundaries(tmp_path, device, n, k):
    """Record counts around one workgroup's group (32736 // record bytes)."""
    state = plyfiles.random_state(n, k, seed=n * 31 + k)
    path = tmp_path / "s.ply"
    print(f"ply round trip n={n} k={k}", flush=True)
    save_ply({key: torch.from_numpy(v).to(device) for key, v in state.items()}, path)
    assert path.read_bytes() == oply.save_ply_bytes(state)
    _equal(load_ply(path, device=device), load_ply(path))


def test_save_ply_device_equals_host_large(tmp_path, device):
    """200k SH3 Gaussians (50 MB): GPU pack equals the host writer byte for
    byte and the GPU load returns the tensors that were saved."""
    n, k = 200_000, 16
    g = torch.Generator().manual_seed(0)
    state = {
        "mean": torch.randn(n, 3, generator=g), "rotation": torch.randn(n, 4, generator=g),
        "scale": torch.randn(n, 3, generator=g), "opacity": torch.randn(n, 1, generator=g),
        "color": torch.randn(n, k, 3, generator=g), "normals": torch.randn(n, 3, generator=g),
    }
    host_path, dev_path = tmp_path / "host.ply", tmp_path / "dev.ply"
    print("ply 200k save/load", flush=True)
    save_ply(state, host_path)
    save_ply({key: v.to(device) for key, v in state.items()}, dev_path)
    assert host_path.read_bytes() == dev_path.read_bytes()
    loaded = load_ply(dev_path, device=device)
    for key, value in state.items():
        assert torch.equal(loaded[key].cpu(), value), key


def test_save_ply_device_without_normals_and_float64(tmp_path, device):
    state = plyfiles.random_state(77, 9, normals=False)
    wide = {key: torch.from_numpy(v.astype(np.float64) * (1 + 1e-9)).to(device)
            for key, v in state.items()}
    path = tmp_path / "s.ply"
    save_ply(wide, path)
    rounded = {key: v.cpu().numpy().astype(np.float32) for key, v in wide.items()}
    assert path.read_bytes() == oply.save_ply_bytes(rounded)


def test_load_ply_device_empty(tmp_path, device):
    path = tmp_path / "empty.ply"
    save_ply({key: torch.from_numpy(v) for key, v in plyfiles.random_state(0, 16).items()}, path)
    out = load_ply(path, device=device)
    assert out["mean"].shape == (0, 3) and out["color"].shape == (0, 16, 3)
    assert out["mean"].is_cuda
