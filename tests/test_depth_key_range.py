"""The depth sort's key remap (gs_bin_tiles_plan's key_base, key_bits) on the
CPU: the remapped keys of the projection's depth keys sort exactly as the
keys themselves (a stable sort of float bits, intersections.py:82's order)."""

from __future__ import annotations

import numpy as np
import pytest

from gaussian_splats_hip.kernels.rasterize.intersections import depth_key_range


def _bits(x):
    return int(np.float32(x).view(np.uint32))


def test_range_of_the_benchmark_planes():
    base, bits = depth_key_range(0.2, 100.0)
    assert base == _bits(0.2)
    span = _bits(100.0) - _bits(0.2)
    assert span == 0x047B3333  # 75182899
    assert bits == 27 and (1 << 26) <= span < (1 << 27)


@pytest.mark.parametrize("near, far", ((0.0, 100.0), (-1.0, 10.0), (5.0, 5.0), (2.0, 1.0),
                                       (0.2, float("inf"))))
def test_planes_without_a_remap(near, far):
    """Non-positive near planes, empty or inverted ranges and infinite far
    planes keep the keys' own 32 bits."""
    assert depth_key_range(near, far) == (0, 32)


@pytest.mark.parametrize("near, far", ((0.2, 100.0), (0.01, 10.0), (1.0, 1.5), (3.0, 3.0001),
                                       (1e-30, 1e30)))
def test_remapped_keys_sort_as_the_keys(near, far):
    """Depths strictly between the planes (the projection's culling) and ~0
    for culled Gaussians: the stable order of min(key - base, 2^bits - 1)
    equals that of the keys, and every visible key maps below the culled
    value."""
    base, bits = depth_key_range(near, far)
    rng = np.random.default_rng(7)
    lo, hi = np.float32(near), np.float32(far)
    n = 20000
    d = np.exp(rng.uniform(np.log(lo), np.log(hi), n)).astype(np.float32)
    d = np.clip(d, np.nextafter(lo, hi), np.nextafter(hi, lo))
    d[:1000] = d[1000:2000]  # ties
    d[2000], d[2001] = np.nextafter(lo, hi), np.nextafter(hi, lo)
    keys = d.view(np.uint32).astype(np.uint64)
    keys[rng.random(n) < 0.1] = 0xFFFFFFFF  # culled
    cap = (1 << bits) - 1
    remapped = np.minimum((keys - base) % (1 << 32), cap)
    visible = keys != 0xFFFFFFFF
    assert remapped[visible].max() < cap
    assert np.array_equal(np.argsort(keys, kind="stable"), np.argsort(remapped, kind="stable"))
