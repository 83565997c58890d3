"""gs_tile_order_noalloc: the compositing dispatch plan computed in the
library's static per-GPU scratch instead of a caller workspace.

Through the C ABI: its plan equals gs_tile_order's (caller workspace) bit for
bit on consecutive calls of decreasing size -- the largest view the scratch
holds, a 1080p view by contributor counts, then a smaller view by list
lengths, so stale keys of the earlier calls remain in the scratch -- and on a
mosaic of views; the 1080p and small orders also equal the order's numpy
model.  The backward plan the op uses (ranges and contributor counts
together, lists above 8192 entries whose walks cross checkpoints) writes the
scratch's second half, the crossings, and holds segment items.  Views beyond the scratch are rejected on the host before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gaussian_splats_hip.kernels.rasterize import _native as nat

MAX_TILES = 1 << 18  # GS_TILE_ORDER_NOALLOC_MAX_TILES


def _ranges(lengths: np.ndarray) -> np.ndarray:
    r = np.zeros((lengths.size, 2), dtype=np.int64)
    r[:, 1] = np.cumsum(lengths)
    r[1:, 0] = r[:-1, 1]
    return r


def _both_orders(device, view, num_tiles, ranges=None, ncon=None):
    lib = nat.library()
    s = nat.stream(device)
    ws = nat.workspace(lib.gs_tile_order_workspace_bytes(num_tiles), device)
    count = lib.gs_tile_order_items(view, int(ncon is not None))
    expected = torch.full((count,), -7, dtype=torch.int32, device=device)
    nat.check(lib.gs_tile_order(nat.ptr(ranges), nat.ptr(ncon), view, nat.ptr(expected),
                                nat.ptr(ws), ws.numel(), 0, s), "tile_order")
    got = torch.full((count,), -7, dtype=torch.int32, device=device)
    nat.check(lib.gs_tile_order_noalloc(nat.ptr(ranges), nat.ptr(ncon), view, nat.ptr(got), s),
              "tile_order_noalloc")
    torch.cuda.synchronize(device)
    return expected.cpu().numpy(), got.cpu().numpy()


def test_noalloc_rejects_what_the_scratch_cannot_hold():
    """Host-side checks only (no GPU call is reached)."""
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    null = ctypes.c_void_p(0)
    ok = nat.make_view(100.0, 100.0, 50.0, 50.0, 100, 100, 16)
    assert lib.gs_tile_order_noalloc(null, null, ok, fake, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_tile_order_noalloc(fake, null, ok, null, null) == nat.GS_ERR_INVALID_ARGUMENT
    # 2048 x 2052 pixels in 4-pixel tiles: 512 x 513 tiles, one row beyond.
    big = nat.make_view(100.0, 100.0, 50.0, 50.0, 2048, 2052, 4)
    assert lib.gs_tile_order_noalloc(fake, null, big, fake, null) == nat.GS_ERR_WORKSPACE
    assert b"static scratch" in lib.gs_last_error()
    bad = nat.make_view(100.0, 100.0, 50.0, 50.0, 100, 100, 3)
    assert lib.gs_tile_order_noalloc(fake, null, bad, fake, null) in (
        nat.GS_ERR_INVALID_ARGUMENT, nat.GS_ERR_UNSUPPORTED)


@pytest.mark.gpu
def test_noalloc_matches_workspace_order(device):
    from parity import expected_plan, plan_tile_keys

    rng = np.random.default_rng(2024)

    # The largest view the scratch holds: 2048 x 2048 pixels, 4-pixel tiles.
    w = h = 2048
    t = (w // 4) * (h // 4)
    assert t == MAX_TILES
    lengths = rng.integers(0, 5000, size=t)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, 4)
    print(f"[noalloc] max tiles {t}", flush=True)
    expected, got = _both_orders(device, view, t, ranges=torch.as_tensor(_ranges(lengths)).to(device))
    np.testing.assert_array_equal(got, expected)
    used = got[got >= 0]
    assert got.size == expected.size and np.array_equal(np.unique(used >> 7), np.arange(t))

    # 1080p by contributor counts (the backward's estimate), partial edge tiles.
    w, h, tile = 1920, 1080, 16
    tw, th = nat.tiles(w, h, tile)
    ncon = rng.integers(0, 600, size=(h, w)).astype(np.int32)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile)
    print(f"[noalloc] 1080p contributors {tw * th} tiles", flush=True)
    expected, got = _both_orders(device, view, tw * th, ncon=torch.as_tensor(ncon).to(device))
    np.testing.assert_array_equal(got, expected)
    np.testing.assert_array_equal(
        got, expected_plan(plan_tile_keys(ncon=ncon, width=w, height=h, tile_size=tile), tile,
                           backward=True))

    # Smaller: 33 x 2 tiles by list length; the scratch still holds the keys
    # of the calls above beyond this view's 66 tiles.
    w, h, tile = 33 * 4 - 3, 2 * 4 - 1, 4
    tw, th = nat.tiles(w, h, tile)
    lengths = rng.integers(0, 3000, size=tw * th)
    lengths[:3] = 70000  # capped at 2^16 - 1: ties broken by index
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile)
    print(f"[noalloc] small ranges {tw * th} tiles", flush=True)
    expected, got = _both_orders(device, view, tw * th,
                                 ranges=torch.as_tensor(_ranges(lengths)).to(device))
    np.testing.assert_array_equal(got, expected)
    np.testing.assert_array_equal(got, expected_plan(lengths, tile))

    # A 2 x 2 mosaic of 200 x 120 views in 8-pixel tiles, by contributors.
    w, h, tile, views, cols = 200, 120, 8, 4, 2
    tw, th = nat.tiles(w, h, tile)
    ncon = rng.integers(0, 300, size=(views, h, w)).astype(np.int32)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile, views=views, mosaic_cols=cols)
    print(f"[noalloc] mosaic {views * tw * th} tiles", flush=True)
    expected, got = _both_orders(device, view, views * tw * th,
                                 ncon=torch.as_tensor(ncon).to(device))
    np.testing.assert_array_equal(got, expected)

    # The op's backward plan: ranges and contributor counts together, with
    # lists above 8192 entries whose walks cross checkpoints, so the crossings
    # half of the scratch is written and the plan holds segment items (tile
    # 8: tiles of 16 pixels or more are split into quarters, without
    # segments, when fewer than 4096 of them have work).
    w, h, tile = 256, 192, 8
    tw, th = nat.tiles(w, h, tile)
    lengths = rng.integers(0, 3000, size=tw * th)
    long_tiles = rng.choice(tw * th, 24, replace=False)
    lengths[long_tiles] = rng.integers(9000, 40000, size=long_tiles.size)
    per_pixel = np.repeat(np.repeat(lengths.reshape(th, tw), tile, 0), tile, 1)[:h, :w]
    ncon = (rng.random((h, w)) * np.minimum(per_pixel, 6000)).astype(np.int32)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, tile)
    print(f"[noalloc] backward plan with crossings, {tw * th} tiles", flush=True)
    expected, got = _both_orders(device, view, tw * th,
                                 ranges=torch.as_tensor(_ranges(lengths)).to(device),
                                 ncon=torch.as_tensor(ncon).to(device))
    np.testing.assert_array_equal(got, expected)
    assert ((got >= 0) & ((got & 0x40) != 0)).any()
