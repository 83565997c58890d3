"""The parity tests' own checkers, pinned on the CPU: the proof that a set of
tile lists is exactly the stable (tile, depth, index) sort, which the full-size
GPU tests rely on, must accept the oracle's lists and reject each kind of
mistake (a swapped pair, a dropped, repeated or foreign entry, a wrong range);
the gradient criterion must accept and reject at its stated bounds."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import rasterizer as orc
from parity import assert_gradients_close, assert_lists_exact, oracle_tile_lists, restrict_lists


def _case(seed=0, n=400, tw=13, th=9):
    rng = np.random.default_rng(seed)
    x = np.sort(rng.integers(0, tw + 1, size=(n, 2)), 1)
    y = np.sort(rng.integers(0, th + 1, size=(n, 2)), 1)
    bounds = np.stack((x, y), 1).astype(np.int32)
    counts = ((x[:, 1] - x[:, 0]) * (y[:, 1] - y[:, 0])).astype(np.int32)
    counts[rng.random(n) < 0.1] = 0
    depth = (rng.integers(1, 40, size=n) / 8).astype(np.float32)  # ties
    keys, ids = orc.emit_intersections(bounds, depth, counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a))
    return t(sid), t(ranges), t(bounds), t(counts), t(depth), tw


def test_list_proof_accepts_the_oracle_lists():
    gids, ranges, bounds, counts, depth, tw = _case()
    stats = assert_lists_exact(gids, ranges, bounds, counts, depth, tw, chunk=97)
    assert stats["intersections"] == gids.numel() > 1000


@pytest.mark.parametrize("mistake", ["swap", "drop", "repeat", "foreign", "range", "uncounted"])
def test_list_proof_rejects_mistakes(mistake):
    gids, ranges, bounds, counts, depth, tw = _case(seed=1)
    gids, ranges, counts = gids.clone(), ranges.clone(), counts.clone()
    lengths = (ranges[:, 1] - ranges[:, 0]).numpy()
    t = int(np.argmax(lengths))
    s = int(ranges[t, 0])
    if mistake == "swap":  # two entries of one tile exchanged
        gids[s], gids[s + 1] = gids[s + 1].clone(), gids[s].clone()
    elif mistake == "drop":  # last entry of a tile replaced by the next tile's first
        e = int(ranges[t, 1])
        gids[e - 1] = gids[e] if e < gids.numel() else gids[0]
    elif mistake == "repeat":
        gids[s + 1] = gids[s]
    elif mistake == "foreign":  # a Gaussian whose rectangle misses the tile
        tx, ty = t % tw, t // tw
        b = bounds.reshape(-1, 4)
        miss = ~((b[:, 0] <= tx) & (tx < b[:, 1]) & (b[:, 2] <= ty) & (ty < b[:, 3]))
        gids[s] = int(torch.nonzero(miss & (counts > 0))[0])
    elif mistake == "range":  # one entry moved across a tile boundary
        ranges[t, 1] -= 1
        ranges[t + 1, 0] -= 1
    else:  # a listed Gaussian marked as culled
        counts[int(gids[s])] = 0
    with pytest.raises(AssertionError):
        assert_lists_exact(gids, ranges, bounds, counts, depth, tw, chunk=64)


def test_oracle_tile_lists_and_restriction_match_the_full_sort():
    gids, ranges, bounds, counts, depth, tw = _case(seed=2)
    tiles = [0, 5, 17, 40, 100]
    ids, r = oracle_tile_lists(bounds.numpy(), counts.numpy(), depth.numpy(), tiles, tw, ranges.shape[0])
    ids2, r2 = restrict_lists(gids.numpy(), ranges.numpy(), tiles)
    assert np.array_equal(ids, ids2) and np.array_equal(r, r2)
    limits = {t: 3 for t in tiles}
    ids3, r3 = restrict_lists(gids.numpy(), ranges.numpy(), tiles, limits)
    ids4, r4 = oracle_tile_lists(bounds.numpy(), counts.numpy(), depth.numpy(), tiles, tw,
                                 ranges.shape[0], limits)
    assert np.array_equal(ids3, ids4) and np.array_equal(r3, r4)
    assert int((r3[:, 1] - r3[:, 0]).max()) <= 3


def test_gradient_criterion_bounds():
    e = torch.tensor([[2.0, 1e-3], [-4.0, 0.0], [0.5, 2e-3]])
    ok = e * (1 + 0.9e-4)
    assert_gradients_close(ok, e, "within rtol")
    # The absolute term is 1e-6 * min(1, column max): 1e-6 on column 0 ...
    assert_gradients_close(e + torch.tensor([[0.0, 0.0], [0.0, 0.0], [0.0, 0.0]]), e, "exact")
    bad = e.clone()
    bad[1, 0] += 4.0 * 1e-4 + 2e-6
    with pytest.raises(AssertionError):
        assert_gradients_close(bad, e, "beyond rtol + atol")
    # ... and 1e-6 * 2e-3 on column 1, whose entries are all small.
    bad = e.clone()
    bad[1, 1] = 3e-9
    with pytest.raises(AssertionError):
        assert_gradients_close(bad, e, "small column")
    assert_gradients_close(bad, e, "explained", explained=torch.tensor([False, True, False]),
                           max_explained=0.34)
    with pytest.raises(AssertionError):
        assert_gradients_close(bad, e, "unexplained", explained=torch.tensor([True, False, True]))


def test_gradient_criterion_float32_clause():
    """A row off by more than the strict bound passes when within
    FLOAT32_FACTOR (8) times the largest error of the float32 evaluations
    on that row, and fails beyond."""
    from parity import FLOAT32_FACTOR

    assert FLOAT32_FACTOR == 8.0
    e = torch.tensor([[88.0, -1e-3, 7.0], [1.0, 2.0, 3.0]], dtype=torch.float64)
    r32 = e.clone()
    r32[0, 1] += 1e-4  # float32 cancellation error of the reference's numerics
    a = e.clone()
    a[0, 1] += 3e-4
    with pytest.raises(AssertionError):
        assert_gradients_close(a, e, "strict")
    stats = assert_gradients_close(a, e, "float32 clause", reference32=r32)
    assert stats["at_float32_accuracy"] == 1
    assert abs(stats["float32_factor_needed"] - 3.0) < 1e-9
    a[0, 1] = e[0, 1] + 7.9e-4
    assert_gradients_close(a, e, "within 8x", reference32=r32)
    other = e.clone()
    other[0, 1] -= 2e-4  # a second float32 evaluation, further off
    a[0, 1] = e[0, 1] + 1.5e-3
    assert_gradients_close(a, e, "within 8x of the largest", reference32=[r32, other])
    with pytest.raises(AssertionError):
        assert_gradients_close(a, e, "beyond 8x", reference32=r32)


def test_ulp_perturbation():
    from parity import ulp_perturbed

    x = torch.tensor([1.0, -2.5, 3e-8, 0.0])
    (same,) = ulp_perturbed([x], 0)
    assert torch.equal(same, x)
    (moved,) = ulp_perturbed([x], 3)
    steps = torch.stack((torch.nextafter(x, torch.full_like(x, math.inf)),
                         torch.nextafter(x, torch.full_like(x, -math.inf))))
    assert bool(((moved == steps[0]) | (moved == steps[1])).all())
    assert not torch.equal(moved, x)


def _near_cut_scene():
    """Two isotropic Gaussians (variance 4, alpha0 0.5) on a 16 x 8 image, one
    tile of 16: the first placed so that pixel (9, 3) sees alpha =
    (1 + 2e-7) / 255, a cut decision within orc.CUT_NEAR of 1/255; the second
    behind it over the whole image."""
    d2 = -2 * math.log(2 * (1 + 2e-7) / 255)  # alpha0 exp(-D/2) = (1 + 2e-7) / 255
    u0 = 9.0 - math.sqrt(4 * d2)
    cols = [torch.tensor([u0, 8.0]), torch.tensor([3.0, 4.0]), torch.tensor([0.25, 0.01]),
            torch.tensor([0.0, 0.0]), torch.tensor([0.25, 0.01]),
            torch.tensor([[0.9, 0.4, 0.2], [0.1, 0.8, 0.3]]), torch.tensor([0.5, 0.5])]
    ids = np.array([0, 1], dtype=np.int32)
    ranges = np.array([[0, 2]], dtype=np.int64)
    return cols, ids, ranges


def test_every_pixel_check_resolves_a_near_cut():
    """The float32 oracle's own image passes; the image of a compositor that
    dropped the near-cut entry passes through the flipped hypothesis; an
    image off by 1e-4 at one pixel fails."""
    from parity import assert_forward_every_pixel

    cols, ids, ranges = _near_cut_scene()
    run = orc.composite(*cols, ids, ranges, 16, 8, 16)
    assert int(run.cut_near[3, 9]) == 1
    stats = assert_forward_every_pixel(run.image, run.final_transmittance, run.n_contributors,
                                       cols, ids, ranges, 16, 8, 16, what="self")
    assert stats["one_near_cut"] >= 1 and stats["matched_flipped"] == 0
    keep, clamped = run.decisions[0]
    dropped = orc.composite(*(c.double() for c in cols), ids, ranges, 16, 8, 16,
                            decisions={0: (keep ^ run.near_pairs[0], clamped)},
                            active_counts=run.n_contributors.numpy())
    assert float((dropped.image - run.image.double()).abs().max()) > 1e-4
    stats = assert_forward_every_pixel(dropped.image.float(), dropped.final_transmittance.float(),
                                       run.n_contributors, cols, ids, ranges, 16, 8, 16,
                                       what="dropped")
    assert stats["matched_flipped"] >= 1
    planted = run.image.clone()
    planted[5, 2, 1] += 1e-4
    with pytest.raises(AssertionError):
        assert_forward_every_pixel(planted, run.final_transmittance, run.n_contributors, cols,
                                   ids, ranges, 16, 8, 16, what="planted")
