"""Host logic of the multi-view op (no GPU): mosaic layout and camera arrays."""

from __future__ import annotations

import math

import pytest
import torch

from gaussian_splats_hip.kernels.rasterize.intersections import MAX_BUCKET_TILES
from gaussian_splats_hip.kernels.rasterize.views import camera_tensors, mosaic_columns
from gaussian_splats_hip.splats import PinholeCamera


@pytest.mark.parametrize("views", [1, 2, 3, 5, 16, 17, 40])
@pytest.mark.parametrize("tiles", [(50, 50), (120, 68), (10, 30)])
def test_mosaic_columns_is_the_squarest_fitting_layout(views, tiles):
    tw, th = tiles
    cols = mosaic_columns(views, tw, th)
    assert 1 <= cols <= views
    rows = math.ceil(views / cols)

    def side(c):
        return max(c * tw, math.ceil(views / c) * th)

    def fits(c):
        return c * tw <= MAX_BUCKET_TILES and math.ceil(views / c) * th <= MAX_BUCKET_TILES

    candidates = [c for c in range(1, views + 1) if fits(c)] or list(range(1, views + 1))
    assert fits(cols) or not any(fits(c) for c in range(1, views + 1))
    assert side(cols) == min(side(c) for c in candidates)
    assert rows * cols >= views


def test_config5_mosaic_is_four_by_four():
    # 16 views of 800 x 800 at tile 16: 50 x 50 tiles each -> a 200 x 200 grid.
    assert mosaic_columns(16, 50, 50) == 4


def test_camera_tensors_shapes_and_values():
    cams = [
        PinholeCamera.look_at(
            (3 * math.sin(a), 0.0, 3 * math.cos(a)), image_size=(64, 48),
            focal_length=(80.0 + a, 70.0), principal_point=(32.0, 24.0 + a),
        )
        for a in (0.0, 1.0, 2.0)
    ]
    r, t, k, w, h = camera_tensors(cams)
    assert (w, h) == (64, 48)
    assert r.shape == (3, 3, 3) and t.shape == (3, 3) and k.shape == (3, 4)
    for i, cam in enumerate(cams):
        assert torch.equal(r[i], cam.rotation_matrix.float())
        assert torch.equal(t[i], cam.translation.float())
        assert k[i].tolist() == [80.0 + i, 70.0, 32.0, 24.0 + i]


def test_camera_tensors_rejects_mixed_sizes_and_empty():
    cams = [
        PinholeCamera.look_at((0.0, 0.0, 3.0), image_size=(64, 64)),
        PinholeCamera.look_at((0.0, 0.0, 3.0), image_size=(64, 48)),
    ]
    with pytest.raises(ValueError, match="one image size"):
        camera_tensors(cams)
    with pytest.raises(ValueError, match="at least one camera"):
        camera_tensors([])
