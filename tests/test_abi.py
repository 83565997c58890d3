"""C-ABI and host-logic checks that need no GPU: the library loads and exports
every symbol include/gs_raster.h declares, host-side validation returns the
documented status codes, and the Python boundary rejects what the reference
rejects.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from gaussian_splats_hip.kernels.rasterize import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "gs_raster.h"


def _declared():
    text = HEADER.read_text()
    return re.findall(r"GS_API\s+[\w\s\*]+?\b(gs_\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    lib = nat.library()
    names = _declared()
    assert len(names) >= 16
    for name in names:
        assert hasattr(lib, name), name
    assert lib.gs_abi_version() == nat.ABI_VERSION


def test_workspace_queries_are_host_only():
    lib = nat.library()
    assert lib.gs_scan_workspace_bytes(0) > 0
    assert lib.gs_sort_workspace_bytes(1 << 20, 8160) >= (1 << 20) * 16
    assert lib.gs_bin_workspace_bytes(1000) > lib.gs_bin_workspace_bytes(10)


def test_tile_order_host_checks():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    null = ctypes.c_void_p(0)
    assert lib.gs_tile_order_workspace_bytes(8160) >= 8160 * 4
    ws = lib.gs_tile_order_workspace_bytes(8160)
    view = _view(tile_size=16)
    assert lib.gs_tile_order(null, null, view, fake, fake, ws, 0, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_tile_order(fake, null, view, null, fake, ws, 0, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_tile_order(fake, null, view, fake, fake, 0, 0, null) == nat.GS_ERR_WORKSPACE
    assert lib.gs_tile_order(fake, null, _view(tile_size=3), fake, fake, ws, 0, null) in (
        nat.GS_ERR_INVALID_ARGUMENT, nat.GS_ERR_UNSUPPORTED)


def test_l1_loss_host_checks():
    """The fused L1 loss validates sizes, pointers and workspace on the host."""
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    ws_bytes = lib.gs_l1_loss_workspace_bytes(1 << 20)
    assert ws_bytes >= 4
    null = ctypes.c_void_p(0)
    assert lib.gs_l1_loss_fwd(fake, fake, -1, 0, fake, fake, fake, ws_bytes, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_l1_loss_fwd(null, fake, 8, 0, fake, fake, fake, ws_bytes, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_l1_loss_fwd(fake, fake, 8, 0, fake, fake, fake, ws_bytes - 1, null) == nat.GS_ERR_WORKSPACE
    assert lib.gs_l1_loss_bwd(null, fake, 8, fake, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_l1_loss_bwd(fake, fake, -1, fake, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_l1_loss_bwd(null, null, 0, null, null) == nat.GS_OK  # empty: nothing to do


def test_ssim_host_checks():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    null = ctypes.c_void_p(0)
    assert lib.gs_ssim_workspace_bytes(10, 100) == 0
    ws = lib.gs_ssim_workspace_bytes(1080, 1920)
    assert ws >= 3 * 1080 * 1920 * 3 * 4
    assert lib.gs_ssim_fwd(fake, fake, 10, 100, fake, fake, ws, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ssim_fwd(null, fake, 1080, 1920, fake, fake, ws, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_ssim_fwd(fake, fake, 1080, 1920, fake, fake, ws - 1, null) == nat.GS_ERR_WORKSPACE
    assert lib.gs_ssim_bwd(fake, fake, 1080, 1920, fake, fake, 16, fake, null) == nat.GS_ERR_WORKSPACE
    assert lib.gs_ssim_bwd(fake, fake, 1080, 1920, null, fake, ws, fake, null) == nat.GS_ERR_INVALID_ARGUMENT


def test_adam_and_regularizer_host_checks():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    null = ctypes.c_void_p(0)
    t = nat.GsAdamTensor(16, 16, 16, 16, 100, 1e-3, 0)  # step 0 is invalid
    arr = (nat.GsAdamTensor * 1)(t)
    p = ctypes.cast(arr, ctypes.c_void_p)
    assert lib.gs_adam_step(p, 1, 0.9, 0.999, 1e-15, 0.0, null) == nat.GS_ERR_INVALID_ARGUMENT
    arr[0].step = 1
    assert lib.gs_adam_step(p, 1, 1.0, 0.999, 1e-15, 0.0, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_adam_step(p, nat.ADAM_MAX_TENSORS + 1, 0.9, 0.999, 1e-15, 0.0, null) == nat.GS_ERR_INVALID_ARGUMENT
    arr[0].grad = None
    assert lib.gs_adam_step(p, 1, 0.9, 0.999, 1e-15, 0.0, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_adam_step(null, 0, 0.9, 0.999, 1e-15, 0.0, null) == nat.GS_OK  # nothing to do
    ws = lib.gs_splat_regularizers_workspace_bytes(1000)
    assert lib.gs_splat_regularizers_fwd(fake, fake, -1, fake, fake, ws, null) == nat.GS_ERR_INVALID_ARGUMENT
    assert lib.gs_splat_regularizers_fwd(fake, fake, 10, fake, fake, ws - 1, null) == nat.GS_ERR_WORKSPACE
    assert lib.gs_splat_regularizers_bwd(fake, null, 10, fake, fake, fake, null) == nat.GS_ERR_INVALID_ARGUMENT


def test_l1_loss_python_checks():
    from gaussian_splats_hip.training import l1_loss

    x = torch.zeros(4, 4, 3)
    with pytest.raises(ValueError, match="ROCm GPU"):
        l1_loss(x, torch.zeros(4, 4, 3))
    with pytest.raises(ValueError, match="target"):
        l1_loss(x, torch.zeros(4, 4, 3, requires_grad=True))
    with pytest.raises(TypeError):
        l1_loss(x.double(), torch.zeros(4, 4, 3))


def test_bucketed_binning_host_checks():
    """Row/column bucketing: grid limits, sizes and inconsistent totals are
    rejected on the host before any launch."""
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    assert lib.gs_bin_tiles_plan_bytes(1000, 120, 68) > lib.gs_bin_tiles_plan_bytes(10, 120, 68)
    assert lib.gs_bin_tiles_plan_bytes(-1, 120, 68) == 0
    assert lib.gs_bin_tiles_emit_bytes(1000, 1 << 20, 1 << 18, 300, 120, 68) >= 3 * 4 * (1 << 18)
    status = lib.gs_bin_tiles_plan(fake, fake, 10, 0, 32, 257, 4, fake, fake, None, fake, 1 << 20,
                                   None, 0, None)
    assert status == nat.GS_ERR_UNSUPPORTED
    assert b"at most 256" in lib.gs_last_error()
    status = lib.gs_bin_tiles_plan(fake, fake, 10, 0, 32, 120, 68, fake, fake, None, fake, 16, None,
                                   0, None)
    assert status == nat.GS_ERR_WORKSPACE
    # the buffer to clear must be 16-byte aligned, a multiple of 4 bytes
    status = lib.gs_bin_tiles_plan(fake, fake, 10, 0, 32, 120, 68, fake, fake, None, fake, 1 << 30,
                                   fake, 6, None)
    assert status == nat.GS_ERR_INVALID_ARGUMENT
    # the row pass's look-back packs a row's entry count into 26 bits
    status = lib.gs_bin_tiles_plan(fake, fake, 1 << 26, 0, 32, 120, 68, fake, fake, None, fake,
                                   1 << 40, None, 0, None)
    assert status == nat.GS_ERR_OVERFLOW
    assert b"fewer than 67108864 Gaussians" in lib.gs_last_error()
    # the depth sort's key range: 1 to 32 bits
    for bits in (0, 33):
        status = lib.gs_bin_tiles_plan(fake, fake, 10, 0, bits, 120, 68, fake, fake, None, fake,
                                       1 << 30, None, 0, None)
        assert status == nat.GS_ERR_INVALID_ARGUMENT
        assert b"key_bits" in lib.gs_last_error()
    status = lib.gs_pack_tile_rects(fake, fake, 10, 257, 4, fake, None)
    assert status == nat.GS_ERR_UNSUPPORTED
    # pass-B workgroups must match the intersection total (ceil(total / 4096) .. + rows)
    status = lib.gs_bin_tiles_emit(
        10, 120, 68, fake, 100000, 5000, 1, fake, 1 << 30, fake, fake, fake, 1 << 30, None
    )
    assert status == nat.GS_ERR_INVALID_ARGUMENT
    status = lib.gs_bin_tiles_emit(
        10, 120, 68, fake, 1 << 33, 5000, 1 << 22, fake, 1 << 30, fake, fake, fake, 1 << 30, None
    )
    assert status == nat.GS_ERR_OVERFLOW


def _view(**kw):
    args = dict(fx=100.0, fy=100.0, cx=50.0, cy=50.0, image_width=100, image_height=100, tile_size=16)
    args.update(kw)
    return nat.make_view(**args)


def test_project_rejects_unsupported_sh_before_launch():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    status = lib.gs_project_and_count(
        fake, fake, fake, fake, fake, 10, 25, fake, fake, _view(), *([fake] * 6), None, None, None,
        None,
    )
    assert status == nat.GS_ERR_UNSUPPORTED
    assert b"SH degrees above 3" in lib.gs_last_error()
    # packed tile rectangles need a grid of at most 256 x 256 tiles
    status = lib.gs_project_and_count(
        fake, fake, fake, fake, fake, 10, 16, fake, fake, _view(image_width=257 * 16), *([fake] * 6),
        None, None, fake, None,
    )
    assert status == nat.GS_ERR_UNSUPPORTED
    assert b"at most 256" in lib.gs_last_error()
    # without bounds the projection needs tile_rects
    status = lib.gs_project_and_count(
        fake, fake, fake, fake, fake, 10, 16, fake, fake, _view(), *([fake] * 4), None, fake,
        None, None, None, None,
    )
    assert status == nat.GS_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("tile", (0, 3, 12, 64))
def test_invalid_tile_sizes(tile):
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    status = lib.gs_composite(fake, 10, fake, 10, fake, None, _view(tile_size=tile), fake, fake,
                              fake, None, 0, None, 0, None, 0, None)
    assert status in (nat.GS_ERR_INVALID_ARGUMENT, nat.GS_ERR_UNSUPPORTED)


def test_backward_rejects_ellipsoid_mode():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    status = lib.gs_composite_bwd(*([fake] * 4), 10, *([fake] * 5), None,
                                  _view(rendering_mode="ellipsoid"), fake, None, None, 0, 0,
                                  None, 0, None)
    assert status == nat.GS_ERR_UNSUPPORTED
    assert b"Gaussian rendering" in lib.gs_last_error()


def test_hit_masks_host_checks():
    """Hit masks are recorded in Gaussian mode only, and their buffer must hold
    gs_composite_hit_mask_bytes: both checked on the host, before any launch."""
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    view = _view(rendering_mode="ellipsoid")
    status = lib.gs_composite(fake, 10, fake, 10, fake, None, view, fake, fake, fake, None, 0,
                              fake, 1 << 20, None, 0, None)
    assert status == nat.GS_ERR_UNSUPPORTED
    assert b"Gaussian rendering" in lib.gs_last_error()
    need = lib.gs_composite_hit_mask_bytes(_view(), 10)
    assert need > 0 and need % 8 == 0
    status = lib.gs_composite(fake, 10, fake, 10, fake, None, _view(), fake, fake, fake, None, 0,
                              fake, need - 8, None, 0, None)
    assert status == nat.GS_ERR_WORKSPACE
    # the backward plan's key buffer holds two words per tile
    tiles = nat.tiles(100, 100, 16)
    status = lib.gs_composite(fake, 10, fake, 10, fake, None, _view(), fake, fake, fake, None, 0,
                              None, 0, fake, 8 * tiles[0] * tiles[1] - 4, None)
    assert status == nat.GS_ERR_WORKSPACE
    assert b"tile key buffer too small" in lib.gs_last_error()
    status = lib.gs_composite_bwd(*([fake] * 4), 10, *([fake] * 5), None, _view(), fake, None,
                                  None, 0, 10, fake, need - 8, None)
    assert status == nat.GS_ERR_WORKSPACE


def test_misaligned_buffers_rejected():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    bad = ctypes.c_void_p(20)
    status = lib.gs_project_and_count(
        fake, bad, fake, fake, fake, 10, 16, fake, fake, _view(), *([fake] * 6), None, None, None,
        None,
    )
    assert status == nat.GS_ERR_INVALID_ARGUMENT


def test_status_codes_map_to_python_exceptions():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    status = lib.gs_composite_bwd(*([fake] * 4), 10, *([fake] * 5), None,
                                  _view(rendering_mode="ellipsoid"), fake, None, None, 0, 0,
                                  None, 0, None)
    with pytest.raises(NotImplementedError):
        nat.check(status, "composite_bwd")


def test_cpu_tensors_are_rejected():
    """The product path has no CPU fallback: host tensors raise before any launch."""
    from gaussian_splats_hip.scenes import edge_case_scene
    from gaussian_splats_hip.splats import GaussianSplat, rasterize

    scene = edge_case_scene(n=40)
    splats = GaussianSplat.from_tensors(*scene.params())
    with pytest.raises(ValueError, match="ROCm GPU"):
        rasterize(splats, scene.cameras[0], tile_size=16)


def test_dispatcher_backends():
    from gaussian_splats_hip.splats import rasterize

    with pytest.raises(ValueError, match="Unknown rasterization backend"):
        rasterize(None, None, backend="cuda")
    with pytest.raises(ValueError, match="CPU path"):
        rasterize(None, None, backend="torch")


def test_tile_size_must_be_power_of_two():
    from gaussian_splats_hip.kernels.rasterize import project_and_count

    with pytest.raises(ValueError):
        project_and_count(*([torch.zeros(1)] * 7), 1.0, 1.0, 0.0, 0.0, 16, 16, 12, 0.1, 10.0,
                          "gaussian", 0.95)


def test_fake_implementation_shapes():
    """The op traces under FakeTensorMode (torch.compile path of the viewer)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.symbolic_shapes import ShapeEnv

    import gaussian_splats_hip.kernels.rasterize.interface  # noqa: F401 (registers the op)

    with FakeTensorMode(shape_env=ShapeEnv(allow_dynamic_output_shape_ops=True)):
        n, k = 7, 16
        args = [torch.empty(n, 3), torch.empty(n, 4), torch.empty(n, 3), torch.empty(n, 1),
                torch.empty(n, k, 3), torch.empty(3, 3), torch.empty(3)]
        out = torch.ops.gaussian_splats_hip.rasterize(*args, 100.0, 100.0, 60.0, 40.0, 120, 90, 16,
                                                  0.999, 0.2, 100.0, "gaussian", 0.95)
    shapes = [tuple(o.shape) for o in out]
    assert shapes[0] == (90, 120, 3) and shapes[1] == (90, 120) and shapes[2] == (90, 120)
    assert shapes[3] == (7, 3) and shapes[4] == (7, 2, 2) and shapes[8] == (8 * 6, 2)
    assert out[8].dtype == torch.int64 and out[7].dtype == torch.int32


def test_multi_view_host_checks():
    lib = nat.library()
    fake = ctypes.c_void_p(16)
    # Negative view counts and mosaic columns are rejected before any launch.
    for kw in (dict(views=-1), dict(mosaic_cols=-2)):
        status = lib.gs_project_views(
            fake, fake, fake, fake, fake, 10, 16, fake, fake, None, _view(**kw), *([fake] * 6),
            None, None, None, None,
        )
        assert status == nat.GS_ERR_INVALID_ARGUMENT
        status = lib.gs_composite(fake, 10, fake, 10, fake, None, _view(**kw), fake, fake, fake,
                                  None, 0, None, 0, None, 0, None)
        assert status == nat.GS_ERR_INVALID_ARGUMENT
    # Virtual Gaussian indices (view * N + i) must fit int32.
    status = lib.gs_project_views(
        fake, fake, fake, fake, fake, 1 << 28, 16, fake, fake, None, _view(views=16, mosaic_cols=4),
        *([fake] * 6), None, None, None, None,
    )
    assert status == nat.GS_ERR_OVERFLOW
    status = lib.gs_project_bwd_views(
        fake, fake, fake, fake, fake, 1 << 28, 16, fake, fake, None, _view(views=16),
        *([fake] * 8), None,
    )
    assert status == nat.GS_ERR_OVERFLOW
    # A mosaic whose tile grid overflows is rejected.
    status = lib.gs_composite(
        fake, 10, fake, 10, fake, None, _view(image_width=1 << 16, image_height=1 << 16,
                                              tile_size=4, views=64, mosaic_cols=8),
        fake, fake, fake, None, 0, None, 0, None, 0, None,
    )
    assert status == nat.GS_ERR_OVERFLOW
    # Zero Gaussians: nothing to do.
    assert lib.gs_project_views(None, None, None, None, None, 0, 16, None, None, None,
                                _view(views=3), *([None] * 9), None) == nat.GS_OK


def test_multi_view_fake_implementation_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.symbolic_shapes import ShapeEnv

    import gaussian_splats_hip.kernels.rasterize.views  # noqa: F401 (registers the op)

    with FakeTensorMode(shape_env=ShapeEnv(allow_dynamic_output_shape_ops=True)):
        n, k, v = 7, 16, 5
        args = [torch.empty(n, 3), torch.empty(n, 4), torch.empty(n, 3), torch.empty(n, 1),
                torch.empty(n, k, 3), torch.empty(v, 3, 3), torch.empty(v, 3), torch.empty(v, 4)]
        out = torch.ops.gaussian_splats_hip.rasterize_views(*args, 120, 90, 16, 0.999, 0.2, 100.0,
                                                        "gaussian", 0.95)
    shapes = [tuple(o.shape) for o in out]
    assert shapes[0] == (v, 90, 120, 3) and shapes[1] == (v, 90, 120) and shapes[2] == (v, 90, 120)
    assert shapes[3] == (v, n, 3) and shapes[4] == (v, n, 2, 2) and shapes[9] == (v, n)
    # 8 x 6 tiles per view; five views in a 3 x 2 mosaic.
    assert shapes[8] == (3 * 8 * 2 * 6, 2)
