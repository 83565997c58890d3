"""The compositing backward's use of its forward's walk state: the hit masks
and checkpoints gs_composite records (no counterpart in the reference, whose
composite_bwd, src/gaussian_splats/kernels/rasterize/composite_bwd.py:207-277,
is a pure function of its arguments).

* ``composite_bwd`` uses a forward's masks and checkpoints only for that
  forward's own arguments and outputs: after composite(A) and composite(B) on
  the same lists, the backward of A equals the backward without masks or
  checkpoints, and so does a backward whose arguments mix A and B.
* A checkpoint buffer with room for one or two records: the crossings past
  them are marked missing and walked from the list's end.  The gradients
  equal the unsegmented backward.
* A checkpoint buffer no forward stamped (zero-filled, so every table slot
  looks like record 0): the backward ignores it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splats_hip import scenes
from gaussian_splats_hip.kernels.rasterize import _native as nat
from gaussian_splats_hip.kernels.rasterize import composite, composite_bwd
from gaussian_splats_hip.kernels.rasterize.composite import tile_order, walk_key
from gaussian_splats_hip.kernels.rasterize.project import pack_records
from oracle import rasterizer as orc
from parity import oracle_camera, segmented_scene

pytestmark = pytest.mark.gpu

THRESHOLD = 0.999


def _plain_backward(device, cols, gids, granges, grad_image, final_t, ncon, w, h, ts,
                    order=None, checkpoints=None, checkpoint_bytes=0):
    """gs_composite_bwd through the C ABI with no hit masks and the given
    checkpoint buffer (none by default)."""
    n = cols[0].shape[0]
    out = torch.zeros((n, 9), dtype=torch.float32, device=device)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, ts, opacity_threshold=THRESHOLD)
    ids32 = gids.to(torch.int32).contiguous()
    nat.check(nat.library().gs_composite_bwd(
        *(nat.ptr(t) for t in cols), n, nat.ptr(ids32), nat.ptr(granges), nat.ptr(grad_image),
        nat.ptr(final_t), nat.ptr(ncon), nat.ptr(order), view, nat.ptr(out), None,
        nat.ptr(checkpoints), checkpoint_bytes, ids32.numel(), None, 0, nat.stream(device)),
        "composite_bwd")
    torch.cuda.synchronize(device)
    return out


def _assert_same_gradient(actual, expected, what):
    """Equal up to the order of the atomic adds: 1e-5 of each column's largest."""
    scale = expected.abs().amax(dim=0, keepdim=True).clamp_min(1e-30)
    err = float(((actual - expected).abs() / scale).max())
    print(f"[walk state] {what}: {err:.2e} of the column maxima", flush=True)
    assert err < 1e-5, what


def test_backward_uses_only_its_own_forwards_masks(device):
    scene = scenes.edge_case_scene(n=800, sh_degree=1, image_size=(80, 64))
    cam = scene.cameras[0]
    w, h = cam.image_size
    ts = 16
    proj = orc.project(*scene.params(), oracle_camera(cam))
    tw, th = nat.tiles(w, h, ts)
    bounds, counts = orc.tile_counts(proj, ts, tw, th, scene.near, scene.far)
    keys, ids = orc.emit_intersections(bounds, proj.mean[:, 2].float().numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    dev = lambda x: x.detach().float().contiguous().to(device)
    cols_a = [dev(proj.mean), dev(proj.inverse), dev(proj.color), dev(proj.opacity)]
    # B: the same lists with every opacity halved, as a finite-difference
    # probe or another threshold would give.
    cols_b = cols_a[:3] + [cols_a[3] * 0.5]
    gids = torch.as_tensor(sid).to(device)
    granges = torch.as_tensor(ranges).to(device)
    grad_image = (torch.rand(h, w, 3, generator=torch.Generator().manual_seed(3)) * 2 - 1).to(device)

    print("[walk state] composite(A), composite(B), composite_bwd(A)", flush=True)
    img_a, t_a, n_a = composite(*cols_a, gids, granges, w, h, ts, THRESHOLD, "gaussian", 0.95)
    img_b, t_b, n_b = composite(*cols_b, gids, granges, w, h, ts, THRESHOLD, "gaussian", 0.95)
    # The masks of A are still recorded with A's outputs and still match A.
    key_a = walk_key(w, h, ts, THRESHOLD, "gaussian", *cols_a, gids, granges, t_a, n_a)
    assert nat.walk_buffers(n_a, key_a)[1] is not None
    grad_a = composite_bwd(*cols_a, gids, granges, grad_image, t_a, n_a, w, h, ts, THRESHOLD,
                           "gaussian")
    _assert_same_gradient(grad_a, _plain_backward(device, cols_a, gids, granges, grad_image,
                                                  t_a, n_a, w, h, ts), "backward of A")
    # Arguments that mix A's projection with B's outputs match no forward.
    key_mix = walk_key(w, h, ts, THRESHOLD, "gaussian", *cols_a, gids, granges, t_b, n_b)
    assert nat.walk_buffers(n_b, key_mix) == (None, None)
    grad_mix = composite_bwd(*cols_a, gids, granges, grad_image, t_b, n_b, w, h, ts, THRESHOLD,
                             "gaussian")
    _assert_same_gradient(grad_mix, _plain_backward(device, cols_a, gids, granges, grad_image,
                                                    t_b, n_b, w, h, ts), "mixed arguments")
    # An output changed in place no longer matches its forward.
    n_a.add_(0)
    assert nat.walk_buffers(n_a, walk_key(w, h, ts, THRESHOLD, "gaussian", *cols_a, gids,
                                          granges, t_a, n_a)) == (None, None)


def _checkpoint_header_bytes(num_intersections):
    """The buffer's counter/stamp block and table (256-byte granules)."""
    table = (num_intersections // 1024 + 2) * 4
    return 256 + -(-table // 256) * 256


@pytest.mark.parametrize("records", (0, 1, 2))
def test_backward_with_a_full_checkpoint_pool(device, records):
    """Room for `records` checkpoint records while the two long lists cross
    two or three checkpoints between them."""
    w = h = 64
    ts = 8
    pmean, pinv, pcol, pop, sid, ranges = segmented_scene(9000, w, h, ts)
    dev = lambda x: x.detach().float().contiguous().to(device)
    cols = [dev(pmean), dev(pinv), dev(pcol), dev(pop)]
    gids = torch.as_tensor(sid).to(device)
    granges = torch.as_tensor(ranges).to(device)
    ids32 = gids.to(torch.int32).contiguous()
    grad_image = (torch.rand(h, w, 3, generator=torch.Generator().manual_seed(5)) * 2 - 1).to(device)
    records_buf = pack_records(*cols, "gaussian", 0.95)
    nbytes = _checkpoint_header_bytes(ids32.numel()) + records * 64 * 16
    full = nat.library().gs_composite_checkpoint_bytes(
        nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, ts), ids32.numel(), 9000)
    assert 0 < nbytes < full
    raw = torch.full((nbytes + 256,), 0x55, dtype=torch.uint8, device=device)
    off = (-raw.data_ptr()) % 256
    ckpt = raw[off:off + nbytes]
    image = torch.empty((h, w, 3), device=device)
    final_t = torch.empty((h, w), device=device)
    ncon = torch.empty((h, w), dtype=torch.int32, device=device)
    view = nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, ts, opacity_threshold=THRESHOLD)
    print(f"[walk state] checkpoint pool of {records} records", flush=True)
    nat.check(nat.library().gs_composite(
        nat.ptr(records_buf), records_buf.shape[0], nat.ptr(ids32), ids32.numel(),
        nat.ptr(granges), None, view, nat.ptr(image), nat.ptr(final_t), nat.ptr(ncon),
        nat.ptr(ckpt), nbytes, None, 0, None, 0, nat.stream(device)), "composite")
    order = tile_order(granges, ncon, w, h, ts)
    plan = order.cpu().numpy()
    assert ((plan >= 0) & ((plan & 0x40) != 0)).any()  # the plan has segment items
    segmented = _plain_backward(device, cols, gids, granges, grad_image, final_t, ncon, w, h, ts,
                                order=order, checkpoints=ckpt, checkpoint_bytes=nbytes)
    whole = _plain_backward(device, cols, gids, granges, grad_image, final_t, ncon, w, h, ts)
    _assert_same_gradient(segmented, whole, f"{records} records")


def test_backward_ignores_an_unstamped_checkpoint_buffer(device):
    """A zero-filled buffer: table slot 0 everywhere, i.e. record 0 (all
    zeros) for every crossing.  Read as checkpoints, those records would start
    every segment at T = 0; the stamp check keeps the backward off them."""
    w = h = 64
    ts = 8
    pmean, pinv, pcol, pop, sid, ranges = segmented_scene(9000, w, h, ts)
    dev = lambda x: x.detach().float().contiguous().to(device)
    cols = [dev(pmean), dev(pinv), dev(pcol), dev(pop)]
    gids = torch.as_tensor(sid).to(device)
    granges = torch.as_tensor(ranges).to(device)
    grad_image = (torch.rand(h, w, 3, generator=torch.Generator().manual_seed(6)) * 2 - 1).to(device)
    image, final_t, ncon = composite(*cols, gids, granges, w, h, ts, THRESHOLD, "gaussian", 0.95,
                                     record_hits=False)
    nbytes = nat.library().gs_composite_checkpoint_bytes(
        nat.make_view(1.0, 1.0, 0.0, 0.0, w, h, ts), gids.numel(), 9000)
    raw = torch.zeros(nbytes + 256, dtype=torch.uint8, device=device)
    off = (-raw.data_ptr()) % 256
    ckpt = raw[off:off + nbytes]
    order = tile_order(granges, ncon, w, h, ts)
    print("[walk state] unstamped checkpoint buffer", flush=True)
    got = _plain_backward(device, cols, gids, granges, grad_image, final_t, ncon, w, h, ts,
                          order=order, checkpoints=ckpt, checkpoint_bytes=nbytes)
    whole = _plain_backward(device, cols, gids, granges, grad_image, final_t, ncon, w, h, ts)
    _assert_same_gradient(got, whole, "unstamped buffer")
    assert np.isfinite(got.cpu().numpy()).all()
