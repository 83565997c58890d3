"""Benchmark of the HIP rasterizer on one MI355X.

A step is one training pass of the headline workload (scenes.CONFIGS['config3']):
render 1M SH-3 Gaussians at 1920x1080, mean |image - target| loss, backward to
all Gaussian parameters.  Inputs are resident in HBM before timing.  Prints one
JSON line with the whole-job Mpix/s, per-stage milliseconds from HIP events,
the roofline of the dominant kernel and the CPU-oracle baseline.

    python bench.py [--steps K] [--warmup W] [--config config3] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "gaussian-splats_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
VALU_CLOCK_HZ = 2.4e9  # MI355X peak engine clock
# The spin between the stages of the staged steps (stage_marker), about 250 us:
# longer than the host's wait for the binning totals and the launches after
# it, so no stage's time includes a host gap.
STAGE_HOLD_CYCLES = 600_000


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="config3")
    ap.add_argument(
        "--scene", default=None,
        help="time the step on a scene file instead (a GaussianSplat .pt checkpoint, e.g. a "
             "baked scene, or a .ply), viewed by a fitted 1920x1080 camera",
    )
    ap.add_argument("--tile-size", type=int, default=16)
    ap.add_argument(
        "--forward-only", action="store_true",
        help="time the forward render alone (configs 1 and 2 are forward-only workloads); the "
             "roofline line is then the forward compositing kernel's",
    )
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-tiles", type=int, default=128, help="tiles in the CPU baseline sample")
    ap.add_argument("--out", default=None, help="also write the JSON line to this file")
    ap.add_argument(
        "--train-step", action="store_true",
        help="time the reference's whole training step instead (train.py:136-152: clamp, "
             "L1 + D-SSIM + regularisers, backward, Adam) with the fused kernels, beside the "
             "same step written with torch ops",
    )
    ap.add_argument(
        "--view-loop", action="store_true",
        help="multi-view scenes: time one rasterize call per camera as the step (the "
             "reference's way) instead of one rasterize_views call over all cameras",
    )
    ap.add_argument(
        "--no-compare", action="store_true",
        help="multi-view scenes: time only the chosen path (for profiles)",
    )
    ap.add_argument(
        "--ply-io", action="store_true",
        help="time scene-file I/O instead: save_ply / load_ply of the config's Gaussians "
             "(GPU record pack/split against the host path)",
    )
    ap.add_argument(
        "--copy-calibration", action="store_true",
        help="only copy 512 MiB device to device three times (the known-size kernel that scales "
             "rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)",
    )
    return ap.parse_args()


def copy_calibration():
    """Three 512 MiB device-to-device copies: FETCH_SIZE / WRITE_SIZE of this
    kernel under rocprofv3 give the KiB-to-bytes factors of the traffic figures."""
    n = 128 * 1024 * 1024  # floats
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print("copied 512 MiB x3", flush=True)


def host_extrinsics(cam):
    """The camera extrinsics the rasterizer passes its kernels (float32, host)."""
    from gaussian_splats_hip.splats.camera import host_extrinsics as extrinsics

    return extrinsics(cam)


def stage_bytes(n, k, total, rows, pixels, processed_fwd, processed_bwd):
    """Algorithmic HBM bytes per stage (n Gaussians with k SH coefficients,
    `total` intersections, `rows` row-list entries)."""
    return {
        # params in (44 + 12k B) -> projected outputs (48 B), record (48 B),
        # depth key and packed tile rectangle (4 + 4 B)
        "project": n * (44 + 12 * k) + 104 * n,
        # depth sort: histogram, then 4 passes moving (key, id, packed
        # rectangle), the first reading only keys and rectangles (its ids are
        # the positions); the tables' rectangle reads; the row-list offset
        # scan (rectangles in, offsets out)
        "bin": 4 * n + 20 * n + 3 * 24 * n + 4 * n + 8 * n,
        # pass A writes (id, packed columns, row-major position) per row
        # entry; pass B reads its windows (packed columns, positions) and
        # writes one id per intersection
        "emit": 12 * rows + 8 * rows + 4 * total,
        "composite": 40 * processed_fwd + 20 * pixels,
        "composite_bwd": 76 * processed_bwd + 20 * pixels,
        # params in and gradients out; per Gaussian its 9 gradient inputs and
        # count (the 2-D inverse is recomputed, not read)
        "project_bwd": 2 * n * (44 + 12 * k) + 40 * n,
    }


# The kernels each stage of the step launches, in order (stage name -> kernels).
STAGE_KERNELS = {
    "project": ["project_fwd_kernel"],
    "bin": ["sweep::clear_kernel", "sweep::hist_kernel", "sweep::scatter_kernel x4 (depth sort)",
            "rect_diff_kernel", "tables_kernel", "sweep::scan_kernel<HeightLoad>"],
    "emit": ["sweep::clear_kernel", "row_bucket_kernel",
             "column_count_wave_kernel (or column_count_block_kernel)", "column_scan_kernel",
             "column_bucket_kernel"],
    # With row/column bucketing the lists leave the emit stage sorted: the
    # "sort" mark launches nothing and is not reported.
    "sort": [],
    "composite": ["checkpoint_clear_kernel (lists above 8192 entries)", "composite_fwd_kernel"],
    "loss": ["l1_fwd_kernel", "l1_finish_kernel", "l1_bwd_kernel", "torch fill (gradient buffer)"],
    "composite_bwd": ["tile_key_kernel", "tile_plan_kernel", "composite_bwd_kernel"],
    "project_bwd": ["project_bwd_kernel"],
}


def stage_entries(stages_ms, bytes_model):
    """Per stage: its kernels, time, algorithmic bytes and HBM fraction; and
    the whole binning (bin + emit) against its own bytes."""
    stages = {}
    for name, ms in stages_ms.items():
        if not STAGE_KERNELS.get(name, True):
            continue  # a mark with no kernel of its own (its time joins "binning")
        entry = {"kernels": STAGE_KERNELS.get(name, []), "ms": round(ms, 4)}
        if name in bytes_model and ms > 0:
            gbs = bytes_model[name] / (ms * 1e-3) / 1e9
            entry.update({"algorithmic_bytes": bytes_model[name], "GB/s": round(gbs, 1),
                          "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        stages[name] = entry
    if "bin" in stages_ms and "emit" in stages_ms:
        ms = stages_ms["bin"] + stages_ms["emit"] + stages_ms.get("sort", 0.0)
        nbytes = bytes_model["bin"] + bytes_model["emit"]
        gbs = nbytes / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
        stages["binning"] = {"kernels": STAGE_KERNELS["bin"] + STAGE_KERNELS["emit"],
                             "ms": round(ms, 4), "algorithmic_bytes": nbytes,
                             "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    return stages


def run_step(splats, cam, target, tile_size, near, far, backward=True):
    from gaussian_splats_hip.splats import rasterize
    from gaussian_splats_hip.training import l1_loss

    if not backward:
        with torch.no_grad():
            return rasterize(splats, cam, tile_size=tile_size, near=near, far=far)
    image = rasterize(splats, cam, tile_size=tile_size, near=near, far=far)
    loss = l1_loss(image, target)  # mean |image - target|, one fused kernel each way
    loss.backward()
    return loss


def stage_marker():
    """Stage timing events: mark(name) ends the running stage and starts the
    next one.  Between the two events the GPU spins (STAGE_HOLD_CYCLES), so the
    next stage's first kernels are queued by the time its start event fires:
    a stage's time then excludes the host's launch gap in front of it.
    Returns (mark, times) where times() gives {stage: ms} once synchronised."""
    starts, ends, order = {}, {}, []

    def mark(name):
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        ends[name] = end
        order.append(name)
        torch.cuda._sleep(STAGE_HOLD_CYCLES)
        start = torch.cuda.Event(enable_timing=True)
        start.record()
        starts[name] = start  # the start of the stage after `name`

    def times():
        return {b: starts[a].elapsed_time(ends[b]) for a, b in zip(order[:-1], order[1:])}

    return mark, times


def staged_step(params, cam, target, tile_size, near, far, backward=True):
    """One fwd+bwd (with ``backward``) through the stage functions with timing
    events around each stage (stage_marker)."""
    from gaussian_splats_hip.kernels.rasterize import composite_bwd, project_and_count, project_bwd
    from gaussian_splats_hip.kernels.rasterize.interface import forward_pipeline
    from gaussian_splats_hip.training import l1_loss_backward, l1_loss_forward

    mark, stage_times = stage_marker()

    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    one = torch.ones((), dtype=torch.float32, device=params[0].device)
    R, t = host_extrinsics(cam)  # host memory: passed to the kernels by value
    out = forward_pipeline(*params, R, t, fx, fy, cx, cy, w, h, tile_size, 0.999, near, far,
                           "gaussian", 0.95, timer=mark, record_hits=backward)
    image, final_t, ncon, pmean, pinv, pcol, pop, gids, ranges, counts = out
    if backward:
        _, code = l1_loss_forward(image, target)
        grad_image = l1_loss_backward(code, one)
        grad_proj = torch.zeros((pmean.shape[0], 9), dtype=torch.float32, device=pmean.device)
        mark("loss")
        composite_bwd(pmean, pinv, pcol, pop, gids, ranges, grad_image, final_t, ncon, w, h,
                      tile_size, 0.999, "gaussian", out=grad_proj)
        mark("composite_bwd")
        project_bwd(*params, R, t, pinv, grad_proj, counts, fx, fy, w, h)
        mark("project_bwd")
    torch.cuda.synchronize()
    ms = stage_times()
    # Row-list entries: tile rows covered by the Gaussians with intersections.
    _, _, _, _, bounds, counts2 = project_and_count(*params, R, t, fx, fy, cx, cy, w, h, tile_size,
                                                    near, far, "gaussian", 0.95)
    b = bounds.view(-1, 4).long()
    rows = int(((b[:, 3] - b[:, 2]) * (counts2 > 0)).sum())
    info = {
        "total": int(gids.numel()),
        "rows": rows,
        "ranges": ranges,
        "ncon": ncon,
        "counts": counts,
    }
    return ms, info


def processed_pairs(ranges, ncon, tile_size, w, h):
    """(tile, Gaussian) pairs visited by the forward (up to the last entry any
    pixel of the tile processed while active) and by the backward."""
    tw = -(-w // tile_size)
    th = -(-h // tile_size)
    pad = torch.zeros(th * tile_size, tw * tile_size, dtype=ncon.dtype, device=ncon.device)
    pad[:h, :w] = ncon
    per_tile = pad.reshape(th, tile_size, tw, tile_size).amax(dim=(1, 3)).reshape(-1).long()
    lengths = (ranges[:, 1] - ranges[:, 0]).long()
    fwd = int(torch.minimum(lengths, per_tile + 1).sum())
    bwd = int(torch.minimum(lengths, per_tile).sum())
    return fwd, bwd


def host_description():
    """CPU model, host memory and usable cores of the machine the baseline ran on."""
    model, mem_kb = "unknown", 0
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
        for line in Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemTotal"):
                mem_kb = int(line.split()[1])
                break
    except OSError:
        pass
    return {"cpu_model": model, "ram_gib": round(mem_kb / 2**20, 1),
            "logical_cpus": os.cpu_count() or 1}


def cpu_config1_full(threads):
    """The reference's CPU-runnable case (config 1: 10k Gaussians, SH0,
    256x256, forward only) rendered whole by the CPU oracle: one warm-up
    frame, then the median of three."""
    from gaussian_splats_hip import scenes
    from oracle import rasterizer as orc

    torch.set_num_threads(threads)
    scene = scenes.config1()
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    ocam = orc.Camera(*host_extrinsics(cam), fx, fy, cx, cy, w, h)
    times = []
    with torch.no_grad():
        for i in range(4):
            t0 = time.perf_counter()
            orc.rasterize(*scene.params(), ocam, tile_size=16, near=scene.near, far=scene.far,
                          diagnostics=False)
            if i > 0:
                times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    return {"value": round((w * h) / 1e6 / med, 4), "unit": "Mpix/s", "s_per_frame": round(med, 4),
            "frames": "warm-up 1, median of 3", "workload": f"config1 forward, {w}x{h}, "
            f"{scene.num_points} Gaussians, SH0, tile 16"}


# The CPU baseline runs the whole algorithm up to these sizes and extrapolates
# beyond them (labelled in its "sample" text).
CPU_SORT_CAP = 40_000_000  # intersections emitted and sorted whole
CPU_LIST_CAP = 20_000      # entries of one sampled tile composited whole
CPU_VIEWS = 2              # views of a multi-view scene timed (the mean is scaled to all)


def _cpu_tile_lists(bounds, counts, depth32, tiles, tiles_w):
    """The (depth bits, index)-ordered lists of the given tiles, straight from
    the rectangles: (ids, {tile: (start, end)})."""
    import numpy as np

    bits = np.ascontiguousarray(depth32, dtype=np.float32).view(np.uint32)
    live = counts > 0
    x0, x1, y0, y1 = bounds[:, 0, 0], bounds[:, 0, 1], bounds[:, 1, 0], bounds[:, 1, 1]
    parts, where, pos = [], {}, 0
    for t in tiles:
        ty, tx = divmod(int(t), tiles_w)
        cover = np.nonzero(live & (x0 <= tx) & (tx < x1) & (y0 <= ty) & (ty < y1))[0]
        ordered = cover[np.lexsort((cover, bits[cover]))].astype(np.int32)
        parts.append(ordered)
        where[int(t)] = (pos, pos + ordered.size)
        pos += ordered.size
    return (np.concatenate(parts) if parts else np.zeros(0, np.int32)), where


def cpu_baseline(scene, tile_size, sample_tiles, cam=None, target=None, backward=True,
                 with_config1=True):
    """The CPU oracle (torch-CPU restatement of the reference torch backend,
    dense per (intersection, pixel), no early exit, without the oracle's
    parity diagnostics) on a bounded sample of one
    view's step, timed on all host threads:

    * projection of all Gaussians, and their binning: emission and stable sort
      of all intersections, or, above CPU_SORT_CAP of them, of a seeded subset
      of Gaussians holding about CPU_SORT_CAP, its time scaled by I log I;
    * forward (and, with ``backward``, backward) compositing of
      ``sample_tiles`` non-empty tiles stratified by list length (equal
      numbers from each eighth of the tiles sorted by length, seeded), each
      eighth timed on its own, less the per-call cost that does not scale
      with the tiles (counted once), and scaled by its tile count.  A list
      above CPU_LIST_CAP entries is composited to that length and its time
      scaled by the full length: the dense oracle's work is linear in it;
    * the projection's backward, once, on the summed gradients.

    Also: config 1 whole (``with_config1``), and the host's CPU and memory."""
    import numpy as np

    from oracle import rasterizer as orc

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cam = cam or scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    ocam = orc.Camera(*host_extrinsics(cam), fx, fy, cx, cy, w, h)
    if target is None:
        if scene.target is None:  # forward-only scenes: a seeded target of the image's shape
            target = torch.rand(h, w, 3, generator=torch.Generator().manual_seed(0))
        else:
            target = scene.target if scene.target.dim() == 3 else scene.target[0]
    params = [p.detach().clone().requires_grad_(backward) for p in scene.params()]
    grad_mode = torch.enable_grad() if backward else torch.no_grad()
    notes = []
    with grad_mode:
        t0 = time.perf_counter()
        proj = orc.project(*params, ocam)
        tw, th = -(-w // tile_size), -(-h // tile_size)
        bounds, counts = orc.tile_counts(proj, tile_size, tw, th, scene.near, scene.far)
        depth32 = proj.mean[:, 2].detach().float().numpy()
        t1 = time.perf_counter()
        project_s = t1 - t0
        total = int(counts.astype(np.int64).sum())
        # Per-tile list lengths: a 2-D difference array of the rectangles.
        diff = np.zeros((th + 1, tw + 1), dtype=np.int64)
        live = counts > 0
        b = bounds[live].astype(np.int64)
        np.add.at(diff, (b[:, 1, 0], b[:, 0, 0]), 1)
        np.add.at(diff, (b[:, 1, 0], b[:, 0, 1]), -1)
        np.add.at(diff, (b[:, 1, 1], b[:, 0, 0]), -1)
        np.add.at(diff, (b[:, 1, 1], b[:, 0, 1]), 1)
        lengths_all = diff.cumsum(0).cumsum(1)[:th, :tw].reshape(-1)
        rng = np.random.default_rng(0)
        tb = time.perf_counter()
        if total <= CPU_SORT_CAP:
            keys, ids = orc.emit_intersections(bounds, depth32, counts, tw)
            sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
            bin_s = time.perf_counter() - tb
            notes.append(f"binning of all {total} intersections ({bin_s:.1f}s)")
            lists = None
        else:
            subset = rng.random(counts.size) < CPU_SORT_CAP / total
            sub_counts = np.where(subset, counts, 0)
            sub_total = int(sub_counts.astype(np.int64).sum())
            keys, ids = orc.emit_intersections(bounds, depth32, sub_counts, tw)
            orc.sort_intersections(keys, ids, tw * th)
            del keys, ids
            sub_s = time.perf_counter() - tb
            bin_s = sub_s * (total / sub_total) * (math.log(total) / math.log(sub_total))
            notes.append(f"binning of a seeded subset of {sub_total} of the {total} "
                         f"intersections ({sub_s:.1f}s), scaled by I log I to {bin_s:.1f}s")
            lists = True
        leaves = [t.detach().requires_grad_(backward)
                  for t in (proj.mean, proj.inverse, proj.color, proj.opacity)]
        pm, pinv, pcol, pop = leaves
        nonempty = np.nonzero(lengths_all > 0)[0]
        by_length = nonempty[np.argsort(lengths_all[nonempty], kind="stable")]
        strata = np.array_split(by_length, 8)
        per = max(1, sample_tiles // len(strata))
        chosen_all = [rng.choice(st, size=min(per, len(st)), replace=False) if len(st) else st
                      for st in strata]
        if lists:
            picked = np.concatenate([c for c in chosen_all if len(c)])
            sid, where = _cpu_tile_lists(bounds, counts, depth32, picked, tw)
        else:
            where = {int(t): (int(ranges[t, 0]), int(ranges[t, 1])) for t in nonempty}

        def mask_of(tiles):
            mask = torch.zeros(th * tile_size, tw * tile_size)
            for t in tiles:
                ty, tx = divmod(int(t), tw)
                mask[ty * tile_size:(ty + 1) * tile_size, tx * tile_size:(tx + 1) * tile_size] = 1
            return mask[:h, :w, None]

        def run(tiles, cap, grad=backward):
            """Composites the tiles' lists (each cut at cap entries) and the
            loss on their pixels (back-propagated with ``grad``); returns the
            scale full / composited."""
            sub = np.zeros((tw * th, 2), dtype=np.int64)
            pieces, pos, full, done = [], 0, 0, 0
            for t in tiles:
                s0, e0 = where[int(t)]
                e = min(e0, s0 + cap)
                pieces.append(sid[s0:e])
                sub[int(t)] = (pos, pos + e - s0)
                pos += e - s0
                full += e0 - s0
                done += e - s0
            ids_sub = np.concatenate(pieces) if pieces else np.zeros(0, np.int32)
            comp = orc.composite(pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1],
                                 pinv[:, 1, 1], pcol, pop[:, 0], ids_sub, sub, w, h, tile_size,
                                 tile_chunk=8, diagnostics=False)
            loss = ((comp.image - target).abs() * mask_of(tiles)).sum() / (w * h * 3)
            if grad:
                loss.backward()
            return full / max(done, 1)

        # The per-call cost that does not scale with the tiles (image-sized
        # buffers, the chunk loop, the loss): one call with every list empty.
        tc0 = te0 = time.perf_counter()
        with torch.no_grad():
            run([], CPU_LIST_CAP, grad=False)
        fixed_s = time.perf_counter() - te0
        composite_s = fixed_s
        sampled, scaled = 0, 0
        for stratum, chosen in zip(strata, chosen_all):
            if len(stratum) == 0:
                continue
            ts0 = time.perf_counter()
            factor = run(chosen, CPU_LIST_CAP)
            dt = max(time.perf_counter() - ts0 - fixed_s, 0.0) * factor
            composite_s += dt / len(chosen) * len(stratum)
            sampled += len(chosen)
            scaled += int(factor > 1.0)
        t2 = time.perf_counter()
        if backward:
            outs = [(o, l.grad) for o, l in zip(
                (proj.mean, proj.inverse, proj.color, proj.opacity), leaves)
                if l.grad is not None and o.requires_grad]
            torch.autograd.backward([o for o, _ in outs], [g for _, g in outs])
        t3 = time.perf_counter()
    full_s = project_s + bin_s + composite_s + (t3 - t2)
    what = "fwd+bwd" if backward else "forward"
    notes.append(
        f"dense {what} compositing of {sampled} non-empty {tile_size}px tiles, {per} from each "
        f"eighth of the tiles by list length ({t2 - tc0:.1f}s), each eighth's time per tile (less the {fixed_s:.2f}s per call that "
        f"does not scale with the tiles, counted once) scaled to its {len(nonempty) // 8}-odd "
        f"tiles" + (f"; {scaled} of the eighths held lists above {CPU_LIST_CAP} entries, composited to "
                    f"that length and scaled linearly by their full length" if scaled else ""))
    if backward:
        notes.append(f"the projection backward ({t3 - t2:.1f}s)")
    out = {
        "value": (w * h) / 1e6 / full_s,
        "unit": "Mpix/s",
        "cores": threads,
        "kind": "port",
        "s_per_view": round(full_s, 2),
        "sample": (f"torch-CPU oracle, float32, one view of {scene.num_points} Gaussians: "
                   f"projection ({project_s:.1f}s) + " + " + ".join(notes)
                   + f"; estimate {full_s:.1f}s per view"),
        "host": host_description(),
    }
    if with_config1:
        out["config1_full"] = cpu_config1_full(threads)
    return out


def views_stage_bytes(n, k, views, total, rows, pixels, processed_fwd, processed_bwd):
    """Algorithmic HBM bytes per stage of the multi-view step: the projection
    reads the parameters once per launch of up to 16 cameras and writes the
    104 B of outputs per (view, Gaussian); the backward reads the parameters
    once, 40 B per (view, Gaussian) and writes the gradients once."""
    launches = -(-views // 16)
    single = stage_bytes(views * n, k, total, rows, pixels, processed_fwd, processed_bwd)
    single["project"] = launches * n * (44 + 12 * k) + 104 * views * n
    single["project_bwd"] = (launches + 1) * n * (44 + 12 * k) + 40 * views * n
    return single


def bench_views(args, scene):
    """Multi-view scenes (config 5): a step renders every camera into a
    [V, H, W, 3] batch with one rasterize_views call (with --view-loop: one
    rasterize call per camera), takes the mean L1 against the per-view targets
    and back-propagates to all parameters."""
    from gaussian_splats_hip.kernels.rasterize import _native, project_and_count
    from gaussian_splats_hip.kernels.rasterize.views import (
        backward_views,
        camera_tensors,
        forward_views,
        mosaic_columns,
    )
    from gaussian_splats_hip.splats import GaussianSplat, rasterize, rasterize_views
    from gaussian_splats_hip.training import l1_loss, l1_loss_backward, l1_loss_forward

    device = torch.device("cuda:0")
    cams = scene.cameras
    views = len(cams)
    w, h = cams[0].image_size
    tile = args.tile_size
    splats = GaussianSplat.from_tensors(*(p.to(device) for p in scene.params()))
    target = scene.target.to(device)
    params = [p.detach() for p in (splats.mean, splats.rotation, splats.scale, splats.opacity,
                                   splats.color)]

    def step_batched():
        images = rasterize_views(splats, cams, tile_size=tile, near=scene.near, far=scene.far)
        l1_loss(images, target).backward()

    def step_loop():
        loss = 0.0
        for v, cam in enumerate(cams):
            image = rasterize(splats, cam, tile_size=tile, near=scene.near, far=scene.far)
            loss = loss + l1_loss(image, target[v])
        (loss / views).backward()

    timed = {}
    kinds = ("loop", "batched") if args.view_loop else ("batched", "loop")
    if args.no_compare:
        kinds = kinds[:1]
    for kind in kinds:
        step = step_batched if kind == "batched" else step_loop
        for _ in range(args.warmup):
            for p in splats.parameters():
                p.grad = None
            step()
        torch.cuda.synchronize()
        with _native.LaunchTimer("composite_bwd", capacity=args.steps * views + 1) as timer:
            t0 = time.perf_counter()
            for _ in range(args.steps):
                for p in splats.parameters():
                    p.grad = None
                step()
            torch.cuda.synchronize()
            timed[kind] = (1e3 * (time.perf_counter() - t0) / args.steps, timer.mean_ms())
        print(f"[bench] {kind}: {timed[kind][0]:.3f} ms/step", file=sys.stderr, flush=True)
    kind = kinds[0]
    ms_per_step, dominant_ms = timed[kind]

    # Per-stage events over the batched path: the median of three staged steps
    # after one untimed one.
    rot, trans, intr, _, _ = camera_tensors(cams)
    runs = []
    for i in range(4):
        mark, stage_times = stage_marker()
        out = forward_views(*params, rot, trans, intr, w, h, tile, 0.999, scene.near, scene.far,
                            "gaussian", 0.95, timer=mark)
        _, code = l1_loss_forward(out[0], target)
        grad_image = l1_loss_backward(code, torch.ones((), device=device))
        mark("loss")
        backward_views(*params, rot, trans, intr, w, h, tile, 0.999, out[1:], grad_image,
                       timer=mark)
        torch.cuda.synchronize()
        if i:
            runs.append(stage_times())
    stages_ms = {k: statistics.median(r[k] for r in runs) for k in runs[0]}

    # Work figures: per-view processed pairs on the mosaic, row-list entries.
    ncon, ranges, gids = out[2], out[8], out[7]
    tw, th = -(-w // tile), -(-h // tile)
    cols = mosaic_columns(views, tw, th)
    rows_m = -(-views // cols)
    grid = ranges.view(rows_m * th, cols * tw, 2)
    fwd_pairs = bwd_pairs = rows = 0
    for v, cam in enumerate(cams):
        vx, vy = v % cols, v // cols
        r = grid[vy * th:(vy + 1) * th, vx * tw:(vx + 1) * tw].reshape(-1, 2)
        f, b = processed_pairs(r, ncon[v], tile, w, h)
        fwd_pairs += f
        bwd_pairs += b
        fx, fy = cam.focal_length
        cx, cy = cam.principal_point
        _, _, _, _, bounds, counts = project_and_count(
            *params, *host_extrinsics(cam), fx, fy, cx, cy, w, h,
            tile, scene.near, scene.far, "gaussian", 0.95)
        bb = bounds.view(-1, 4).long()
        rows += int(((bb[:, 3] - bb[:, 2]) * (counts > 0)).sum())
    model = views_stage_bytes(scene.num_points, scene.color.shape[1], views, int(gids.numel()),
                              rows, views * w * h, fwd_pairs, bwd_pairs)
    stages = stage_entries(stages_ms, model)
    # composite_bwd launches: one per step batched, one per camera in the loop.
    achieved = model["composite_bwd"] / (views if kind == "loop" else 1) / (dominant_ms * 1e-3) / 1e9
    other = "loop" if kind == "batched" else "batched"
    compared = {f"{other}_ms_per_step": round(timed[other][0], 4)} if other in timed else {}
    # The batched backward's measured counters (config 5 only): HBM traffic
    # per launch and VALU busy; the bound is VALU issue above 90% busy.
    traffic, valu = None, None
    counters = ROOT / "profiles" / "traffic_composite_bwd_config5.json"
    if counters.exists() and scene.name == "config5" and kind == "batched" and tile == 16:
        measured = json.loads(counters.read_text())
        traffic = measured["hbm_bytes_per_launch"]
        m = measured["valu"]
        insts = m["sq_insts_valu_per_launch"]
        issue_ms = insts * 4 / (1024 * VALU_CLOCK_HZ) * 1e3
        valu = {"valu_busy_measured": m["valu_busy"], "formula": m["formula"],
                "instructions": insts, "issue_ms_at_4_cycles": round(issue_ms, 4),
                "issue_frac": round(issue_ms / dominant_ms, 4)}
    bound = "valu" if valu is not None and valu["valu_busy_measured"] > 0.9 else "hbm"
    result = {
        "metric": "fwd+bwd Mpix/s, multi-view batch",
        "value": round(views * w * h / 1e6 / (ms_per_step * 1e-3), 3),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded scenes.CONFIGS distributions)",
        "config": {
            "workload": (f"{scene.name}: {scene.num_points} Gaussians, "
                         f"SH{math.isqrt(scene.color.shape[1]) - 1}, {views} views of "
                         f"{w}x{h}, fwd+bwd, L1 loss"),
            "tile_size": tile,
            "path": "rasterize_views (one mosaic)" if kind == "batched" else "rasterize per view",
            "intersections": int(gids.numel()),
        },
        **compared,
        "stages": stages,
        "roofline": {
            "kernel": "composite_bwd_kernel",
            "bound": bound,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "launch_ms": round(dominant_ms, 4),
            "valu_issue": valu,
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        # Views are independent on the CPU path (the reference renders one
        # camera per call): time CPU_VIEWS of them, each on its own sample,
        # and scale their mean time to all views.
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        picked = list(range(0, views, max(1, views // CPU_VIEWS)))[:CPU_VIEWS]
        per_view = [cpu_baseline(scene, tile, max(8, args.cpu_tiles // len(picked)), cam=cams[v],
                                 target=scene.target[v], with_config1=(i == 0))
                    for i, v in enumerate(picked)]
        seconds = sum(p["s_per_view"] for p in per_view) / len(per_view) * views
        cpu = dict(per_view[0])
        cpu.update({
            "value": views * w * h / 1e6 / seconds,
            "s_per_step": round(seconds, 1),
            "sample": (f"views {picked} of {views}, each: " + per_view[0]["sample"]
                       + f"; the views' mean time scaled to all {views} views: "
                       f"{seconds:.1f}s per step"),
            "views_timed": [{"view": v, "s": p["s_per_view"]} for v, p in zip(picked, per_view)],
        })
        cpu.pop("s_per_view", None)
        result["cpu_baseline"] = cpu
    line = json.dumps(result)
    print(line, flush=True)
    if args.out:
        Path(args.out).write_text(line + "\n")


# Hyper-parameters of the reference's training step (train.py:76-87, 115).
LAMBDA_DSSIM, OPACITY_REG, SCALE_REG = 0.2, 1e-2, 1e-2
LRS = {"mean": 1.6e-4, "rotation": 1e-3, "scale": 5e-3, "opacity": 5e-2, "color": 2.5e-3}


def train_step_fused(splats, cam, target, tile_size, near, far, optimizer):
    from gaussian_splats_hip.splats import rasterize
    from gaussian_splats_hip.training import l1_loss, splat_regularizers, ssim

    image = rasterize(splats, cam, tile_size=tile_size, near=near, far=far)
    l1 = l1_loss(image, target, clamp=True)
    dssim = 1 - ssim(image.clamp(0, 1), target)
    regs = splat_regularizers(splats.opacity, splats.scale)
    loss = (1 - LAMBDA_DSSIM) * l1 + LAMBDA_DSSIM * dssim + OPACITY_REG * regs[0] + SCALE_REG * regs[1]
    loss.backward()
    optimizer.step()
    optimizer.zero_grad()
    return loss


def train_step_torch(splats, cam, target, tile_size, near, far, optimizer, window):
    """The same step with torch ops for everything but the rasterizer: torch's
    L1, SSIM by conv2d (the formulation torchmetrics uses), regularisers and
    torch.optim.Adam."""
    import torch.nn.functional as F

    from gaussian_splats_hip.splats import rasterize

    image = rasterize(splats, cam, tile_size=tile_size, near=near, far=far).clamp(0, 1)
    l1 = (image - target).abs().mean()
    x = image.permute(2, 0, 1)[None]
    y = target.permute(2, 0, 1)[None]
    p, q = F.pad(x, (5, 5, 5, 5), mode="reflect"), F.pad(y, (5, 5, 5, 5), mode="reflect")
    out = F.conv2d(torch.cat((p, q, p * p, q * q, p * q)), window, groups=3)
    mx, my, exx, eyy, exy = out.split(1)
    sxx, syy = torch.clamp(exx - mx * mx, min=0.0), torch.clamp(eyy - my * my, min=0.0)
    s = ((2 * mx * my + 1e-4) * (2 * (exy - mx * my) + 9e-4)) / (
        (mx * mx + my * my + 1e-4) * (sxx + syy + 9e-4))
    dssim = 1 - s[..., 5:-5, 5:-5].mean()
    loss = ((1 - LAMBDA_DSSIM) * l1 + LAMBDA_DSSIM * dssim
            + OPACITY_REG * splats.opacity.sigmoid().mean() + SCALE_REG * splats.scale.exp().mean())
    loss.backward()
    optimizer.step()
    optimizer.zero_grad()
    return loss


def bench_train_step(args):
    """One JSON line: the reference's training step (config 3) per second with
    the fused kernels, and the same step with torch ops for the loss terms and
    the optimiser."""
    from gaussian_splats_hip import scenes
    from gaussian_splats_hip.kernels.rasterize import _native
    from gaussian_splats_hip.splats import GaussianSplat
    from gaussian_splats_hip.training import FusedAdam

    _native.library()
    device = torch.device("cuda:0")
    scene = scenes.CONFIGS[args.config]()
    cam = scene.cameras[0]
    w, h = cam.image_size
    if scene.target is None:
        target = torch.rand(h, w, 3, device=device)
    else:
        target = (scene.target[0] if scene.target.dim() == 4 else scene.target).to(device)
    g = torch.exp(-((torch.arange(11, dtype=torch.float32) - 5) / 1.5) ** 2 / 2)
    g = (g / g.sum()).to(device)
    window = (g[:, None] @ g[None, :]).expand(3, 1, 11, 11).contiguous()
    results = {}
    for kind in ("fused", "torch"):
        splats = GaussianSplat.from_tensors(*(p.to(device) for p in scene.params()))
        groups = [{"params": [getattr(splats, k)], "lr": lr, "name": k} for k, lr in LRS.items()]
        opt = FusedAdam(groups, eps=1e-15) if kind == "fused" else torch.optim.Adam(groups, eps=1e-15)

        def step():
            if kind == "fused":
                return train_step_fused(splats, cam, target, args.tile_size, scene.near, scene.far, opt)
            return train_step_torch(splats, cam, target, args.tile_size, scene.near, scene.far, opt,
                                    window)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        results[kind] = 1e3 * (time.perf_counter() - t0) / args.steps
        print(f"[bench] train step ({kind}): {results[kind]:.3f} ms", file=sys.stderr, flush=True)
    result = {
        "metric": "training steps/s at 1M Gaussians SH3 1080p (rasterize + L1 + D-SSIM + "
                  "regularisers + backward + Adam)",
        "value": round(1e3 / results["fused"], 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(results["fused"], 4),
        "higher_is_better": True,
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded scenes.CONFIGS distributions)",
        "config": {"workload": f"{scene.name}: training step of train.py:136-152",
                   "tile_size": args.tile_size},
        "torch_ops_ms_per_step": round(results["torch"], 4),
    }
    line = json.dumps(result)
    print(line, flush=True)
    if args.out:
        Path(args.out).write_text(line + "\n")


def bench_ply_io(args):
    """Scene-file I/O of the config's Gaussians (config 3: 1M SH3, a 248 MB
    file in the page cache): save_ply of GPU tensors (records packed on the
    GPU, one download) and load_ply(device=...) (one upload, records split on
    the GPU), each beside the host path (numpy records, per-tensor copies)."""
    import tempfile

    from gaussian_splats_hip import scenes
    from gaussian_splats_hip.kernels.rasterize import _native
    from gaussian_splats_hip.splats.ply import load_ply, save_ply

    _native.library()
    device = torch.device("cuda:0")
    scene = scenes.CONFIGS[args.config]()
    names = ("mean", "rotation", "scale", "opacity", "color")
    host_state = dict(zip(names, (p.contiguous() for p in scene.params())))
    dev_state = {k: v.to(device) for k, v in host_state.items()}
    n, k = scene.num_points, scene.color.shape[1]
    record_bytes = 4 * (14 + 3 * k)
    reps = max(1, args.steps)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return 1e3 * (time.perf_counter() - t0) / reps

    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "scene.ply"
        save_host = timed(lambda: save_ply(host_state, path))
        with _native.LaunchTimer("ply_pack", capacity=reps + 2) as pack_timer:
            save_dev = timed(lambda: save_ply(dev_state, path))
        file_bytes = path.stat().st_size

        def load_host():
            return {key: v.to(device) for key, v in load_ply(path).items()}

        load_host_ms = timed(load_host)
        with _native.LaunchTimer("ply_unpack", capacity=reps + 2) as unpack_timer:
            load_dev_ms = timed(lambda: load_ply(path, device=device))
        loaded = load_ply(path, device=device)
        for key in names:
            assert torch.equal(loaded[key], dev_state[key]), key
    unpack_ms, pack_ms = unpack_timer.mean_ms(), pack_timer.mean_ms()
    kernel_bytes = 2 * n * record_bytes  # records in, parameters out (or the reverse)
    line = {
        "metric": "scene file I/O GB/s (PLY, page cache)", "unit": "GB/s", "n_gpus": 1,
        "config": {"workload": f"{scene.name}: {n} Gaussians, SH {k} coefficients, "
                               f"{file_bytes / 1e6:.0f} MB file"},
        "load_to_hbm": {"gpu_split_ms": round(load_dev_ms, 2), "host_path_ms": round(load_host_ms, 2),
                        "GB/s": round(file_bytes / load_dev_ms / 1e6, 2)},
        "save_from_hbm": {"gpu_pack_ms": round(save_dev, 2), "host_path_ms": round(save_host, 2),
                          "GB/s": round(file_bytes / save_dev / 1e6, 2)},
        "kernels": {
            "ply_unpack": {"ms": round(unpack_ms, 4),
                           "GB/s": round(kernel_bytes / unpack_ms / 1e6, 1),
                           "frac_hbm": round(kernel_bytes / unpack_ms / 1e6 / HBM_PEAK_GBS, 4)},
            "ply_pack": {"ms": round(pack_ms, 4),
                         "GB/s": round(kernel_bytes / pack_ms / 1e6, 1),
                         "frac_hbm": round(kernel_bytes / pack_ms / 1e6 / HBM_PEAK_GBS, 4)},
        },
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the rasterizer runs on a single device; sharding by view or by screen band is "
              "not built)",
              file=sys.stderr)
        sys.exit(2)
    if args.train_step:
        bench_train_step(args)
        return
    if args.ply_io:
        bench_ply_io(args)
        return
    from gaussian_splats_hip import scenes
    from gaussian_splats_hip.kernels.rasterize import _native
    from gaussian_splats_hip.splats import GaussianSplat

    _native.library()
    device = torch.device("cuda:0")
    scene = scenes.from_file(args.scene) if args.scene else scenes.CONFIGS[args.config]()
    if len(scene.cameras) > 1:
        bench_views(args, scene)
        return
    cam = scene.cameras[0]
    w, h = cam.image_size
    splats = GaussianSplat.from_tensors(*(p.to(device) for p in scene.params()))
    if scene.target is None:
        target = torch.rand(h, w, 3, device=device)
    else:  # multi-view scenes hold one target per camera; the step renders view 0
        target = (scene.target[0] if scene.target.dim() == 4 else scene.target).to(device)
    params = [splats.mean.detach(), splats.rotation.detach(), splats.scale.detach(),
              splats.opacity.detach(), splats.color.detach()]

    backward = not args.forward_only
    print(f"[bench] {scene.name}: N={scene.num_points} {w}x{h} tile={args.tile_size}"
          f"{'' if backward else ' forward only'}", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        for p in splats.parameters():
            p.grad = None
        run_step(splats, cam, target, args.tile_size, scene.near, scene.far, backward)
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    # The dominant kernel, timed per launch with HIP events that its launch
    # carries (the kernel's own start and end timestamps, no marker packets
    # on the stream): the compositing backward, or the forward compositing
    # for a forward step.
    dominant = "composite_bwd" if backward else "composite"
    with _native.LaunchTimer(dominant, capacity=args.steps + 1) as timer:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            for p in splats.parameters():
                p.grad = None
            run_step(splats, cam, target, args.tile_size, scene.near, scene.far, backward)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    ms_per_step = 1e3 * elapsed / args.steps
    mpix = (w * h) / 1e6
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step", file=sys.stderr, flush=True)
    # The other kernels' per-launch times, the same way, from as many further
    # steps outside the timed region.
    with _native.LaunchTimer("project", capacity=args.steps + 1) as project_timer, \
            _native.LaunchTimer("project_bwd", capacity=args.steps + 1) as project_bwd_timer:
        for _ in range(args.steps):
            for p in splats.parameters():
                p.grad = None
            run_step(splats, cam, target, args.tile_size, scene.near, scene.far, backward)
        torch.cuda.synchronize()

    # Per-stage event timing: the median of five staged steps after one
    # untimed one (the stage functions allocate their own buffers, and a first
    # allocation of a size inside a stage would put its host wait in that
    # stage's time).
    stage_runs = []
    for i in range(6):
        ms, info = staged_step(params, cam, target, args.tile_size, scene.near, scene.far,
                               backward)
        if i:
            stage_runs.append(ms)
    stages_ms = {k: statistics.median(r[k] for r in stage_runs) for k in stage_runs[0]}
    print("[bench] staged runs (ms): " + "; ".join(
        ", ".join(f"{k} {v:.3f}" for k, v in r.items()) for r in stage_runs),
        file=sys.stderr, flush=True)
    fwd_pairs, bwd_pairs = processed_pairs(info["ranges"], info["ncon"], args.tile_size, w, h)
    bytes_model = stage_bytes(scene.num_points, scene.color.shape[1], info["total"], info["rows"],
                              w * h, fwd_pairs, bwd_pairs)
    stages = stage_entries(stages_ms, bytes_model)

    # Dominant kernel, timed per launch with the HIP events its launches
    # carried during the timed steps.
    dominant_ms = timer.mean_ms()
    achieved = bytes_model[dominant] / (dominant_ms * 1e-3) / 1e9
    traffic = None
    valu = None
    traffic_file = ROOT / "profiles" / "traffic_composite_bwd_config3.json"
    if (traffic_file.exists() and args.config == "config3" and args.tile_size == 16
            and backward and not args.scene):
        measured = json.loads(traffic_file.read_text())
        traffic = measured["hbm_bytes_per_launch"]
        if "valu" in measured:
            # The kernel's real bound is VALU issue: measured VALU busy (the
            # share of SIMD cycles issuing VALU work, transcendental
            # instructions included), and the issue time of its wave64 fp32
            # VALU instructions at 4 cycles each on the 1024 SIMDs (256 CUs x
            # 4) at 2.4 GHz, against the measured launch time.
            m = measured["valu"]
            insts = m["sq_insts_valu_per_launch"]
            issue_ms = insts * 4 / (1024 * VALU_CLOCK_HZ) * 1e3
            valu = {"valu_busy_measured": m["valu_busy"], "formula": m["formula"],
                    "instructions": insts, "issue_ms_at_4_cycles": round(issue_ms, 4),
                    "issue_frac": round(issue_ms / dominant_ms, 4)}
    # The bound is the resource the kernel saturates: VALU issue when its
    # measured VALU busy exceeds 90%, else HBM; frac stays the HBM fraction.
    bound = "valu" if valu is not None and valu["valu_busy_measured"] > 0.9 else "hbm"
    kernel = "composite_bwd_kernel" if backward else "composite_fwd_kernel"
    roofline = {
        "kernel": f"{kernel}<{args.tile_size}>",
        "bound": bound,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "launch_ms": round(dominant_ms, 4),
        "algorithmic_bytes": bytes_model[dominant],
        "valu_issue": valu,
    }

    # The HBM-bound kernels, timed per launch the same way: algorithmic bytes
    # of the projection (parameters in, 104 B of outputs per Gaussian out)
    # and of its backward (parameters and dL/d projected in, gradients out).
    kernels = {}
    for name, t, nbytes in (("project_fwd_kernel", project_timer, bytes_model["project"]),
                            ("project_bwd_kernel", project_bwd_timer, bytes_model["project_bwd"])):
        ms = t.mean_ms()
        if ms > 0:
            gbs = nbytes / (ms * 1e-3) / 1e9
            kernels[name] = {"launch_ms": round(ms, 4), "algorithmic_bytes": nbytes,
                             "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(scene, args.tile_size, args.cpu_tiles, target=target.cpu(),
                           backward=backward)

    result = {
        "metric": ("fwd+bwd Mpix/s at 1M Gaussians SH3 1080p" if backward
                   else "fwd Mpix/s (forward-only workload)"),
        "value": round(mpix / (ms_per_step * 1e-3), 3),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded scenes.CONFIGS distributions)",
        "config": {
            "workload": (f"{scene.name}: {scene.num_points} Gaussians, "
                         f"SH{math.isqrt(scene.color.shape[1]) - 1}, {w}x{h}, "
                         + ("fwd+bwd, L1 loss" if backward else "forward")),
            "tile_size": args.tile_size,
            "intersections": info["total"],
        },
        "stages": stages,
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    line = json.dumps(result)
    print(line, flush=True)
    if args.out:
        Path(args.out).write_text(line + "\n")


if __name__ == "__main__":
    main()
