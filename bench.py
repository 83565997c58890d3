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
# Spin before the projection's start event (about 100 us at the engine clock),
# so its per-launch time excludes the host's launch latency after the idle
# gap at the start of a step.
PROJECT_HOLD_CYCLES = 250_000
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
        # params in (44 + 12k B) -> projected outputs, record, bounds, count, key (116 B)
        "project": n * (44 + 12 * k) + 116 * n,
        # depth sort: histogram + 4 passes of (key, id) in and out; rectangles
        # for the tables; row-list offset scan (order, key, gathered rectangle)
        "bin": 4 * n + 4 * 16 * n + 20 * n + 28 * n,
        # pass A writes (id, packed columns) per row entry; the width scan
        # reads and writes them; pass B reads its windows and writes one id
        # per intersection
        "emit": 8 * rows + 8 * rows + 8 * rows + 4 * total,
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
    "emit": ["sweep::clear_kernel", "row_bucket_kernel", "sweep::tile_sum_kernel<WidthLoad>",
             "sweep::tile_offsets_kernel", "sweep::scan_kernel<WidthLoad>", "column_count_kernel",
             "column_scan_kernel", "column_bucket_kernel"],
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


def run_step(splats, cam, target, tile_size, near, far):
    from gaussian_splats_hip.splats import rasterize
    from gaussian_splats_hip.training import l1_loss

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


def staged_step(params, cam, target, tile_size, near, far):
    """One fwd+bwd through the stage functions with timing events around each
    stage (stage_marker)."""
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
                           "gaussian", 0.95, timer=mark)
    image, final_t, ncon, pmean, pinv, pcol, pop, gids, ranges, counts = out
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
            orc.rasterize(*scene.params(), ocam, tile_size=16, near=scene.near, far=scene.far)
            if i > 0:
                times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    return {"value": round((w * h) / 1e6 / med, 4), "unit": "Mpix/s", "s_per_frame": round(med, 4),
            "frames": "warm-up 1, median of 3", "workload": f"config1 forward, {w}x{h}, "
            f"{scene.num_points} Gaussians, SH0, tile 16"}


def cpu_baseline(scene, tile_size, sample_tiles):
    """The CPU oracle (torch-CPU restatement of the reference torch backend) on a
    bounded sample: full projection + binning of all Gaussians, then dense
    fwd+bwd compositing of ``sample_tiles`` non-empty tiles, stratified by list
    length (equal numbers of tiles from each eighth of the non-empty tiles
    sorted by length, seeded), each stratum timed on its own and its time per
    tile scaled by the stratum's tile count.  Also: config 1 whole, and the
    host's CPU and memory."""
    import numpy as np

    from oracle import rasterizer as orc

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cam = scene.cameras[0]
    fx, fy = cam.focal_length
    cx, cy = cam.principal_point
    w, h = cam.image_size
    ocam = orc.Camera(*host_extrinsics(cam), fx, fy, cx, cy, w, h)
    params = [p.detach().clone().requires_grad_(True) for p in scene.params()]
    t0 = time.perf_counter()
    proj = orc.project(*params, ocam)
    tw, th = -(-w // tile_size), -(-h // tile_size)
    bounds, counts = orc.tile_counts(proj, tile_size, tw, th, scene.near, scene.far)
    keys, ids = orc.emit_intersections(bounds, proj.mean[:, 2].detach().numpy(), counts, tw)
    sid, ranges, _ = orc.sort_intersections(keys, ids, tw * th)
    t1 = time.perf_counter()
    # Compositing runs on detached copies of the projected tensors, so each
    # stratum back-propagates only through its own compositing; the
    # projection's backward runs once at the end on the summed gradients.
    leaves = [t.detach().requires_grad_(True)
              for t in (proj.mean, proj.inverse, proj.color, proj.opacity)]
    pm, pinv, pcol, pop = leaves
    rng = np.random.default_rng(0)
    nonempty = np.nonzero(ranges[:, 1] > ranges[:, 0])[0]
    lengths = ranges[nonempty, 1] - ranges[nonempty, 0]
    by_length = nonempty[np.argsort(lengths, kind="stable")]
    strata = np.array_split(by_length, 8)
    per = max(1, sample_tiles // len(strata))

    def mask_of(tiles):
        mask = torch.zeros(th * tile_size, tw * tile_size)
        for t in tiles:
            ty, tx = divmod(int(t), tw)
            mask[ty * tile_size:(ty + 1) * tile_size, tx * tile_size:(tx + 1) * tile_size] = 1
        return mask[:h, :w, None]

    # The per-call cost that does not scale with the tiles (image-sized
    # buffers, the chunk loop, the loss): one call with every list empty; it
    # is taken off each stratum's time before scaling and counted once.
    empty = ranges.copy()
    empty[:, 1] = empty[:, 0]
    te0 = time.perf_counter()
    with torch.no_grad():
        comp = orc.composite(pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1],
                             pcol, pop[:, 0], sid, empty, w, h, tile_size, tile_chunk=8)
        ((comp.image - scene.target).abs() * mask_of([])).sum()
    fixed_s = time.perf_counter() - te0
    composite_s = fixed_s
    sampled_tiles = 0
    for stratum in strata:
        if len(stratum) == 0:
            continue
        chosen = rng.choice(stratum, size=min(per, len(stratum)), replace=False)
        keep = np.zeros(tw * th, dtype=bool)
        keep[chosen] = True
        sampled = ranges.copy()
        sampled[~keep] = sampled[~keep, :1]  # empty the other tiles
        ts0 = time.perf_counter()
        comp = orc.composite(pm[:, 0], pm[:, 1], pinv[:, 0, 0], pinv[:, 0, 1], pinv[:, 1, 1],
                             pcol, pop[:, 0], sid, sampled, w, h, tile_size, tile_chunk=8)
        loss = ((comp.image - scene.target).abs() * mask_of(chosen)).sum() / (w * h * 3)
        loss.backward()
        dt = max(time.perf_counter() - ts0 - fixed_s, 0.0)
        composite_s += dt / len(chosen) * len(stratum)
        sampled_tiles += len(chosen)
    t2 = time.perf_counter()
    outs = [(o, l.grad) for o, l in zip((proj.mean, proj.inverse, proj.color, proj.opacity), leaves)
            if l.grad is not None and o.requires_grad]
    torch.autograd.backward([o for o, _ in outs], [g for _, g in outs])
    t3 = time.perf_counter()
    full_s = (t1 - t0) + composite_s + (t3 - t2)
    return {
        "value": (w * h) / 1e6 / full_s,
        "unit": "Mpix/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"torch-CPU oracle, float32: projection+binning of all {scene.num_points} Gaussians "
            f"({t1 - t0:.1f}s) + dense fwd+bwd compositing of {sampled_tiles} non-empty "
            f"{tile_size}px tiles, {per} from each eighth of the tiles by list length "
            f"({t2 - t1:.1f}s), each eighth's time per tile (less the {fixed_s:.2f}s per call "
            f"that does not scale with the tiles, counted once) scaled to its "
            f"{len(nonempty) // 8}-odd tiles + the projection backward ({t3 - t2:.1f}s); "
            f"estimate {full_s:.1f}s per step"
        ),
        "host": host_description(),
        "config1_full": cpu_config1_full(threads),
    }


def views_stage_bytes(n, k, views, total, rows, pixels, processed_fwd, processed_bwd):
    """Algorithmic HBM bytes per stage of the multi-view step: the projection
    reads the parameters once per launch of up to 16 cameras and writes the
    116 B of outputs per (view, Gaussian); the backward reads the parameters
    once, 40 B per (view, Gaussian) and writes the gradients once."""
    launches = -(-views // 16)
    single = stage_bytes(views * n, k, total, rows, pixels, processed_fwd, processed_bwd)
    single["project"] = launches * n * (44 + 12 * k) + 116 * views * n
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

    # Per-stage events over the batched path.
    rot, trans, intr, _, _ = camera_tensors(cams)
    runs = []
    for _ in range(3):
        mark, stage_times = stage_marker()
        out = forward_views(*params, rot, trans, intr, w, h, tile, 0.999, scene.near, scene.far,
                            "gaussian", 0.95, timer=mark)
        _, code = l1_loss_forward(out[0], target)
        grad_image = l1_loss_backward(code, torch.ones((), device=device))
        mark("loss")
        backward_views(*params, rot, trans, intr, w, h, tile, 0.999, out[1:], grad_image,
                       timer=mark)
        torch.cuda.synchronize()
        runs.append(stage_times())
    stages_ms = {k: sum(r[k] for r in runs) / len(runs) for k in runs[0]}

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
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "launch_ms": round(dominant_ms, 4),
        },
        "cpu_baseline": None,
    }
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

    print(f"[bench] {scene.name}: N={scene.num_points} {w}x{h} tile={args.tile_size}", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        for p in splats.parameters():
            p.grad = None
        run_step(splats, cam, target, args.tile_size, scene.near, scene.far)
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    torch.cuda.synchronize()
    with _native.LaunchTimer("composite_bwd", capacity=args.steps + 1) as timer:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            for p in splats.parameters():
                p.grad = None
            run_step(splats, cam, target, args.tile_size, scene.near, scene.far)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    ms_per_step = 1e3 * elapsed / args.steps
    mpix = (w * h) / 1e6
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step", file=sys.stderr, flush=True)
    # The other kernels' per-launch times, from as many further steps outside
    # the timed region (their timing events would add to the step time).
    with _native.LaunchTimer("project", capacity=args.steps + 1,
                             hold_cycles=PROJECT_HOLD_CYCLES) as project_timer, \
            _native.LaunchTimer("project_bwd", capacity=args.steps + 1) as project_bwd_timer:
        for _ in range(args.steps):
            for p in splats.parameters():
                p.grad = None
            run_step(splats, cam, target, args.tile_size, scene.near, scene.far)
        torch.cuda.synchronize()

    # Per-stage event timing (averaged over a few staged steps).
    stage_runs = []
    for _ in range(3):
        ms, info = staged_step(params, cam, target, args.tile_size, scene.near, scene.far)
        stage_runs.append(ms)
    stages_ms = {k: sum(r[k] for r in stage_runs) / len(stage_runs) for k in stage_runs[0]}
    fwd_pairs, bwd_pairs = processed_pairs(info["ranges"], info["ncon"], args.tile_size, w, h)
    bytes_model = stage_bytes(scene.num_points, scene.color.shape[1], info["total"], info["rows"],
                              w * h, fwd_pairs, bwd_pairs)
    stages = stage_entries(stages_ms, bytes_model)

    # Dominant kernel: composite_bwd_kernel, timed per launch with HIP events
    # on its stream during the timed steps.
    dominant_ms = timer.mean_ms()
    achieved = bytes_model["composite_bwd"] / (dominant_ms * 1e-3) / 1e9
    traffic = None
    valu = None
    traffic_file = ROOT / "profiles" / "traffic_composite_bwd_config3.json"
    if traffic_file.exists() and args.config == "config3" and args.tile_size == 16:
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
    roofline = {
        "kernel": "composite_bwd_kernel<16>" if args.tile_size == 16 else "composite_bwd_kernel",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "launch_ms": round(dominant_ms, 4),
        "algorithmic_bytes": bytes_model["composite_bwd"],
        "valu_issue": valu,
    }

    # The HBM-bound kernels, timed per launch the same way: algorithmic bytes
    # of the projection (parameters in, 116 B of outputs per Gaussian out)
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
        cpu = cpu_baseline(scene, args.tile_size, args.cpu_tiles)

    result = {
        "metric": "fwd+bwd Mpix/s at 1M Gaussians SH3 1080p",
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
                         f"SH{math.isqrt(scene.color.shape[1]) - 1}, {w}x{h}, fwd+bwd, L1 loss"),
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
