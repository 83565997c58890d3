"""End-to-end rasterizer benchmark over a camera trajectory (reference:
src/gaussian_splats/kernels/rasterize/benchmark.py:1-253).

The scene (a seeded random scene, or a checkpoint / PLY file subsampled to
``num_splats``) is viewed by ``frames`` cameras orbiting it with a fixed
downward pitch.  Two measurements, per backend:

* first frame: forward (no grad) and forward + backward of
  ``image.square().mean()``, timed by ``do_bench``;
* trajectory: wall-clock milliseconds to render every frame.

Backends: ``hip`` (``rasterize``), ``hip_compiled`` (``torch.compile(rasterize,
dynamic=True)``: the custom op runs opaque inside the compiled graph, as the
viewer's compile path uses it) and, for the trajectory, ``hip_views``: the
frames rendered ``views_per_call`` at a time as one mosaic by
``rasterize_views`` (tile 16; images are tile-size independent).  The reference
compared its torch and Triton backends; neither is part of this build.  Frames
of the other backends are compared with ``hip``'s; GIFs of the frames and of
10x their difference, and ``measurements.json``, are written to a timestamped
directory.  ``python -m gaussian_splats_hip.kernels.rasterize.benchmark --help``.
"""

from __future__ import annotations

import json
import math
import time
from datetime import datetime, timezone
from pathlib import Path
from typing import Annotated, Callable, Optional

import torch
import typer

from ...splats.camera import PinholeCamera
from ...splats.splats import GaussianSplat
from .interface import rasterize
from .views import rasterize_views

app = typer.Typer(add_completion=False)


def random_scene(num_splats: int, seed: int, device: str | torch.device = "cuda") -> GaussianSplat:
    """SH-1 Gaussians in a slab 2-6 units in front of the origin (benchmark.py:26-34)."""
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        splats = GaussianSplat(num_splats, sh_degree=1)
        with torch.no_grad():
            splats.mean[:, :2].normal_(std=0.5)
            splats.mean[:, 2].uniform_(2.0, 6.0)
            splats.scale.fill_(-2.0)
    return splats.to(device)


def select_splats(splats: GaussianSplat, num_splats: int | None, seed: int) -> GaussianSplat:
    """A seeded random subset of ``num_splats`` Gaussians (benchmark.py:37-55)."""
    if num_splats is None or num_splats >= splats.num_points:
        return splats
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        indices = torch.randperm(splats.num_points)[:num_splats]
    selected = GaussianSplat(num_splats, sh_degree=splats.sh_degree).to(splats.mean.device)
    indices = indices.to(splats.mean.device)
    with torch.no_grad():
        for name in ("mean", "rotation", "scale", "opacity", "color", "normals"):
            getattr(selected, name).copy_(getattr(splats, name)[indices])
    return selected


def generate_trajectory(
    splats: GaussianSplat, image_size: tuple[int, int], num_frames: int
) -> list[PinholeCamera]:
    """Cameras orbiting the y axis (frame f at 360 f / num_frames degrees)
    then pitched by a fixed 45 degrees about x (world-to-camera R_x R_y), each
    fitted to the scene's points (benchmark.py:58-90)."""
    width, height = image_size
    half_elevation = math.radians(45) / 2
    cos_e, sin_e = math.cos(half_elevation), math.sin(half_elevation)
    cameras = []
    for frame in range(num_frames):
        half_angle = math.pi * frame / num_frames
        cos_a, sin_a = math.cos(half_angle), math.sin(half_angle)
        # q_x(-elevation) * q_y(angle) as a (w, x, y, z) product.
        rotation = splats.mean.new_tensor(
            [cos_a * cos_e, -cos_a * sin_e, sin_a * cos_e, -sin_a * sin_e]
        )
        camera = PinholeCamera(
            image_size=image_size,
            focal_length=(0.75 * width, 0.75 * width),
            principal_point=(0.5 * width, 0.5 * height),
            rotation=rotation,
        )
        cameras.append(camera.fit_to_points(splats.mean.detach()))
    return cameras


def do_bench(
    fn: Callable[[], object],
    warmup: float = 25.0,
    rep: float = 100.0,
    grad_to_none: list[torch.Tensor] | None = None,
) -> float:
    """Mean milliseconds per call of ``fn``: the call is timed once, then run
    for about ``warmup`` ms untimed and ``rep`` ms timed (at least once each),
    each call bracketed by events on the current stream after the L2 cache is
    overwritten (a 512 MiB fill) and the listed gradients are cleared."""
    flush = torch.empty(128 << 20, dtype=torch.int32, device="cuda")

    def clear_grads():
        for t in grad_to_none or ():
            t.grad = None

    clear_grads()
    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(3):
        clear_grads()
        fn()
    end.record()
    end.synchronize()
    estimate = max(start.elapsed_time(end) / 3, 1e-3)
    for _ in range(max(1, int(warmup / estimate))):
        clear_grads()
        fn()
    times = []
    for _ in range(max(1, int(rep / estimate))):
        clear_grads()
        flush.zero_()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        times.append((s, e))
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in times) / len(times)


def _render_views(splats, cameras, views_per_call: int) -> list[torch.Tensor]:
    frames = []
    for i in range(0, len(cameras), views_per_call):
        frames.extend(rasterize_views(splats, cameras[i:i + views_per_call], tile_size=16).unbind(0))
    return frames


def save_gif(frames: list[torch.Tensor], path: Path) -> None:
    from PIL import Image

    images = [
        Image.fromarray(frame.detach().clamp(0, 1).mul(255).byte().cpu().numpy(), "RGB")
        for frame in frames
    ]
    images[0].save(path, save_all=True, append_images=images[1:], duration=40, loop=0)


def run(
    *,
    checkpoint: str | Path | None,
    output_dir: str | Path,
    device: str | None,
    image_size: tuple[int, int],
    num_splats: int | None,
    frames: int,
    repeats: int,
    seed: int,
    views_per_call: int = 16,
    gifs: bool = True,
) -> dict:
    """Runs the benchmark and returns the measurements (also written to
    ``output_dir/<timestamp>/measurements.json``)."""
    assert torch.cuda.is_available(), "a ROCm GPU is required for benchmarking"
    device = torch.device(device or "cuda")
    output_root = Path(output_dir)
    run_id = datetime.now(timezone.utc).strftime("%Y%m%dT%H%M%S.%fZ")
    out = output_root / run_id
    out.mkdir(parents=True, exist_ok=False)
    typer.echo(f"Benchmarking to {out}")

    if checkpoint is None:
        splats = random_scene(num_splats or 10_000, seed, device)
    else:
        path = Path(checkpoint)
        if path.suffix.lower() == ".ply":
            from ...splats.ply import load_ply

            splats = GaussianSplat.from_tensors(**load_ply(path, device=device))
        else:
            splats = GaussianSplat.from_checkpoint(path).to(device)
        splats = select_splats(splats, num_splats, seed)

    trajectory = generate_trajectory(splats, image_size, frames)
    funcs = {"hip": rasterize, "hip_compiled": torch.compile(rasterize, dynamic=True)}
    params = list(splats.parameters())

    first = trajectory[0]
    bars: dict[str, dict[str, float]] = {}
    for backend, func in funcs.items():
        with torch.no_grad():
            forward = do_bench(lambda f=func: f(splats, first), warmup=2, rep=repeats)
        backward = do_bench(
            lambda f=func: f(splats, first).square().mean().backward(),
            warmup=2, rep=repeats, grad_to_none=params,
        )
        bars[backend] = {"forward": forward, "backward": backward}
        typer.echo(f"first frame {backend}: forward {forward:.3f} ms, forward+backward {backward:.3f} ms")

    renderers = {name: (lambda f=f: [f(splats, cam) for cam in trajectory]) for name, f in funcs.items()}
    renderers["hip_views"] = lambda: _render_views(splats, trajectory, views_per_call)
    records: dict[str, float] = {}
    rendered: dict[str, list[torch.Tensor]] = {}
    for backend, render in renderers.items():
        with torch.no_grad():
            render()  # compile / warm up
            torch.cuda.synchronize()
            start = time.perf_counter()
            rendered[backend] = render()
            torch.cuda.synchronize()
        records[backend] = (time.perf_counter() - start) * 1_000
        typer.echo(f"trajectory {backend}: {records[backend]:.2f} ms for {frames} frames")

    reference = rendered["hip"]
    differences = {
        backend: max(float((a - b).abs().max()) for a, b in zip(reference, frames_, strict=True))
        for backend, frames_ in rendered.items()
        if backend != "hip"
    }
    if gifs:
        save_gif(reference, out / "hip.gif")
        save_gif([(a - b).abs() * 10 for a, b in zip(reference, rendered["hip_views"])],
                 out / "absolute_difference.gif")
    measurements = {
        "first_frame": bars,
        "trajectory": records,
        "max_abs_difference_vs_hip": differences,
        "config": {"num_splats": splats.num_points, "image_size": list(image_size),
                   "frames": frames, "views_per_call": views_per_call},
    }
    (out / "measurements.json").write_text(json.dumps(measurements, indent=2))
    return measurements


@app.command()
def benchmark(
    checkpoint: Annotated[Optional[str], typer.Option(help="Scene checkpoint (.pt) or PLY path.")] = None,
    output: Annotated[str, typer.Option(help="Output directory.")] = "output/rasterize-benchmark",
    device: Annotated[Optional[str], typer.Option(help="Torch device (default cuda).")] = None,
    width: Annotated[int, typer.Option(min=8)] = 640,
    height: Annotated[int, typer.Option(min=8)] = 480,
    num_splats: Annotated[Optional[int], typer.Option(min=1)] = None,
    frames: Annotated[
        int, typer.Option("--trajectory-frames", "--frames", min=2, help="Camera trajectory frames.")
    ] = 120,
    repeats: Annotated[int, typer.Option(min=1)] = 3,
    seed: Annotated[int, typer.Option()] = 42,
    views_per_call: Annotated[int, typer.Option(min=1, help="Frames per rasterize_views call.")] = 16,
) -> None:
    """Benchmark full rasterization over a continuous camera trajectory."""
    run(
        checkpoint=checkpoint, output_dir=output, device=device, image_size=(width, height),
        num_splats=num_splats, frames=frames, repeats=repeats, seed=seed,
        views_per_call=views_per_call,
    )


def main() -> None:
    app()


if __name__ == "__main__":
    app()
