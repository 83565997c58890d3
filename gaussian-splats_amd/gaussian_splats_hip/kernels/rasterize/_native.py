"""ctypes binding of the C-ABI library ``libgs_raster.so`` (include/gs_raster.h).

The library is built in-tree by ``gaussian-splats_amd/build.py``.  There is no
fallback: every stage raises if the library is missing or if it is handed
tensors that do not live on a ROCm GPU.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parents[2] / "_lib" / "libgs_raster.so"
ABI_VERSION = 17

GS_OK = 0
GS_ERR_INVALID_ARGUMENT = 1
GS_ERR_UNSUPPORTED = 2
GS_ERR_OVERFLOW = 3
GS_ERR_HIP = 4
GS_ERR_WORKSPACE = 5

MODES = {"gaussian": 0, "ellipsoid": 1}


class GsAdamTensor(ctypes.Structure):
    _fields_ = [
        ("param", c_void_p),
        ("grad", c_void_p),
        ("exp_avg", c_void_p),
        ("exp_avg_sq", c_void_p),
        ("numel", c_int64),
        ("lr", ctypes.c_double),
        ("step", c_int64),
    ]


ADAM_MAX_TENSORS = 8


class GsView(ctypes.Structure):
    _fields_ = [
        ("fx", c_float),
        ("fy", c_float),
        ("cx", c_float),
        ("cy", c_float),
        ("image_width", c_int32),
        ("image_height", c_int32),
        ("tile_size", c_int32),
        ("near_plane", c_float),
        ("far_plane", c_float),
        ("rendering_mode", c_int32),
        ("confidence", c_float),
        ("opacity_threshold", c_float),
        ("covariance_epsilon", c_float),
        ("views", c_int32),
        ("mosaic_cols", c_int32),
        ("active_tiles", c_int32),
    ]


def make_view(
    fx: float,
    fy: float,
    cx: float,
    cy: float,
    image_width: int,
    image_height: int,
    tile_size: int = 16,
    near: float = 0.2,
    far: float = 100.0,
    rendering_mode: str = "gaussian",
    confidence: float = 0.95,
    opacity_threshold: float = 0.999,
    covariance_epsilon: float = 0.03,
    views: int = 1,
    mosaic_cols: int = 1,
    active_tiles: int = 0,
) -> GsView:
    if rendering_mode not in MODES:
        raise ValueError(f"Invalid rendering mode: {rendering_mode}")
    return GsView(
        float(fx), float(fy), float(cx), float(cy), int(image_width), int(image_height),
        int(tile_size), float(near), float(far), MODES[rendering_mode], float(confidence),
        float(opacity_threshold), float(covariance_epsilon), int(views), int(mosaic_cols),
        int(active_tiles),
    )


_ACTIVE_ATTR = "_gs_active_tiles"


def set_active_tiles(ranges: torch.Tensor, count: int) -> None:
    """Records on ``ranges`` how many tiles have a non-empty list (binning
    reads it back with the totals); the compositing launches use it to pick
    their shape.  Only a hint: results do not depend on it."""
    setattr(ranges, _ACTIVE_ATTR, int(count))


def active_tiles(ranges: torch.Tensor | None) -> int:
    """The count recorded by ``set_active_tiles``, or 0 (unknown)."""
    return int(getattr(ranges, _ACTIVE_ATTR, 0)) if ranges is not None else 0


_LONGEST_ATTR = "_gs_longest_list"


def set_longest_list(ranges: torch.Tensor, length: int) -> None:
    """Records on ``ranges`` the longest list (binning returns it with its
    totals): the compositing walk records checkpoints only for long lists."""
    setattr(ranges, _LONGEST_ATTR, int(length))


def longest_list(ranges: torch.Tensor) -> int:
    """The length recorded by ``set_longest_list``, else read from the
    ranges (one device-to-host copy)."""
    value = getattr(ranges, _LONGEST_ATTR, None)
    if value is None:
        value = int((ranges[:, 1] - ranges[:, 0]).max().item()) if ranges.numel() else 0
    return int(value)


_WALK_ATTR = "_gs_walk_state"


def _stamp(t):
    """A tensor's identity as a kernel read it: storage address, in-place
    version counter, shape and dtype."""
    if t is None:
        return None
    return (t.data_ptr(), t._version, tuple(t.shape), t.dtype)


def walk_fingerprint(key: tuple, *tensors) -> tuple:
    """Fingerprint of one compositing walk: the view parameters in ``key``
    and the identity of every tensor the walk read or wrote.  gs_composite's
    checkpoints and hit masks are valid for a backward only when its
    arguments have the same fingerprint."""
    return (tuple(key),) + tuple(_stamp(t) for t in tensors)


def set_walk_state(n_contributors: torch.Tensor, fingerprint: tuple | None,
                   checkpoints: torch.Tensor | None, hits: torch.Tensor | None) -> None:
    """Records on the forward's own ``n_contributors`` output the checkpoint
    and hit-mask buffers gs_composite wrote, with the fingerprint of that
    call (``None`` for the op's outputs, which are consumed together)."""
    setattr(n_contributors, _WALK_ATTR, (fingerprint, checkpoints, hits))


def walk_buffers(n_contributors: torch.Tensor | None, fingerprint: tuple | None = None):
    """``(checkpoints, hit_masks)`` recorded with ``n_contributors``, or
    ``(None, None)``.  With a ``fingerprint``, only when it equals the one
    recorded: a backward whose arguments are not exactly the forward's
    (another projection, lists changed in place, another threshold) walks
    every entry from the list's end.  That keeps it a pure function of its
    arguments."""
    state = getattr(n_contributors, _WALK_ATTR, None) if n_contributors is not None else None
    if state is None:
        return None, None
    recorded, checkpoints, hits = state
    if fingerprint is not None and recorded != fingerprint:
        return None, None
    return checkpoints, hits


_FORWARD_BUFFERS_ATTR = "_gs_forward_buffers"


def set_forward_buffer(n_contributors: torch.Tensor, name: str, buffer: torch.Tensor) -> None:
    """Records on the forward's ``n_contributors`` a buffer the forward
    prepared for its backward: "grad_accumulator", the [N, 9] buffer the
    compositing backward accumulates into (zeroed by the binning's side
    stream), or "tile_keys", the backward's dispatch keys (gs_composite's
    tile_keys)."""
    buffers = getattr(n_contributors, _FORWARD_BUFFERS_ATTR, None)
    if buffers is None:
        buffers = {}
        setattr(n_contributors, _FORWARD_BUFFERS_ATTR, buffers)
    buffers[name] = buffer


def take_forward_buffer(n_contributors: torch.Tensor | None, name: str) -> torch.Tensor | None:
    """The buffer recorded under ``name`` with ``n_contributors``, once (a
    later call gets None and must make its own).  None while tracing
    (torch.compile), where the outputs are fake tensors."""
    if n_contributors is None or torch.compiler.is_compiling():
        return None
    buffers = getattr(n_contributors, _FORWARD_BUFFERS_ATTR, None)
    return buffers.pop(name, None) if buffers else None


def checkpoint_buffer(view: GsView, num_intersections: int, longest: int,
                      device: torch.device):
    """A checkpoint buffer for gs_composite (256-byte aligned), or None when
    the walk records none (no list long enough, or every tile split into
    quarters)."""
    nbytes = library().gs_composite_checkpoint_bytes(view, int(num_intersections), int(longest))
    if nbytes == 0:
        return None
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    off = (-buf.data_ptr()) % 256
    return buf[off:off + nbytes]


def hit_mask_buffer(view: GsView, num_intersections: int, device: torch.device) -> torch.Tensor:
    """A hit-mask buffer for gs_composite (int64 words; the forward writes the
    batches it walks, the backward reads the same ones)."""
    nbytes = library().gs_composite_hit_mask_bytes(view, int(num_intersections))
    return torch.empty(max(int(nbytes) // 8, 1), dtype=torch.int64, device=device)


def buffer_bytes(t: torch.Tensor | None) -> int:
    """Size in bytes of an optional buffer argument (0 for None)."""
    return t.numel() * t.element_size() if t is not None else 0


_SIGNATURES = {
    "gs_abi_version": (c_int, []),
    "gs_last_error": (ctypes.c_char_p, []),
    "gs_arm_launch_events": (c_int, [c_void_p, c_void_p]),
    "gs_disarm_launch_events": (c_int, []),
    "gs_project_and_count": (
        c_int,
        [c_void_p] * 5 + [c_int64, c_int32, c_void_p, c_void_p, GsView] + [c_void_p] * 10,
    ),
    "gs_project_views": (
        c_int,
        [c_void_p] * 5 + [c_int64, c_int32, c_void_p, c_void_p, c_void_p, GsView] + [c_void_p] * 10,
    ),
    "gs_pack_records": (c_int, [c_void_p] * 4 + [c_int64, GsView, c_void_p, c_void_p]),
    "gs_scan_workspace_bytes": (c_size_t, [c_int64]),
    "gs_scan_counts": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_size_t, c_void_p]),
    "gs_emit_intersections": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p, c_void_p],
    ),
    "gs_sort_workspace_bytes": (c_size_t, [c_int64, c_int32]),
    "gs_sort_intersections": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "gs_bin_workspace_bytes": (c_size_t, [c_int64]),
    "gs_bin_gaussians": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "gs_emit_tiles": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int32, c_void_p, c_void_p, c_void_p],
    ),
    "gs_sort_tiles": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "gs_bin_tiles_plan_bytes": (c_size_t, [c_int64, c_int32, c_int32]),
    "gs_bin_tiles_plan": (
        c_int,
        [c_void_p] * 2 + [c_int64, ctypes.c_uint32, c_int32, c_int32, c_int32] + [c_void_p] * 4
        + [c_size_t, c_void_p, c_size_t, c_void_p],
    ),
    "gs_pack_tile_rects": (
        c_int, [c_void_p, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p]
    ),
    "gs_bin_tiles_emit_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int64, c_int32, c_int32]),
    "gs_bin_tiles_emit": (
        c_int,
        [c_int64, c_int32, c_int32, c_void_p, c_int64, c_int64, c_int64,
         c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "gs_tile_order_workspace_bytes": (c_size_t, [c_int32]),
    "gs_tile_order_items": (c_int64, [GsView, c_int32]),
    "gs_tile_order": (
        c_int, [c_void_p, c_void_p, GsView, c_void_p, c_void_p, c_size_t, c_int32, c_void_p]
    ),
    "gs_tile_order_noalloc": (c_int, [c_void_p, c_void_p, GsView, c_void_p, c_void_p]),
    "gs_composite_checkpoint_bytes": (c_size_t, [GsView, c_int64, c_int64]),
    "gs_composite_hit_mask_bytes": (c_size_t, [GsView, c_int64]),
    "gs_composite": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, GsView]
        + [c_void_p] * 4 + [c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p],
    ),
    "gs_composite_bwd": (
        c_int,
        [c_void_p] * 4 + [c_int64] + [c_void_p] * 6
        + [GsView, c_void_p, c_void_p, c_void_p, c_size_t, c_int64, c_void_p, c_size_t, c_void_p],
    ),
    "gs_device_errors": (c_int, [c_void_p, c_int32, c_void_p]),
    "gs_project_bwd": (
        c_int,
        [c_void_p] * 5 + [c_int64, c_int32, c_void_p, c_void_p, GsView] + [c_void_p] * 9,
    ),
    "gs_project_bwd_views": (
        c_int,
        [c_void_p] * 5 + [c_int64, c_int32, c_void_p, c_void_p, c_void_p, GsView] + [c_void_p] * 9,
    ),
    "gs_l1_loss_workspace_bytes": (c_size_t, [c_int64]),
    "gs_l1_loss_fwd": (
        c_int,
        [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "gs_l1_loss_bwd": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "gs_splat_regularizers_workspace_bytes": (c_size_t, [c_int64]),
    "gs_splat_regularizers_fwd": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_size_t, c_void_p]
    ),
    "gs_splat_regularizers_bwd": (
        c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]
    ),
    "gs_adam_step": (
        c_int, [c_void_p, c_int32, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                ctypes.c_double, c_void_p]
    ),
    "gs_ssim_workspace_bytes": (c_size_t, [c_int32, c_int32]),
    "gs_ssim_fwd": (
        c_int, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_size_t, c_void_p]
    ),
    "gs_ssim_bwd": (
        c_int,
        [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p],
    ),
    "gs_ply_unpack": (
        c_int, [c_void_p, c_int64, c_int32, c_void_p, c_int32, c_int32] + [c_void_p] * 7
    ),
    "gs_ply_pack": (c_int, [c_void_p] * 6 + [c_int64, c_int32, c_void_p, c_void_p]),
}

PLY_MAX_FIELDS = 89

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """Loads (once) and returns the HIP rasterizer library."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"HIP rasterizer library not built ({LIB_PATH}); run "
                    "`python gaussian-splats_amd/build.py`"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if lib.gs_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"libgs_raster ABI {lib.gs_abi_version()} != expected {ABI_VERSION}"
                )
            _lib = lib
    return _lib


# Bits of the device's sticky check-failure word (GS_DEVICE_* in gs_raster.h).
DEVICE_FLAGS = {
    1: "a look-back wait of a sort or binning pass hit its spin limit",
    2: "a binning workgroup's owner window exceeded its tile",
    4: "sizes passed to a binning pass differ from the plan's device totals",
}


def raise_device_flags(flags: int, where: str) -> None:
    """Raises RuntimeError naming the failed device-side checks in ``flags``."""
    if flags:
        what = "; ".join(text for bit, text in DEVICE_FLAGS.items() if flags & bit) or "unknown"
        raise RuntimeError(
            f"{where}: a device-side check failed in a binning or sort call on this GPU "
            f"(flags {flags:#x}: {what}); the intersection lists of that call are incomplete"
        )


def device_errors(device: torch.device, clear: bool = True) -> int:
    """The device's sticky check-failure word after the work enqueued so far on
    its current stream (synchronises that stream); cleared when ``clear``."""
    flags = ctypes.c_uint32(0)
    check(library().gs_device_errors(ctypes.byref(flags), int(clear), stream(device)),
          "device_errors")
    return int(flags.value)


def check_device_errors(device: torch.device) -> None:
    """Raises if a device-side check has failed on ``device`` (and clears the
    word, so each failure is reported once)."""
    raise_device_flags(device_errors(device, clear=True), "device check")


def check(status: int, what: str) -> None:
    if status == GS_OK:
        return
    message = library().gs_last_error().decode(errors="replace")
    text = f"{what}: {message}"
    if status == GS_ERR_INVALID_ARGUMENT:
        raise ValueError(text)
    if status == GS_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)


def ptr(t: torch.Tensor | None) -> c_void_p:
    return c_void_p(0 if t is None else t.data_ptr())


def stream(device: torch.device) -> c_void_p:
    return c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must be on the same ROCm GPU; returns that device."""
    device = None
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(
                "the HIP rasterizer needs tensors on a ROCm GPU device "
                f"(got a tensor on {t.device})"
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    assert device is not None
    return device


def prepare(t: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Contiguous tensor of ``dtype`` whose data pointer is 16-byte aligned."""
    if t.dtype != dtype:
        raise TypeError(f"expected {dtype}, got {t.dtype}")
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


class LaunchTimer:
    """Times every launch of one entry point's main kernel while active
    (``with LaunchTimer("composite_bwd")``).  The launch carries the timing
    events (gs_arm_launch_events), so each pair holds the kernel's own start
    and end timestamps: no marker packet is queued on the stream, and the
    host's launch latency is not counted.  Used by the benchmark to measure a
    kernel's per-launch duration in place."""

    def __init__(self, name: str, capacity: int = 256):
        self.name = name
        self.events: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []
        self._pool = [self._pair() for _ in range(capacity)]
        torch.cuda.synchronize()

    @staticmethod
    def _pair() -> tuple[torch.cuda.Event, torch.cuda.Event]:
        # torch creates the HIP event at its first record; the launch then
        # re-records it with the kernel's timestamps.
        pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        for e in pair:
            e.record()
        return pair

    def next_pair(self) -> tuple[torch.cuda.Event, torch.cuda.Event]:
        if self._pool:
            return self._pool.pop()
        pair = self._pair()
        pair[1].synchronize()
        return pair

    def __enter__(self) -> "LaunchTimer":
        _TIMERS[self.name] = self
        return self

    def __exit__(self, *exc) -> None:
        _TIMERS.pop(self.name, None)

    def mean_ms(self) -> float:
        torch.cuda.synchronize()
        return sum(s.elapsed_time(e) for s, e in self.events) / max(1, len(self.events))


_TIMERS: dict[str, LaunchTimer] = {}


def launch(name: str, call):
    """Runs ``call()`` (one C-ABI entry point); while a LaunchTimer for
    ``name`` is active its main kernel's launch carries a pair of timing
    events, kept when a launch took them."""
    timer = _TIMERS.get(name)
    if timer is None:
        return call()
    start, end = timer.next_pair()
    lib = library()
    check(lib.gs_arm_launch_events(start.cuda_event, end.cuda_event), "arm_launch_events")
    try:
        status = call()
    finally:
        taken = lib.gs_disarm_launch_events()
    if taken:
        timer.events.append((start, end))
    return status


def host_floats(t: torch.Tensor, numel: int, name: str) -> torch.Tensor:
    """Contiguous float32 copy in host memory (the C-ABI passes camera
    extrinsics to the kernels by value); a GPU tensor costs one device sync."""
    t = t.detach()
    if t.numel() != numel:
        raise ValueError(f"{name} must have {numel} elements, got {t.numel()}")
    return t.to(device="cpu", dtype=torch.float32).contiguous()


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def dispatch_plan(
    view: GsView,
    num_tiles: int,
    device: torch.device,
    ranges: torch.Tensor | None = None,
    n_contributors: torch.Tensor | None = None,
) -> torch.Tensor:
    """Work items of the compositing kernels for ``view`` (gs_tile_order):
    each XCD's region of tiles, longest expected work first.  The estimate is
    the list length from ``ranges`` alone (a plan for gs_composite) or the
    largest contributor count of each tile's pixels from ``n_contributors``
    (a plan for gs_composite_bwd; with ``ranges`` too, tiles whose walk
    crosses the forward's checkpoints are split into segments).  The
    compositing call must get the same view."""
    if ranges is None and n_contributors is None:
        raise ValueError("dispatch_plan needs ranges or n_contributors")
    lib = library()
    count = lib.gs_tile_order_items(view, int(n_contributors is not None))
    if count < 0:
        check(GS_ERR_INVALID_ARGUMENT, "tile_order_items")
    items = torch.empty(int(count), dtype=torch.int32, device=device)
    ws = workspace(lib.gs_tile_order_workspace_bytes(num_tiles), device)
    check(
        lib.gs_tile_order(
            ptr(ranges), ptr(n_contributors), view, ptr(items), ptr(ws), ws.numel(), 0,
            stream(device),
        ),
        "tile_order",
    )
    return items


def tiles(image_width: int, image_height: int, tile_size: int) -> tuple[int, int]:
    """(tiles_w, tiles_h), partial tiles included."""
    return -(-image_width // tile_size), -(-image_height // tile_size)
