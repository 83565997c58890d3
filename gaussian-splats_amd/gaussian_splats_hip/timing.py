"""Stage timings (reference: src/gaussian_splats/timing.py:1-70).

``with record_timings(device) as times:`` collects milliseconds per
``times[tag][title]``.  ``timed`` (decorator or context manager) times host
code and synchronises the device around it, as the reference's does.  The HIP
rasterizer's stages are recorded without synchronising: the op asks
``stage_timer()`` for a marker, records one event on the current stream
between stages ("Project", "Bin", "Emit", "Sort", "Composite", tag
"default"), and the events are read once, when the ``record_timings`` block
ends.  Set ``GAUSSIAN_SPLATS_DEBUG=0`` to disable all timing.
"""

from __future__ import annotations

import os
from collections.abc import Callable, Iterator
from contextlib import contextmanager
from contextvars import ContextVar
from functools import wraps
from time import perf_counter
from typing import Any

import torch

DEBUG = os.getenv("GAUSSIAN_SPLATS_DEBUG", "1") != "0"


class _Recording:
    def __init__(self, times: dict[str, dict[str, float]], device: torch.device):
        self.times = times
        self.device = torch.device(device)
        self.events: list[tuple[str, str, torch.cuda.Event, torch.cuda.Event]] = []

    def add(self, tag: str, title: str, ms: float) -> None:
        group = self.times.setdefault(tag, {})
        group[title] = group.get(title, 0.0) + ms

    def resolve(self) -> None:
        if not self.events:
            return
        self.events[-1][3].synchronize()
        for tag, title, start, end in self.events:
            self.add(tag, title, start.elapsed_time(end))
        self.events.clear()


_timers: ContextVar[_Recording | None] = ContextVar("timings", default=None)


@contextmanager
def record_timings(device: torch.device | str) -> Iterator[dict[str, dict[str, float]]]:
    times: dict[str, dict[str, float]] = {}
    recording = _Recording(times, device)
    token = _timers.set(recording)
    try:
        yield times
    finally:
        _timers.reset(token)
        recording.resolve()


def timed(title: str | Callable[..., Any] | None = None, *, tag: str = "default") -> Any:
    """``@timed``, ``@timed("Title")`` or ``with timed("Title"):``."""
    if callable(title):
        return _decorate(title, title.__name__.replace("_", " ").title(), tag)
    if title is None:
        return lambda function: _decorate(function, function.__name__.replace("_", " ").title(), tag)
    return _timer(title, tag)


def _decorate(function: Callable[..., Any], title: str, tag: str) -> Callable[..., Any]:
    @wraps(function)
    def wrapped(*args: Any, **kwargs: Any) -> Any:
        with _timer(title, tag):
            return function(*args, **kwargs)

    return wrapped


@contextmanager
def _timer(title: str, tag: str) -> Iterator[None]:
    recording = _timers.get()
    if not DEBUG or recording is None:
        yield
        return
    _synchronize(recording.device)
    start = perf_counter()
    try:
        yield
    finally:
        _synchronize(recording.device)
        recording.add(tag, title, 1000 * (perf_counter() - start))


def _synchronize(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def stage_timer(tag: str = "default") -> Callable[[str], None] | None:
    """Marker for a GPU pipeline while a recording is active (else None):
    ``mark(name)`` records an event on the current stream; the time between
    two marks is added to ``times[tag][Name]`` of the later one."""
    recording = _timers.get()
    if not DEBUG or recording is None or recording.device.type != "cuda":
        return None
    last: list[torch.cuda.Event | None] = [None]

    def mark(name: str) -> None:
        event = torch.cuda.Event(enable_timing=True)
        event.record()
        if last[0] is not None:
            title = name.replace("_", " ").title()
            recording.events.append((tag, title, last[0], event))
        last[0] = event

    return mark
