"""Per-kernel HIP-event timing for the benchmark.

When a ``KernelTimer`` is active, every C-ABI launch made through
``flashgrpo_amd.kernels`` is bracketed by two ``torch.cuda.Event`` records on
the stream the kernel is launched on (torch's current stream). Labels set with
``label(...)`` refine the kernel name (e.g. the LM-head GEMM of the packed tree
rows vs. the Medusa rows). Off by default: no events are recorded.
"""
from __future__ import annotations

import contextlib
import threading
from collections import defaultdict

import torch

_state = threading.local()


class KernelTimer:
    """Collects (start, end) event pairs per kernel name. ``only``: a set of C-ABI
    entry-point names to time (None: every launch)."""

    def __init__(self, only=None, every: int = 1, reserve: int = 0):
        self.events = defaultdict(list)
        self.only = None if only is None else set(only)
        self.every = max(1, int(every))  # time one launch in `every` of each name
        self.seen = defaultdict(int)
        # Event pairs created up front (each recorded once so the runtime object
        # exists): creating events inside a timed region has cost tens of ms when
        # the runtime grows its signal pool.
        self.pool = []
        for _ in range(max(0, int(reserve))):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            e.record()
            self.pool.append((s, e))

    def pair(self):
        if self.pool:
            return self.pool.pop()
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def summary(self) -> dict:
        """{name: {"count", "total_ms", "avg_ms"}} after synchronising."""
        torch.cuda.synchronize()
        out = {}
        for name, evs in self.events.items():
            ms = [s.elapsed_time(e) for s, e in evs]
            out[name] = {"count": len(ms), "total_ms": float(sum(ms)), "avg_ms": float(sum(ms) / max(len(ms), 1))}
        return out


def _timer():
    return getattr(_state, "timer", None)


def idle() -> bool:
    """True when no KernelTimer is active on this thread."""
    return getattr(_state, "timer", None) is None


def _labels():
    if not hasattr(_state, "labels"):
        _state.labels = []
    return _state.labels


@contextlib.contextmanager
def active(timer: KernelTimer | None):
    prev = _timer()
    _state.timer = timer
    try:
        yield timer
    finally:
        _state.timer = prev


@contextlib.contextmanager
def label(name: str):
    _labels().append(name)
    try:
        yield
    finally:
        _labels().pop()


@contextlib.contextmanager
def launch(kernel: str):
    t = _timer()
    if t is None or (t.only is not None and kernel not in t.only):
        yield
        return
    labels = _labels()
    name = kernel + (":" + labels[-1] if labels else "")
    n = t.seen[name]
    t.seen[name] = n + 1
    if n % t.every:
        yield
        return
    s, e = t.pair()
    s.record()
    try:
        yield
    finally:
        e.record()
        t.events[name].append((s, e))
