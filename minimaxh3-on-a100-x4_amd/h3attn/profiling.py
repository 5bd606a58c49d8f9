"""Per-component GPU timing of the attention path.

The reference's profiler node (custom_nodes/h3_profiler/__init__.py:78-126)
wraps each sub-operation of the DiT attention in a CUDA-event pair and, after
one synchronisation, sums the pairs per component over all blocks of one
denoise step.  `OpTimer` does the same for the patched forward of
`h3attn.hooks`, with the same component names, so tools that read the
reference's `profile_step.json` read this report unchanged:

    attn.qkv          qkv_proj
    attn.qknorm_rope  the in-place qk-RMSNorm + RoPE prologue
    attn.softmax      attention (dense HIP kernel, or the active override)
    attn.out          out_proj

Events are recorded on the current stream, the stream the work is enqueued
on.  Nothing is timed while the timer is disarmed, so the hook costs one
attribute check per call.
"""
from __future__ import annotations

from typing import Callable

COMPONENTS = ("attn.qkv", "attn.qknorm_rope", "attn.softmax", "attn.out")


def _cuda_event():
    import torch

    return torch.cuda.Event(enable_timing=True)


def _cuda_sync():
    import torch

    torch.cuda.synchronize()


class OpTimer:
    """Accumulate (start, end) event pairs per component while armed.

    `event_factory` returns an object with record() and elapsed_time(other)
    (a timing-enabled torch.cuda.Event by default); `synchronize` waits for
    the recorded work.  Both are injectable so the bookkeeping is testable
    without a GPU.
    """

    def __init__(self, event_factory: Callable = _cuda_event, synchronize: Callable = _cuda_sync):
        self._new = event_factory
        self._sync = synchronize
        self.armed = False
        self._ev: dict[str, list] = {}

    def arm(self) -> None:
        """Start a new measurement (drops earlier pairs)."""
        self._ev = {}
        self.armed = True

    def disarm(self) -> None:
        self.armed = False

    def mark(self, name: str, fn: Callable, *args, **kwargs):
        """Run fn(*args, **kwargs); while armed, bracket it with an event pair under `name`."""
        if not self.armed:
            return fn(*args, **kwargs)
        start, end = self._new(), self._new()
        start.record()
        out = fn(*args, **kwargs)
        end.record()
        self._ev.setdefault(name, []).append((start, end))
        return out

    def report(self, total_ms: float | None = None) -> dict:
        """Summed GPU ms per component (one synchronisation), call counts, and
        with `total_ms` (the whole step) the remainder and the percentages, as
        the reference's profile_step.json lays them out."""
        self._sync()
        comp = {name: round(sum(s.elapsed_time(e) for s, e in pairs), 3) for name, pairs in self._ev.items()}
        summed = round(sum(comp.values()), 3)
        rep = {"components_ms": comp, "calls": {n: len(p) for n, p in self._ev.items()},
               "sum_components_ms": summed}
        if total_ms is not None:
            rep["total_forward_ms"] = round(total_ms, 3)
            rep["other_ms"] = round(total_ms - summed, 3)
            rep["components_pct"] = {n: round(100.0 * v / total_ms, 1) for n, v in comp.items()} if total_ms else {}
        return rep


def passthrough(name: str, fn: Callable, *args, **kwargs):
    """The `mark` of no timer: call fn directly."""
    del name
    return fn(*args, **kwargs)
