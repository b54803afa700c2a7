"""Labelled HIP-event timers for the merged global-attention path.

Mirrors the reference's `VGGT_PROFILE_ATTENTION_DETAIL` timers
(vggt_omega/models/layers/attention.py:25-63) and their `global.*` labels.
Events are recorded on torch's current stream, so they bracket exactly the
kernels launched there; nothing synchronises until `summary()`.
Enabled by `enable()` or by the environment variable VGO_PROFILE_ATTENTION=1.
"""
from __future__ import annotations

import contextlib
import os

import torch

_enabled = os.environ.get("VGO_PROFILE_ATTENTION", "0") == "1"
_only: frozenset[str] | None = None
_events: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []


def enable(flag: bool = True, only=None) -> None:
    """Switch recording on or off; `only` restricts it to the given labels."""
    global _enabled, _only
    _enabled = flag
    _only = None if only is None else frozenset(only)


def enabled() -> bool:
    return _enabled


def reset() -> None:
    _events.clear()


def span(label: str):
    """Context manager recording a begin/end event pair under `label` (a no-op context
    when recording is off or while torch.compile traces the caller)."""
    if not _enabled or torch.compiler.is_compiling() or (_only is not None and label not in _only):
        return contextlib.nullcontext()
    return _Span(label)


class _Span:
    """Records a begin/end event pair under `label`."""

    __slots__ = ("label", "begin")

    def __init__(self, label: str):
        self.label = label
        self.begin = None

    def __enter__(self):
        self.begin = torch.cuda.Event(enable_timing=True)
        self.begin.record()
        return self

    def __exit__(self, *exc):
        if self.begin is not None:
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            _events.append((self.label, self.begin, end))
        return False


def summary() -> dict[str, tuple[float, int]]:
    """label -> (total ms, calls); synchronises once."""
    if not _events:
        return {}
    torch.cuda.synchronize()
    totals: dict[str, list[float]] = {}
    for label, begin, end in _events:
        entry = totals.setdefault(label, [0.0, 0])
        entry[0] += begin.elapsed_time(end)
        entry[1] += 1
    return {label: (total, int(calls)) for label, (total, calls) in totals.items()}


def attention_kernel_timing(flag: bool = True) -> None:
    """Switch the library's kernel timing on or off: while on, every launch of the
    workspace attention kernel on the current device is bracketed by its own HIP
    event pair (the V^T pack and the split-task merge of the same call are not)."""
    from . import _lib

    lib = _lib.load()
    _lib.check(lib.vgo_attn_kernel_timing(1 if flag else 0))


def attention_kernel_clock() -> dict | None:
    """Mean shader clock of the attention launches timed since the last
    `attention_kernel_summary` (the first 512 of them), from the counters each
    work-group's wave 0 reads at its start and end; None when none were sampled.
    Call it before `attention_kernel_summary`, which empties the record.

    `clock_ghz` takes the constant counter at its 100 MHz rate; `const_mhz` is that
    rate as the launches' constant-clock spans over their HIP-event durations
    show it (a little low: the events also hold the launch's start-up and drain)."""
    import ctypes

    from . import _lib

    lib = _lib.load()
    cycles, ticks, span_ticks, span_ms = (ctypes.c_double(0.0) for _ in range(4))
    launches = ctypes.c_int64(0)
    _lib.check(lib.vgo_attn_kernel_clock_read(ctypes.byref(cycles), ctypes.byref(ticks),
                                              ctypes.byref(span_ticks), ctypes.byref(span_ms),
                                              ctypes.byref(launches)))
    if launches.value == 0 or ticks.value <= 0 or span_ms.value <= 0:
        return None
    return {"clock_ghz": cycles.value / ticks.value * 0.1,
            "const_mhz": span_ticks.value / span_ms.value / 1e3,
            "launches": int(launches.value)}


def attention_kernel_summary() -> tuple[float, int]:
    """(total ms, launches) of the attention kernel launches timed since the last
    call; waits for them, then empties the record."""
    import ctypes

    from . import _lib

    lib = _lib.load()
    total = ctypes.c_double(0.0)
    launches = ctypes.c_int64(0)
    dropped = ctypes.c_int64(0)
    _lib.check(lib.vgo_attn_kernel_timing_read(ctypes.byref(total), ctypes.byref(launches),
                                               ctypes.byref(dropped)))
    if dropped.value:
        raise RuntimeError(f"attention kernel timing: {dropped.value} launches were not recorded "
                           "(more than the library's 4096 event pairs)")
    return total.value, int(launches.value)
