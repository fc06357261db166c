# -*- coding: utf-8 -*-
"""Per-op wall-clock timer table for the op-level HIP backend.

The reference times its GPU ops with ``RVC_PROFILE=1`` and prints a table of
name / calls / time per call / total / share (``runtime/profiler.py:19-79``,
applied to ``vulkan_ops`` through the ``traced`` decorator,
``runtime/vulkan_ops.py:35-48``).  This module keeps the same switch, names
and report columns for ``rvc_hip.hip_ops``.  Each entry is the host time of
one op call from argument checks to the downloaded result (upload, launch,
synchronising download), so it is what a caller of the op waits for.

Off by default: with ``RVC_PROFILE`` unset an op pays one flag test.
``set_enabled`` switches it at run time (tests, notebooks).
"""

from __future__ import annotations

import os
import threading
import time

_enabled = os.environ.get("RVC_PROFILE", "0").strip().lower() in ("1", "true", "on")
_lock = threading.Lock()
_table: dict = {}  # name -> [calls, total microseconds]


def enabled() -> bool:
    return _enabled


def set_enabled(on: bool) -> None:
    global _enabled
    _enabled = bool(on)


class profile_op:
    """``with profile_op("conv1d/gpu"):`` adds the block's wall time to the
    entry ``name`` when profiling is on (the name carries the device suffix,
    as in the reference)."""

    __slots__ = ("name", "t0")

    def __init__(self, name: str, device: str = "gpu"):
        self.name = name
        self.t0 = 0.0

    def __enter__(self):
        self.t0 = time.perf_counter()
        return self

    def __exit__(self, *exc):
        if _enabled:
            us = (time.perf_counter() - self.t0) * 1e6
            with _lock:
                ent = _table.setdefault(self.name, [0, 0.0])
                ent[0] += 1
                ent[1] += us
        return False


def reset() -> None:
    with _lock:
        _table.clear()


def snapshot() -> dict:
    """{name: {"n": calls, "us": total microseconds}}."""
    with _lock:
        return {k: {"n": v[0], "us": v[1]} for k, v in _table.items()}


def report(total_us: float | None = None) -> str:
    """The table, heaviest entry first: name, calls, us per call, total us,
    share of ``total_us`` (default: the sum of the entries)."""
    snap = snapshot()
    if not snap:
        return "[profiler] no entries (set RVC_PROFILE=1 and run again)"
    if total_us is None:
        total_us = sum(v["us"] for v in snap.values())
    rows = sorted(snap.items(), key=lambda kv: -kv[1]["us"])
    out = [f"[profiler] per-op totals ({total_us / 1000.0:.1f} ms)",
           f"{'name':<40} {'calls':>8} {'per/us':>10} {'total/us':>12} {'%':>7}",
           "-" * 82]
    for name, v in rows:
        per = v["us"] / v["n"] if v["n"] else 0.0
        pct = 100.0 * v["us"] / total_us if total_us else 0.0
        out.append(f"{name:<40} {v['n']:>8d} {per:>10.1f} {v['us']:>12.0f} {pct:>6.1f}%")
    return "\n".join(out)
