# -*- coding: utf-8 -*-
"""CPU checks of the op surface's observability: the upload / download
counters (``stats_reset`` / ``stats_snapshot``, the reference's
``runtime/vulkan_ops.py:139-150, 225-249``) and the ``RVC_PROFILE`` per-op
timer table (``runtime/profiler.py:19-79``).

No GPU here: the ops run against a stub of the C library that accepts every
call and hands out buffer ids, so what is checked is the host-side count of
transfers each op makes, not the arithmetic (the GPU tests cover that)."""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest


class _StubLib:
    """Every export returns 0; the int64 out-parameter of upload / alloc
    receives a fresh buffer id."""

    def __init__(self):
        self.next_id = 100
        self.calls = []

    def __getattr__(self, name):
        def call(*args):
            self.calls.append(name)
            if name in ("rvc_mem_upload_bytes", "rvc_mem_alloc"):
                self.next_id += 1
                args[-1]._obj.value = self.next_id
            return 0

        return call


@pytest.fixture()
def ops(monkeypatch):
    from rvc_hip import hip_ops

    ctx = object.__new__(hip_ops.HipContext)
    ctx._lib = _StubLib()
    ctx.handle = 1
    ctx._lock = threading.RLock()
    monkeypatch.setattr(hip_ops, "_context", ctx)
    hip_ops.stats_reset()
    return hip_ops


def _f(*shape):
    return np.ones(shape, np.float32)


def test_stats_start_at_zero(ops):
    assert ops.stats_snapshot() == {"uploads": 0, "downloads": 0, "upload_bytes": 0, "download_bytes": 0}


def test_conv1d_counts_each_argument_and_the_result(ops):
    x, w, b = _f(2, 3, 10), _f(4, 3, 3), _f(4)
    ops.conv1d(x, w, b, padding=1)
    assert ops.stats_snapshot() == {"uploads": 3, "downloads": 1,
                                    "upload_bytes": x.nbytes + w.nbytes + b.nbytes,
                                    "download_bytes": 2 * 4 * 10 * 4}
    ops.conv1d(x, w)  # no bias: one upload fewer
    s = ops.stats_snapshot()
    assert (s["uploads"], s["downloads"]) == (5, 2)


def test_resident_weights_are_not_uploaded_again(ops):
    x, w = _f(1, 3, 8), _f(2, 3, 1)
    pw = ops.get_context().persistent_upload(w)
    assert ops.stats_snapshot()["uploads"] == 1
    ops.stats_reset()
    ops.conv1d(x, w, buf_w=pw)
    assert ops.stats_snapshot() == {"uploads": 1, "downloads": 1, "upload_bytes": x.nbytes,
                                    "download_bytes": 2 * 8 * 4}
    pw.update(w)
    assert ops.stats_snapshot()["uploads"] == 2


def test_matmul_and_elementwise_counts(ops):
    a, b = _f(3, 5), _f(5, 7)
    ops.matmul(a, b)
    ops.add(a, a)
    ops.relu(a)
    s = ops.stats_snapshot()
    assert s["uploads"] == 2 + 2 + 1
    assert s["downloads"] == 3
    assert s["download_bytes"] == (3 * 7 + 3 * 5 + 3 * 5) * 4
    ops.stats_reset()
    assert ops.stats_snapshot()["uploads"] == 0


def test_empty_results_make_no_transfers(ops):
    ops.matmul(_f(0, 4), _f(4, 3))
    assert ops.stats_snapshot()["uploads"] == 0


def test_profile_table(ops):
    from rvc_hip import profiler

    profiler.reset()
    profiler.set_enabled(False)
    try:
        ops.conv1d(_f(1, 2, 4), _f(2, 2, 1))
        assert profiler.snapshot() == {}
        assert "no entries" in profiler.report()
        profiler.set_enabled(True)
        ops.conv1d(_f(1, 2, 4), _f(2, 2, 1))
        ops.conv1d(_f(1, 2, 4), _f(2, 2, 1))
        ops.layer_norm(_f(3, 4), _f(4), _f(4))
        snap = profiler.snapshot()
        assert snap["conv1d/gpu"]["n"] == 2 and snap["layer_norm/gpu"]["n"] == 1
        assert all(v["us"] > 0 for v in snap.values())
        rep = profiler.report()
        lines = rep.splitlines()
        assert lines[1].split() == ["name", "calls", "per/us", "total/us", "%"]
        body = {ln.split()[0]: ln.split() for ln in lines[3:]}
        assert body["conv1d/gpu"][1] == "2"
        shares = [float(r[-1].rstrip("%")) for r in body.values()]
        assert abs(sum(shares) - 100.0) < 0.5
        # heaviest first
        totals = [float(r[3]) for r in body.values()]
        assert totals == sorted(totals, reverse=True)
    finally:
        profiler.set_enabled(False)
        profiler.reset()


def test_profile_op_context_manager():
    from rvc_hip import profiler

    profiler.reset()
    profiler.set_enabled(True)
    try:
        with profiler.profile_op("x/gpu"):
            pass
        with pytest.raises(ZeroDivisionError):
            with profiler.profile_op("x/gpu"):
                1 / 0
        assert profiler.snapshot()["x/gpu"]["n"] == 2
        assert "x/gpu" in profiler.report(total_us=1e6)
    finally:
        profiler.set_enabled(False)
        profiler.reset()
