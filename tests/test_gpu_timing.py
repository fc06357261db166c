# -*- coding: utf-8 -*-
"""The synthesizer's per-family timing (``set_timing`` / ``get_timing``), which
bench.py's roofline and breakdown read.  A span of consecutive timed launches
starts with an event record and ends either with an event attached to its
last kernel's own dispatch (the persistent ResBlock conv, the ConvTranspose
and conv_post launches) or, for other kernels, with an event record.  Both
kinds must count every launch once, add the host's FLOP figures, and time
no more than the calls' wall clock, and a timed call must produce the same
waveform as an untimed one."""

from __future__ import annotations

import time

import numpy as np
import pytest

from rvc_hip import synthetic as syn

pytestmark = pytest.mark.gpu

GEOM = syn.GEOM_40K
P = 1000  # config 2: the ResBlock launches take the persistent kernel


@pytest.fixture(scope="module")
def setup():
    from rvc_hip import _hip
    from rvc_hip.hip_ops import get_context
    from rvc_hip.synth import HipSynthesizer

    assert _hip.has_so, _hip.so_load_error
    ctx = get_context()
    s = HipSynthesizer(syn.make_weights(GEOM, seed=0), sr=GEOM.sr, ctx=ctx)
    inp = syn.make_synth_inputs(GEOM, P, seed=3)
    ids = (
        ctx.upload(np.ascontiguousarray(inp["phone"], np.float32)),
        ctx.upload(np.ascontiguousarray(inp["pitch"], np.int64)),
        ctx.upload(np.ascontiguousarray(inp["nsff0"], np.float32)),
        ctx.upload(np.ascontiguousarray(inp["sid"], np.int64)),
        ctx.upload(np.ascontiguousarray(inp["nz"], np.float32)),
        ctx.upload(np.ascontiguousarray(inp["ns"], np.float32).reshape(-1)),
    )
    wave = ctx.alloc(P * GEOM.upp)

    def call():
        s.infer_dev(*ids, 1, P, wave)
        return ctx.download(wave, (P * GEOM.upp,))

    ref = call()  # untimed; also allocates the workspace
    return s, call, ref


# (tag, launches per call): 4 stages x 6 ResBlock launches; one conv_post;
# four upsamplers; stage 1's six launches alone; the averages of stages 0-2
# (stage 3's is folded into conv_post); conv_pre; enc_p and the flow (spans
# of many launches, most ending with an event record)
CASES = [("dec.rb", 24), ("dec.post", 1), ("dec.ups", 4), ("dec.rb.s1", 6), ("dec.avg", 3), ("dec.pre", 1),
         ("enc", None), ("flow", None)]


@pytest.mark.parametrize("tag,per_call", CASES)
def test_span_counts_and_bounds(setup, tag, per_call):
    s, call, ref = setup
    n = 3
    s.set_timing(tag)
    try:
        t0 = time.perf_counter()
        for _ in range(n):
            out = call()
            np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))
        wall_ms = (time.perf_counter() - t0) * 1e3
        t = s.get_timing()
    finally:
        s.set_timing("")
    print(f"{tag}: {t['launches']} launches, {t['ms']:.3f} ms of {wall_ms:.1f} ms wall, {t['flops'] / 1e9:.2f} GFLOP")
    assert t["launches"] > 0 and t["launches"] % n == 0
    if per_call is not None:
        assert t["launches"] == n * per_call
    assert 0.0 < t["ms"] < wall_ms
    # every launch of the family takes at least a few microseconds
    assert t["ms"] / t["launches"] > 2e-3


def test_resblock_flops_and_rate(setup):
    """The ResBlock family's FLOPs are the host's sum of 2 C^2 k L over the
    launch groups; the timed rate stays physical (below the fp32 MFMA peak)."""
    s, call, _ = setup
    s.set_timing("dec.rb")
    try:
        call()
        t = s.get_timing()
    finally:
        s.set_timing("")
    want = 0.0
    L = P
    for C, rate in zip((256, 128, 64, 32), (10, 10, 2, 2)):
        L *= rate
        want += 2 * 2 * C * C * (3 + 7 + 11) * 3 * L  # two convs per dilation, three dilations
    assert t["flops"] == pytest.approx(want, rel=1e-9)
    tflops = t["flops"] / (t["ms"] * 1e-3) / 1e12
    assert 20.0 < tflops < 157.3
