# -*- coding: utf-8 -*-
"""Deferred synthesis and the resident phone input on the GPU.

The reference's ``SynthesizerTrn.infer(..., phone_gpu=..., _defer=True)``
returns a holder whose ``collect()`` waits for the decoder and downloads the
waveform, so ``Pipeline`` prepares chunk i+1 on the host while the GPU
synthesises chunk i (``runtime/models/vits.py:2352-2402, 2551-2595``,
``runtime/pipeline.py:1010-1080``).  Every deferred result must equal the
synchronous call on the same inputs bit for bit, with several calls
outstanding and collected in any order."""

from __future__ import annotations

import numpy as np
import pytest

from rvc_hip import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny():
    from rvc_hip import _hip
    from rvc_hip.synth import HipSynthesizer

    assert _hip.has_so, _hip.so_load_error
    w = syn.make_weights(syn.GEOM_TINY, seed=5)
    return HipSynthesizer(w, sr=syn.GEOM_TINY.sr)


def _inputs(geom, P, seed):
    inp = syn.make_synth_inputs(geom, P=P, seed=seed)
    return inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"]


def test_two_outstanding_bit_identical(tiny):
    a = _inputs(syn.GEOM_TINY, 24, 1)
    b = _inputs(syn.GEOM_TINY, 24, 2)
    wa = tiny.infer_controlled(*a)
    wb = tiny.infer_controlled(*b)
    ha = tiny.infer_controlled(*a, _defer=True)
    hb = tiny.infer_controlled(*b, _defer=True)
    assert hasattr(ha, "collect") and hasattr(hb, "collect")
    # collected out of submission order
    np.testing.assert_array_equal(hb.collect(), wb)
    np.testing.assert_array_equal(ha.collect(), wa)
    with pytest.raises(RuntimeError):
        ha.collect()


def test_unequal_lengths_outstanding(tiny):
    """A longer second call grows the workspace while the first is queued."""
    a = _inputs(syn.GEOM_TINY, 10, 3)
    b = _inputs(syn.GEOM_TINY, 37, 4)
    wa, wb = tiny.infer_controlled(*a), tiny.infer_controlled(*b)
    ha = tiny.infer_controlled(*a, _defer=True)
    hb = tiny.infer_controlled(*b, _defer=True)
    hc = tiny.infer_controlled(*a, _defer=True)
    np.testing.assert_array_equal(ha.collect(), wa)
    np.testing.assert_array_equal(hb.collect(), wb)
    np.testing.assert_array_equal(hc.collect(), wa)


def test_resident_phone(tiny):
    a = _inputs(syn.GEOM_TINY, 16, 6)
    want = tiny.infer_controlled(*a)
    pb = tiny.ctx.persistent_upload(a[0][0])
    try:
        np.testing.assert_array_equal(tiny.infer_controlled(*a, phone_gpu=pb), want)
        h = tiny.infer_controlled(*a, phone_gpu=pb, _defer=True)
        np.testing.assert_array_equal(h.collect(), want)
        # the seeded infer route forwards phone_gpu / _defer too
        np.testing.assert_array_equal(tiny.infer(*a[:4], seed=9, phone_gpu=pb, _defer=True).collect(),
                                      tiny.infer(*a[:4], seed=9))
    finally:
        pb.free()
    # a freed buffer is ignored: phone is uploaded instead
    np.testing.assert_array_equal(tiny.infer_controlled(*a, phone_gpu=pb), want)


def test_abort_and_limit(tiny):
    a = _inputs(syn.GEOM_TINY, 8, 7)
    want = tiny.infer_controlled(*a)
    hs = [tiny.infer_controlled(*a, _defer=True) for _ in range(8)]
    with pytest.raises(RuntimeError, match="outstanding"):
        tiny.infer_controlled(*a, _defer=True)
    hs[3].abort()
    hs[3].abort()  # idempotent
    h9 = tiny.infer_controlled(*a, _defer=True)
    for i, h in enumerate(hs):
        if i != 3:
            np.testing.assert_array_equal(h.collect(), want)
    np.testing.assert_array_equal(h9.collect(), want)


def test_partial_ignores_defer(tiny):
    a = _inputs(syn.GEOM_TINY, 30, 8)
    got = tiny.infer(*a[:4], seed=4, skip_head=5, return_length=10, _defer=True)
    assert isinstance(got, np.ndarray)
    np.testing.assert_array_equal(got, tiny.infer(*a[:4], seed=4, skip_head=5, return_length=10))


def test_config2_two_outstanding():
    """BASELINE config 2 (40k, 10 s): two deferred calls in flight equal the
    synchronous calls bit for bit."""
    from rvc_hip.synth import HipSynthesizer

    geom = syn.GEOM_40K
    s = HipSynthesizer(syn.make_weights(geom, seed=0), sr=geom.sr)
    a = _inputs(geom, 1000, 31)
    b = _inputs(geom, 1000, 32)
    wa, wb = s.infer_controlled(*a), s.infer_controlled(*b)
    ha = s.infer_controlled(*a, _defer=True)
    hb = s.infer_controlled(*b, _defer=True)
    np.testing.assert_array_equal(ha.collect(), wa)
    np.testing.assert_array_equal(hb.collect(), wb)
    assert np.isfinite(wa).all() and np.abs(wa).max() <= 1.0
