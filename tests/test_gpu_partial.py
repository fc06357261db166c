# -*- coding: utf-8 -*-
"""Noise draw, partial synthesis and ragged batched decode on the GPU.

Against vectors the reference's own numpy code wrote
(tests/golden/synth_partial_tiny.npz, tests/golden/make_golden_partial.py)
and the numpy oracle: ``make_noise`` / ``infer(seed)`` /
``RVC_FIXED_SEED``, ``_phase_offsets``, ``prep_dec`` full and partial,
``decode_batch(preps)`` over chunks of unequal lengths and
``infer(skip_head, return_length)`` (runtime/models/vits.py:2337-2531,
1484-1491, 1847-1878).  Tolerances: waveform max-abs <= 1e-3, intermediates
rel L2 <= 1e-4; integer-like outputs (noise,
segment bounds) exact.  Plus the device path's rejection of out-of-range
pitch / speaker ids."""

from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_l2
from oracle import nn_ref as nn
from oracle import vits_ref as V
from rvc_hip import synthetic as syn

pytestmark = pytest.mark.gpu

WAVE_TOL = 1e-3
OP_TOL = 1e-4


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "synth_partial_tiny.npz"))


@pytest.fixture(scope="module")
def hip(gold):
    from rvc_hip import _hip
    from rvc_hip.synth import HipSynthesizer

    assert _hip.has_so, _hip.so_load_error
    w = syn.make_weights(syn.GEOM_TINY, seed=int(gold["wseed"]))
    assert syn.weights_digest(w) == str(gold["digest"])
    return HipSynthesizer(w, sr=syn.GEOM_TINY.sr)


def _args(g):
    return g["phone"], g["pitch"], g["nsff0"], g["sid"]


def test_noise_and_infer_with_seed(gold, hip, monkeypatch):
    from rvc_hip import synth as synth_mod

    P = gold["phone"].shape[1]
    nz, ns = hip.make_noise(P, int(gold["seed"]))
    np.testing.assert_array_equal(nz, gold["nz"])
    np.testing.assert_array_equal(ns, gold["ns"])
    wave = hip.infer(*_args(gold), seed=int(gold["seed"]))
    assert np.abs(wave - gold["wave"]).max() <= WAVE_TOL
    monkeypatch.setattr(synth_mod, "_FIXED_SEED", "77")
    fz, fs = hip.make_noise(P, None)
    np.testing.assert_array_equal(fz, gold["fixed77_nz"])
    np.testing.assert_array_equal(fs, gold["fixed77_ns"])
    np.testing.assert_array_equal(hip.infer(*_args(gold)), hip.infer(*_args(gold), seed=77))


def test_phase_offsets(gold, hip):
    got = hip.phase_offsets(gold["nsff0"])
    assert got.shape == gold["phase_offsets"].shape
    np.testing.assert_allclose(got, gold["phase_offsets"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("P", [16383, 16384, 20000, 70001])
def test_phase_offsets_long(hip, P):
    """Past one LDS block of the scan (4096 frames) and past the old
    16 384-frame cap: bit-for-bit against the oracle's float32 cumsum."""
    rng = np.random.default_rng(P)
    f0 = rng.uniform(80.0, 400.0, size=(1, P)).astype(np.float32)
    f0[:, rng.random(P) < 0.2] = 0.0
    got = hip.phase_offsets(f0)
    want = V.Synthesizer.phase_offsets(hip_oracle_stub(hip), f0)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got, want)


def hip_oracle_stub(hip):
    """The oracle's phase_offsets needs only cfg.sr and cfg.upp."""
    class _S:
        pass

    s = _S()
    s.cfg = hip.cfg
    return s


@pytest.mark.parametrize("i", [0, 1, 2])
def test_partial_prep_and_infer(gold, hip, i):
    head, length = (int(v) for v in gold["parts"][i])
    seed = int(gold["seed"])
    p = hip.prep_dec(*_args(gold), seed=seed, skip_head=head, return_length=length)
    assert p["s0"] == int(gold[f"part{i}_s0"]) and p["n_out"] == int(gold[f"part{i}_n_out"])
    np.testing.assert_allclose(p["off"], gold[f"part{i}_off"], rtol=0, atol=1e-6)
    np.testing.assert_array_equal(p["ns_seg"], gold[f"part{i}_ns_seg"])
    np.testing.assert_array_equal(p["nsff0_seg"], gold[f"part{i}_nsff0_seg"])
    assert rel_l2(p["z_seg"], gold[f"part{i}_z_seg"]) < OP_TOL
    wave = hip.infer(*_args(gold), seed=seed, skip_head=head, return_length=length)
    assert wave.shape == gold[f"part{i}_wave"].shape
    assert np.abs(wave - gold[f"part{i}_wave"]).max() <= WAVE_TOL


def test_decode_batch_unequal_preps(gold, hip):
    """decode_batch(preps) over a full chunk and three partial chunks of
    three different lengths: each equals the reference's, and each equals
    the decoder run on that chunk alone bit for bit."""
    seed = int(gold["seed"])
    preps = [hip.prep_dec(*_args(gold), seed=seed)]
    preps += [hip.prep_dec(*_args(gold), seed=seed, skip_head=int(h), return_length=int(n))
              for h, n in gold["parts"]]
    assert len({p["z_seg"].shape[-1] for p in preps}) >= 3
    waves = hip.decode_batch(preps)
    for i, (p, wv) in enumerate(zip(preps, waves)):
        assert np.abs(wv - gold[f"batch{i}_wave"]).max() <= WAVE_TOL
        one = hip.dec.forward(p["z_seg"], p["nsff0_seg"], p["g"], p["ns_seg"], seg_offsets=p["off"])
        np.testing.assert_array_equal(wv, one[:, :, p["s0"]:p["s0"] + p["n_out"]])


def test_generator_decode_batch_ragged_vs_oracle():
    """_GeneratorNSF.decode_batch with unequal lengths, offsets on some
    chunks and none on others, no speaker (g=None), at the 40k geometry:
    every chunk against the oracle's forward."""
    from rvc_hip.synth import HipSynthesizer

    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=12)
    s = HipSynthesizer(w, sr=geom.sr)
    gen = V.GeneratorNSF(w, V.VitsConfig(w, sr=geom.sr))
    rng = np.random.default_rng(3)
    chunks = []
    for P, with_off in ((23, False), (40, True), (23, True), (31, False), (40, False)):
        d = syn.make_dec_inputs(geom, P, seed=int(rng.integers(1 << 30)))
        off = (rng.random((1, P, 1)) - 0.5).astype(np.float32) if with_off else None
        chunks.append((d, off))
    waves = s.dec.decode_batch([d["z"] for d, _ in chunks], None, [d["f0"] for d, _ in chunks],
                               [d["ns"] for d, _ in chunks], [o for _, o in chunks])
    with nn.conv_formulation("taps"):
        for (d, off), wv in zip(chunks, waves):
            want = gen.forward(d["z"], d["f0"], None, d["ns"], seg_offsets=off)
            assert wv.shape == want.shape
            assert np.abs(wv - want).max() <= WAVE_TOL


def test_device_path_rejects_out_of_range_ids():
    """rvc_synth_infer_dev: an out-of-range pitch or sid id fails the call
    (the host path and numpy's take raise too), an in-range negative id wraps."""
    from rvc_hip.hip_ops import get_context
    from rvc_hip.synth import HipSynthesizer

    geom = syn.GEOM_TINY
    w = syn.make_weights(geom, seed=5)
    ctx = get_context()
    s = HipSynthesizer(w, sr=geom.sr, ctx=ctx)
    P = 12
    inp = syn.make_synth_inputs(geom, P, seed=4)
    rows = w["enc_p.emb_pitch.weight"].shape[0]
    n_spk = w["emb_g.weight"].shape[0]

    def run(pitch, sid):
        ids = [ctx.upload(inp["phone"].astype(np.float32)), ctx.upload(pitch.astype(np.int64)),
               ctx.upload(inp["nsff0"].astype(np.float32)), ctx.upload(sid.astype(np.int64)),
               ctx.upload(inp["nz"].astype(np.float32)), ctx.upload(inp["ns"].astype(np.float32).reshape(-1))]
        wave = ctx.alloc(P * geom.upp)
        try:
            s.infer_dev(*ids, 1, P, wave)
            return ctx.download(wave, (1, 1, P * geom.upp))
        finally:
            for b in ids + [wave]:
                ctx.free(b)

    good = run(inp["pitch"], inp["sid"])
    want = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    np.testing.assert_array_equal(good, want)
    bad = inp["pitch"].copy()
    bad[0, 3] = rows
    with pytest.raises(RuntimeError, match="pitch id out of range"):
        run(bad, inp["sid"])
    with pytest.raises(RuntimeError, match="sid out of range"):
        run(inp["pitch"], np.array([n_spk]))
    wrap = inp["pitch"].copy()
    wrap[0, 3] = wrap[0, 3] - rows  # -rows <= id < 0 wraps like numpy
    np.testing.assert_array_equal(run(wrap, inp["sid"]), good)
    # the session is still usable after a rejected call
    np.testing.assert_array_equal(run(inp["pitch"], inp["sid"]), good)
