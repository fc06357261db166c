# -*- coding: utf-8 -*-
"""Pin the oracle's noise draw and partial-synthesis path against vectors
the reference's own numpy code wrote (tests/golden/synth_partial_tiny.npz,
from tests/golden/make_golden_partial.py): ``_make_noise`` (nz before ns,
RVC_FIXED_SEED for seed=None), ``infer(seed)``, ``_phase_offsets``,
``prep_dec`` full and partial, ``decode_batch(preps)`` over unequal chunks
and ``infer(skip_head, return_length)`` (runtime/models/vits.py:2337-2531).

Everything here is float32 numpy in both programs with the same operation
order, so the comparison is exact up to BLAS summation order (which the two
share on one machine): noise, offsets and crop bounds are compared bit for
bit, waves at max-abs 1e-5."""

from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import vits_ref as V
from rvc_hip import synthetic as syn

WAVE_TOL = 1e-5


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(GOLDEN, "synth_partial_tiny.npz"))


@pytest.fixture(scope="module")
def ref(gold):
    w = syn.make_weights(syn.GEOM_TINY, seed=int(gold["wseed"]))
    assert syn.weights_digest(w) == str(gold["digest"])
    return V.Synthesizer(w, sr=syn.GEOM_TINY.sr)


def _args(g):
    return g["phone"], g["pitch"], g["nsff0"], g["sid"]


def test_noise_draw_order_and_fixed_seed(gold, ref):
    P = gold["phone"].shape[1]
    nz, ns = ref.make_noise(P, int(gold["seed"]))
    np.testing.assert_array_equal(nz, gold["nz"])
    np.testing.assert_array_equal(ns, gold["ns"])
    fz, fs = ref.make_noise(P, None, fixed_seed="77")
    np.testing.assert_array_equal(fz, gold["fixed77_nz"])
    np.testing.assert_array_equal(fs, gold["fixed77_ns"])
    # drawing ns first would give other arrays: the order is pinned, not assumed
    rng = np.random.RandomState(int(gold["seed"]))
    assert not np.array_equal(rng.standard_normal(ns.shape).astype(np.float32), gold["ns"])


def test_infer_with_seed(gold, ref):
    wave = ref.infer(*_args(gold), seed=int(gold["seed"]))
    assert np.abs(wave - gold["wave"]).max() <= WAVE_TOL


def test_phase_offsets(gold, ref):
    np.testing.assert_array_equal(ref.phase_offsets(gold["nsff0"]), gold["phase_offsets"])


@pytest.mark.parametrize("i", [0, 1, 2])
def test_partial_prep_and_infer(gold, ref, i):
    head, length = (int(v) for v in gold["parts"][i])
    p = ref.prep_dec(*_args(gold), seed=int(gold["seed"]), skip_head=head, return_length=length)
    assert p["s0"] == int(gold[f"part{i}_s0"]) and p["n_out"] == int(gold[f"part{i}_n_out"])
    np.testing.assert_array_equal(p["off"], gold[f"part{i}_off"])
    np.testing.assert_array_equal(p["nsff0_seg"], gold[f"part{i}_nsff0_seg"])
    np.testing.assert_array_equal(p["ns_seg"], gold[f"part{i}_ns_seg"])
    assert np.abs(p["z_seg"] - gold[f"part{i}_z_seg"]).max() <= WAVE_TOL
    wave = ref.infer(*_args(gold), seed=int(gold["seed"]), skip_head=head, return_length=length)
    assert wave.shape == gold[f"part{i}_wave"].shape
    assert np.abs(wave - gold[f"part{i}_wave"]).max() <= WAVE_TOL


def test_decode_batch_of_unequal_preps(gold, ref):
    seed = int(gold["seed"])
    preps = [ref.prep_dec(*_args(gold), seed=seed)]
    preps += [ref.prep_dec(*_args(gold), seed=seed, skip_head=int(h), return_length=int(n))
              for h, n in gold["parts"]]
    waves = ref.decode_batch(preps)
    assert len(waves) == 4
    for i, wv in enumerate(waves):
        assert np.abs(wv - gold[f"batch{i}_wave"]).max() <= WAVE_TOL


def test_partial_rejects_out_of_range(gold, ref):
    P = gold["phone"].shape[1]
    with pytest.raises(ValueError):
        ref.prep_dec(*_args(gold), seed=1, skip_head=P, return_length=1)
    with pytest.raises(ValueError):
        ref.infer(*_args(gold), seed=1, skip_head=P - 2, return_length=3)
