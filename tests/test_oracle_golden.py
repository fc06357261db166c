# -*- coding: utf-8 -*-
"""The numpy oracle against golden vectors written by the reference's own
numpy code (tests/golden/make_golden.py).  CPU only."""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_l2
from oracle import nn_ref as nn
from oracle import vits_ref as V
from rvc_hip import synthetic as syn

GEOMS = {"tiny": syn.GEOM_TINY, "40k": syn.GEOM_40K, "48k": syn.GEOM_48K}


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def _weights(geom, seed, digest):
    w = syn.make_weights(geom, seed=int(seed))
    assert syn.weights_digest(w) == str(digest), "weight generator drifted from the fixtures"
    return w


def test_sine_gen_golden():
    d = _load("sine_gen.npz")
    w = _weights(syn.GEOM_TINY, d["seed"], d["digest"])
    gen = V.GeneratorNSF(w, V.VitsConfig(w, sr=int(d["sr"])))
    np.testing.assert_allclose(gen.sine_gen(d["f0"], d["ns"]), d["har"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(gen.sine_gen(d["f0_const"], d["ns"]), d["har_const"], rtol=0, atol=1e-6)


def test_vits_config_golden():
    with open(os.path.join(GOLDEN, "vits_config.json")) as f:
        cases = json.load(f)
    for name, case in cases.items():
        geom = GEOMS[name.split("_")[0]]
        w = syn.make_weights(geom, seed=1)
        c = V.VitsConfig(w, case["config"], sr=case["sr_arg"])
        for k, v in case["derived"].items():
            assert getattr(c, k) == v, (name, k)


def test_encoder_flow_golden():
    d = _load("enc_flow_40k.npz")
    w = _weights(syn.GEOM_40K, d["seed"], d["digest"])
    s = V.Synthesizer(w, sr=40000)
    for P in (5, 40):
        x = s.enc_p.embed(d[f"P{P}_phone"], d[f"P{P}_pitch"])
        x = nn.leaky_relu(x * math.sqrt(s.cfg.hidden), 0.1)
        assert rel_l2(x, d[f"P{P}_enc_in"]) < 1e-6
        h = s.enc_p.encode(x, np.ones((1, 1, P), np.float32))
        assert rel_l2(h, d[f"P{P}_enc_out"]) < 1e-6
        m, logs = s.enc_p.stats(h)
        assert rel_l2(m, d[f"P{P}_m"]) < 1e-6 and rel_l2(logs, d[f"P{P}_logs"]) < 1e-6
    g = s.resolve_g(d["flow_sid"])
    z = s.flow.reverse(d["flow_zp"], np.ones((1, 1, 40), np.float32), g)
    assert rel_l2(z, d["flow_z"]) < 1e-6


@pytest.mark.parametrize("name", ["synth_tiny_P8.npz", "synth_40k_P12.npz", "synth_48k_P10.npz"])
def test_end_to_end_golden(name):
    d = _load(name)
    geom = GEOMS[name.split("_")[1]]
    w = _weights(geom, d["wseed"], d["digest"])
    cfg = geom.config_array() if bool(d["use_config"]) else None
    s = V.Synthesizer(w, config=cfg, sr=None if cfg is not None else geom.sr)
    wave = s.infer_controlled(d["phone"], d["pitch"], d["nsff0"], d["sid"], d["nz"], d["ns"])
    assert np.abs(wave - d["wave"]).max() < 1e-5
    dw = s.dec.forward(d["dec_z"], d["dec_f0"], d["dec_g"], d["dec_ns"])
    assert np.abs(dw - d["dec_wave"]).max() < 1e-5
