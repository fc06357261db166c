# -*- coding: utf-8 -*-
"""The HuBERT oracle (oracle/hubert_ref.py) against the reference's own
outputs (tests/golden/hubert_base.npz, written by make_golden_hubert.py) and
against closed forms.  CPU only."""

from __future__ import annotations

import math
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_l2
from oracle import hubert_ref as H
from rvc_hip import synthetic as syn


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "hubert_base.npz"))


@pytest.fixture(scope="module")
def ref(golden):
    sd = syn.make_hubert_weights(syn.HUBERT_BASE, seed=int(golden["wseed"]))
    assert syn.weights_digest(sd) == str(golden["digest"]), "HuBERT weight generator drifted from the fixture"
    return H.HubertRef(sd)


def test_gelu_matches_reference_and_erf(golden):
    y = H.gelu_erf(golden["gelu_x"])
    np.testing.assert_array_equal(y, golden["gelu_y"])
    # A&S 7.1.26 has |erf error| <= 1.5e-7, so |GELU error| <= 0.5 |x| 1.5e-7 + float32 rounding
    x = golden["gelu_x"].astype(np.float64)
    exact = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in x])
    assert np.all(np.abs(y - exact) <= 0.5 * np.abs(x) * 1.5e-7 + 4e-7 * np.maximum(np.abs(exact), 1e-3))


def test_group_norm_is_per_group_standardisation():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 6, 17)).astype(np.float32) * 3 + 1
    g, b = rng.standard_normal(6).astype(np.float32), rng.standard_normal(6).astype(np.float32)
    y = H.group_norm(x, g, b, num_groups=3)
    xd = x.astype(np.float64).reshape(1, 3, 2, 17)
    mu = xd.mean(axis=(2, 3), keepdims=True)
    sd = np.sqrt(((xd - mu) ** 2).mean(axis=(2, 3), keepdims=True) + 1e-5)
    want = ((xd - mu) / sd).reshape(1, 6, 17) * g.reshape(1, 6, 1) + b.reshape(1, 6, 1)
    assert rel_l2(y, want) < 1e-6


def test_pos_conv_weight_norm_special_case():
    rng = np.random.default_rng(1)
    v = rng.standard_normal((8, 2, 5)).astype(np.float32)
    g = np.sqrt((v.astype(np.float64) ** 2).sum(axis=(0, 1))).astype(np.float32).reshape(1, 1, 5)
    assert rel_l2(H.pos_conv_weight(g, v), v) < 1e-6
    # scaling g per tap scales that tap only
    g2 = g.copy()
    g2[0, 0, 3] *= 2
    w2 = H.pos_conv_weight(g2, v)
    assert rel_l2(w2[:, :, 3], 2 * v[:, :, 3]) < 1e-6 and rel_l2(w2[:, :, :3], v[:, :, :3]) < 1e-6


def test_grouped_conv_equals_block_diagonal_conv():
    from oracle import loops

    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 6, 20)).astype(np.float32)
    w = rng.standard_normal((6, 2, 5)).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    dense = np.zeros((6, 6, 5), np.float32)
    for gi in range(3):
        dense[2 * gi:2 * gi + 2, 2 * gi:2 * gi + 2] = w[2 * gi:2 * gi + 2]
    y = H.grouped_conv1d(x, w, b, groups=3, padding=2)
    assert rel_l2(y, loops.conv1d(x, dense, b, 1, 2, 2, 1)) < 1e-6


def test_frame_count_config3():
    assert syn.HUBERT_BASE.frames(160000) == 499
    assert syn.HUBERT_BASE.frames(1600) == 4


@pytest.mark.parametrize("T", [1600, 4000])
def test_stages_match_reference_golden(golden, ref, T):
    x = golden[f"T{T}_x"]
    feats = ref.feature_extractor(x)
    assert rel_l2(feats, golden[f"T{T}_feats"]) < 1e-5
    proj = ref.feature_projection(golden[f"T{T}_feats"])
    assert rel_l2(proj, golden[f"T{T}_proj"]) < 1e-5
    hs = ref.encoder(golden[f"T{T}_proj"], upto=1)
    assert rel_l2(hs[0], golden[f"T{T}_entry"]) < 1e-5
    assert rel_l2(hs[1], golden[f"T{T}_layer1"]) < 1e-5
    assert rel_l2(ref.encode(x, version=2), golden[f"T{T}_v2"]) < 1e-5
    assert rel_l2(ref.encode(x, version=1), golden[f"T{T}_v1"]) < 1e-5
