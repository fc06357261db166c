# -*- coding: utf-8 -*-
"""CPU checks that pin ``oracle/pipeline_ref.py`` (the conversion glue):
golden vectors written by the reference's own ``runtime/pipeline.py`` /
``runtime/retrieval.py`` (``tests/golden/make_golden_pipeline.py``), a float64
brute-force neighbour ranking, ``torch.nn.functional.interpolate`` for the
linear resamplers, float64 frame loops for the RMS curve and the closed form
of the int16 normalisation."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import pipeline_ref as pr

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pipeline_glue.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("case", ["a", "b", "c", "d"])
def test_vc_prepare_matches_reference(gold, case):
    g = lambda k: gold[f"prep_{case}_{k}"]  # noqa: E731
    rate, protect = (float(v) for v in g("params"))
    feats, pitch, pitchf = pr.vc_prepare(g("feats"), g("pitch"), g("pitchf"), g("vecs"), rate, protect)
    np.testing.assert_array_equal(pitch, g("out_pitch"))
    np.testing.assert_array_equal(pitchf, g("out_pitchf"))
    assert feats.shape == g("out_feats").shape and feats.dtype == np.float32
    np.testing.assert_allclose(feats, g("out_feats"), rtol=1e-6, atol=1e-6)


def test_search_l2_matches_reference(gold):
    sc, ix = pr.search_l2(gold["search_q"], gold["search_db"], k=8)
    np.testing.assert_array_equal(ix, gold["search_inds"])
    np.testing.assert_allclose(sc, gold["search_scores"], rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("case", ["a", "b", "c"])
def test_change_rms_matches_reference(gold, case):
    sr1, sr2, rate = gold[f"rms_{case}_params"]
    out = pr.change_rms(gold[f"rms_{case}_d1"], gold[f"rms_{case}_d2"], int(sr1), int(sr2), float(rate))
    np.testing.assert_allclose(out, gold[f"rms_{case}_out"], rtol=1e-6, atol=1e-7)


def test_search_l2_is_the_float64_ranking():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((30, 24)).astype(np.float32)
    db = rng.standard_normal((500, 24)).astype(np.float32)
    sc, ix = pr.search_l2(q, db, k=8)
    d64 = ((q[:, None, :].astype(np.float64) - db[None].astype(np.float64)) ** 2).sum(-1)
    ref = np.argsort(d64, axis=1, kind="stable")[:, :8]
    np.testing.assert_array_equal(ix, ref)
    np.testing.assert_allclose(sc, np.take_along_axis(d64, ref, axis=1), rtol=1e-4, atol=1e-3)
    # fewer rows than k: k = N, every row returned
    sc2, ix2 = pr.search_l2(q[:3], db[:5], k=8)
    assert sc2.shape == (3, 5) and sorted(ix2[0].tolist()) == [0, 1, 2, 3, 4]


def test_feature_blend_closed_form():
    rng = np.random.default_rng(2)
    vecs = rng.standard_normal((50, 8)).astype(np.float32)
    feats = rng.standard_normal((4, 8)).astype(np.float32)
    sc, ix = pr.search_l2(feats, vecs, k=8)
    out = pr.feature_blend(feats, vecs, sc, ix, 0.4)
    w = 1.0 / sc.astype(np.float64) ** 2
    w /= w.sum(axis=1, keepdims=True)
    blend = (vecs.astype(np.float64)[ix] * w[:, :, None]).sum(1)
    np.testing.assert_allclose(out, blend * 0.4 + feats * 0.6, rtol=1e-5, atol=1e-6)


def test_interpolations_match_torch():
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 5, 13)).astype(np.float32)
    ref = F.interpolate(torch.from_numpy(x), scale_factor=2, mode="linear", align_corners=False).numpy()
    np.testing.assert_allclose(pr.interpolate_linear(x, 2), ref, rtol=0, atol=1e-6)
    r = rng.random((1, 7)).astype(np.float32)
    for n_out in (1, 6, 7, 19, 1000):
        t = F.interpolate(torch.from_numpy(r.astype(np.float64))[None], size=n_out, mode="linear",
                          align_corners=False).numpy()[0]
        np.testing.assert_allclose(pr.interp_linear_size(r, n_out), t.astype(np.float32), rtol=1e-6, atol=1e-7)


def test_rms_curve_is_the_frame_rms():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(3333).astype(np.float32)
    sr = 1000
    hop = sr // 2
    got = pr.rms_curve(x, sr)[0]
    assert got.shape == (1 + len(x) // hop,)
    xp = np.concatenate([np.zeros(hop), x.astype(np.float64), np.zeros(hop)])
    ref = [np.sqrt(np.mean(xp[t * hop:t * hop + 2 * hop] ** 2)) for t in range(len(got))]
    np.testing.assert_allclose(got, ref, rtol=1e-5)


def test_to_int16_closed_form():
    x = np.array([0.5, -0.25, 1.0, -1.6, 0.0], dtype=np.float32)
    out = pr.to_int16(x)
    # peak 1.6 > 0.99: every value scaled by 0.99 * 32768 / 1.6, truncated toward zero
    s = np.float32(32768.0) / (np.float32(1.6) / np.float32(0.99))
    np.testing.assert_array_equal(out, np.trunc(x * s).astype(np.int16))
    assert out[3] == -32440 and out[4] == 0
    quiet = np.array([0.3, -0.7], dtype=np.float32)
    np.testing.assert_array_equal(pr.to_int16(quiet), np.array([9830, -22937], dtype=np.int16))


def test_protect_mask_cases():
    feats = np.ones((1, 2, 3), dtype=np.float32)
    pitch = np.array([[5, 6, 7, 8]], dtype=np.int64)
    pitchf = np.array([[200.0, 0.0, 0.5, 1.0]], dtype=np.float32)
    out, p, pf = pr.vc_prepare(feats * 2, pitch, pitchf, None, 0.0, 0.25)
    # no retrieval: feats == feats0, so the mask is the identity whatever pff is
    np.testing.assert_array_equal(out, np.full((1, 4, 3), 2.0, dtype=np.float32))
    np.testing.assert_array_equal(p, pitch)
