# -*- coding: utf-8 -*-
"""GPU parity of the conversion glue (``rvc_vc_*``) against the oracle and the
reference's golden vectors.

Tolerances: the elementwise steps (interpolation, protect mask, int16) are
bit-identical to the reference's float32 expressions; retrieval distances come
from an MFMA GEMM whose summation order differs from BLAS, so neighbour sets
are compared exactly where the oracle's ranking has no near-tie and the
blended features at relative 1e-5; RMS frame sums and powf differ in the last
bits, so change_rms is checked at relative 1e-5."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import pipeline_ref as pr

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "pipeline_glue.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def hp():
    from rvc_hip import _hip

    if not _hip.has_so:
        pytest.fail(f"HIP backend missing: {_hip.so_load_error}")
    from rvc_hip.pipeline import HipPipeline

    p = HipPipeline(tgt_sr=40000)
    yield p
    p.glue.close()


def _check_neighbours(sc_ref, ix_ref, sc, ix, gap):
    """Indices equal wherever the oracle's consecutive distances differ by
    more than `gap` (a near-tie may legitimately swap); scores close."""
    assert ix.shape == ix_ref.shape and sc.shape == sc_ref.shape
    d = np.diff(np.concatenate([sc_ref, np.full((sc_ref.shape[0], 1), np.inf, np.float32)], axis=1), axis=1)
    ok = (d > gap) & np.concatenate([np.ones((d.shape[0], 1), bool), d[:, :-1] > gap], axis=1)
    assert ok.mean() > 0.9
    np.testing.assert_array_equal(ix[ok], ix_ref[ok])
    np.testing.assert_allclose(sc, sc_ref, rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("N,F,D", [(5, 7, 16), (400, 37, 32), (4099, 129, 64), (50000, 200, 768)])
def test_search_matches_oracle(hp, N, F, D):
    print(f"search N={N} F={F} D={D}", flush=True)
    rng = np.random.default_rng(N + F)
    db = rng.standard_normal((N, D)).astype(np.float32)
    q = rng.standard_normal((F, D)).astype(np.float32)
    hp.glue.set_index(db)
    sc, ix = hp.glue.search(q, 8)
    sc_ref, ix_ref = pr.search_l2(q, db, 8)
    _check_neighbours(sc_ref, ix_ref, sc, ix, gap=1e-3 * max(1.0, float(np.abs(sc_ref).max())) * 1e-2)


def test_search_golden(hp, gold):
    hp.glue.set_index(gold["search_db"])
    sc, ix = hp.glue.search(gold["search_q"], 8)
    np.testing.assert_array_equal(ix, gold["search_inds"])
    np.testing.assert_allclose(sc, gold["search_scores"], rtol=1e-5, atol=1e-4)


def test_search_l2_and_feature_index_surface():
    from rvc_hip.pipeline import HipFeatureIndex, search_l2

    rng = np.random.default_rng(7)
    db = rng.standard_normal((300, 20)).astype(np.float32)
    q = rng.standard_normal((11, 20)).astype(np.float32)
    sc, ix = search_l2(q, db, k=8)
    sc_ref, ix_ref = pr.search_l2(q, db, 8)
    np.testing.assert_array_equal(ix, ix_ref)
    idx = HipFeatureIndex(db)
    assert idx.ntotal == 300 and idx.dim == 20 and idx.metric == "L2"
    sc2, ix2 = idx.search(q, 3)
    np.testing.assert_array_equal(ix2, ix_ref[:, :3])
    np.testing.assert_array_equal(idx.reconstruct_n(10, 2), db[10:12])
    sc3, ix3 = search_l2(q, db[:4], k=8)  # fewer rows than k
    assert ix3.shape == (11, 4)
    np.testing.assert_array_equal(ix3, pr.search_l2(q, db[:4], 8)[1])


@pytest.mark.parametrize("case", ["a", "b", "c", "d"])
def test_vc_prepare_golden(hp, gold, case):
    from rvc_hip.pipeline import HipFeatureIndex

    g = lambda k: gold[f"prep_{case}_{k}"]  # noqa: E731
    rate, protect = (float(v) for v in g("params"))
    index = HipFeatureIndex(g("vecs"))
    res = hp._vc_prepare(None, 0, np.zeros(160, np.float32), g("pitch"), g("pitchf"), [0.0, 0.0, 0.0], index, None,
                         rate, 2, protect, feats=g("feats"))
    np.testing.assert_array_equal(res["pitch"], g("out_pitch"))
    np.testing.assert_array_equal(res["pitchf"], g("out_pitchf"))
    assert res["feats"].shape == g("out_feats").shape
    np.testing.assert_allclose(res["feats"], g("out_feats"), rtol=1e-5, atol=1e-5)


def test_vc_prepare_full_width(hp):
    rng = np.random.default_rng(11)
    F, D, N = 499, 768, 20000
    feats = rng.standard_normal((1, F, D)).astype(np.float32)
    vecs = rng.standard_normal((N, D)).astype(np.float32)
    pitch = rng.integers(1, 256, size=(1, 2 * F - 1)).astype(np.int64)
    pitchf = rng.uniform(0, 400, size=(1, 2 * F - 1)).astype(np.float32)
    pitchf[0, ::7] = 0.0
    from rvc_hip.pipeline import HipFeatureIndex

    ref, rp, rpf = pr.vc_prepare(feats, pitch, pitchf, vecs, 0.75, 0.33)
    res = hp._vc_prepare(None, 0, np.zeros(160, np.float32), pitch, pitchf, None, HipFeatureIndex(vecs), None, 0.75,
                         2, 0.33, feats=feats)
    np.testing.assert_array_equal(res["pitch"], rp)
    np.testing.assert_allclose(res["feats"], ref, rtol=1e-5, atol=1e-5)


def test_vc_prepare_without_retrieval_is_bit_exact(hp):
    rng = np.random.default_rng(12)
    F, D = 300, 768
    feats = rng.standard_normal((1, F, D)).astype(np.float32)
    pitch = rng.integers(1, 256, size=(1, 2 * F + 3)).astype(np.int64)
    pitchf = rng.uniform(-1, 3, size=(1, 2 * F + 3)).astype(np.float32)
    for protect in (0.33, 0.5):
        ref, _, _ = pr.vc_prepare(feats, pitch, pitchf, None, 0.0, protect)
        res = hp._vc_prepare(None, 0, np.zeros(160, np.float32), pitch, pitchf, None, None, None, 0.0, 2, protect,
                             feats=feats)
        np.testing.assert_array_equal(res["feats"], ref)


def test_vc_prepare_dev_matches_host(hp):
    from rvc_hip.hip_ops import get_context

    ctx = get_context()
    rng = np.random.default_rng(13)
    F, D, N = 64, 256, 999
    feats = rng.standard_normal((F, D)).astype(np.float32)
    pitchf = rng.uniform(0, 300, size=2 * F).astype(np.float32)
    hp.glue.set_index(rng.standard_normal((N, D)).astype(np.float32))
    host = hp.glue.prepare(feats, 0.5, pitchf, 0.3)
    fi, pi, oi = ctx.upload(feats), ctx.upload(pitchf), ctx.alloc(2 * F * D)
    try:
        hp.glue.prepare_dev(fi, F, D, 0.5, pi, 0.3, oi)
        np.testing.assert_array_equal(ctx.download(oi, (2 * F, D)), host)
    finally:
        for b in (fi, pi, oi):
            ctx.free(b)


@pytest.mark.parametrize("case", ["a", "b", "c"])
def test_change_rms_golden(hp, gold, case):
    sr1, sr2, rate = gold[f"rms_{case}_params"]
    out = hp.change_rms(gold[f"rms_{case}_d1"], gold[f"rms_{case}_d2"], int(sr1), int(sr2), float(rate))
    np.testing.assert_allclose(out, gold[f"rms_{case}_out"], rtol=1e-5, atol=1e-7)


def test_change_rms_full_size(hp):
    rng = np.random.default_rng(14)
    d1 = (rng.standard_normal(160000) * 0.1).astype(np.float32)
    d2 = (rng.standard_normal(400000) * np.linspace(0.02, 0.6, 400000)).astype(np.float32)
    for rate in (0.25, 1.0):
        np.testing.assert_allclose(hp.change_rms(d1, d2, 16000, 40000, rate), pr.change_rms(d1, d2, 16000, 40000,
                                                                                             rate),
                                   rtol=1e-5, atol=1e-7)
    np.testing.assert_array_equal(hp.change_rms(d1, d2[:0], 16000, 40000, 0.5), d2[:0])


def test_to_int16_bit_exact(hp):
    rng = np.random.default_rng(15)
    for scale in (0.3, 2.5):
        x = (rng.standard_normal(400000) * scale).astype(np.float32)
        np.testing.assert_array_equal(hp.to_int16(x), pr.to_int16(x))


def test_errors_are_reported(hp):
    from rvc_hip.pipeline import HipVcGlue

    g = HipVcGlue()
    try:
        with pytest.raises(ValueError):
            g.search(np.zeros((2, 4), np.float32))
        g.set_index(np.ones((3, 4), np.float32))
        with pytest.raises(ValueError):
            g.search(np.zeros((2, 5), np.float32))
        with pytest.raises(RuntimeError, match="index width"):
            g.prepare(np.zeros((2, 5), np.float32), 0.5)
    finally:
        g.close()
    with pytest.raises(NotImplementedError):
        class _Ivf:
            ntotal = 3
            vectors_by_rows = staticmethod(lambda ix: ix)
        hp._vc_prepare(None, 0, np.zeros(160, np.float32), None, None, None, _Ivf(), None, 0.5, 2, 0.5,
                       feats=np.zeros((1, 2, 4), np.float32))
