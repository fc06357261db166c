# -*- coding: utf-8 -*-
"""Write golden vectors for the conversion glue by running the reference.

Run ONLY in the build container, where the reference is mounted read-only at
``/root/reference`` (override with ``RVC_REFERENCE_ROOT``)::

    python tests/golden/make_golden_pipeline.py

It imports ``runtime.pipeline`` and ``runtime.retrieval`` from the reference
and records inputs and outputs of
  * ``Pipeline._vc_prepare`` (``runtime/pipeline.py:488-614``) with features
    given and a ``FeatureIndex`` (the retrieval blend, 2x interpolation,
    pitch alignment and protect mask, whose composition only the reference's
    own code pins);
  * ``search_l2`` (``runtime/retrieval.py:35-83``);
  * ``change_rms`` (``runtime/pipeline.py:164-188``);
into ``pipeline_glue.npz`` next to this script.  All inputs are seeded random
data; no reference source travels with the fixture.
"""

from __future__ import annotations

import os
import sys
import types

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("RVC_REFERENCE_ROOT", "/root/reference")


def _import_reference():
    os.environ["RVC_BACKEND"] = "numpy"
    sys.path.insert(0, REF)
    from runtime import pipeline, retrieval  # noqa: PLC0415

    return pipeline, retrieval


def _pitchf(rng, n):
    f = rng.uniform(80.0, 400.0, size=(1, n)).astype(np.float32)
    f[0, rng.random(n) < 0.25] = 0.0          # unvoiced
    f[0, rng.random(n) < 0.1] = 0.5           # in (0, 1): protect branch after the > 0 branch
    return f


def main():
    pipeline, retrieval = _import_reference()
    rng = np.random.default_rng(20261202)
    out = {}
    me = types.SimpleNamespace(window=160)
    cases = [
        # name, F, D, N, index_rate, protect, P (pitch frames before alignment)
        ("a", 37, 64, 300, 0.75, 0.33, 72),   # pad pitch (72 < 74)
        ("b", 25, 64, 300, 0.0, 0.5, 53),     # no retrieval, no protect, truncate pitch
        ("c", 19, 48, 5, 0.6, 0.2, 38),       # N < 8: k = 5
        ("d", 1, 32, 40, 1.0, 0.1, 2),        # one frame, index_rate 1
    ]
    for name, F, D, N, rate, protect, P in cases:
        feats = rng.standard_normal((1, F, D)).astype(np.float32)
        vecs = rng.standard_normal((N, D)).astype(np.float32)
        pitch = rng.integers(1, 256, size=(1, P)).astype(np.int64)
        pitchf = _pitchf(rng, P)
        idx = retrieval.FeatureIndex(dim=D)
        idx.add(vecs)
        audio0 = np.zeros(160 * 2 * F, dtype=np.float32)
        res = pipeline.Pipeline._vc_prepare(me, None, 0, audio0, pitch.copy(), pitchf.copy(), [0.0, 0.0, 0.0],
                                            idx, idx.reconstruct_n(0, idx.ntotal), rate, 2, protect,
                                            feats=feats.copy(), retrieval_mode="ivf", brute_mix=0.0)
        for k, v in (("feats", feats), ("vecs", vecs), ("pitch", pitch), ("pitchf", pitchf)):
            out[f"prep_{name}_{k}"] = v
        out[f"prep_{name}_params"] = np.array([rate, protect], dtype=np.float64)
        out[f"prep_{name}_out_feats"] = np.asarray(res["feats"], dtype=np.float32)
        out[f"prep_{name}_out_pitch"] = np.asarray(res["pitch"])
        out[f"prep_{name}_out_pitchf"] = np.asarray(res["pitchf"], dtype=np.float32)

    q = rng.standard_normal((20, 32)).astype(np.float32)
    db = rng.standard_normal((400, 32)).astype(np.float32)
    sc, ix = retrieval.search_l2(q, db, k=8)
    out.update(search_q=q, search_db=db, search_scores=sc, search_inds=ix)

    for name, n1, n2, sr2, rate in (("a", 16000, 41000, 40000, 0.25), ("b", 8001, 24000, 48000, 0.0),
                                    ("c", 8000, 20500, 40000, 0.75)):
        d1 = (rng.standard_normal(n1) * 0.1).astype(np.float32)
        d2 = (rng.standard_normal(n2) * np.linspace(0.01, 0.5, n2)).astype(np.float32)
        r = pipeline.change_rms(d1, d2, 16000, sr2, rate)
        out.update({f"rms_{name}_d1": d1, f"rms_{name}_d2": d2,
                    f"rms_{name}_params": np.array([16000, sr2, rate], dtype=np.float64),
                    f"rms_{name}_out": np.asarray(r, dtype=np.float32)})

    np.savez_compressed(os.path.join(HERE, "pipeline_glue.npz"), **out)
    print("wrote", os.path.join(HERE, "pipeline_glue.npz"), len(out), "arrays")


if __name__ == "__main__":
    main()
