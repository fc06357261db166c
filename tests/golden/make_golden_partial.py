# -*- coding: utf-8 -*-
"""Write golden vectors for the noise draw and the partial-synthesis path by
running the reference's own numpy code.

Run ONLY in the build container, where the reference is mounted read-only at
``/root/reference`` (override with ``RVC_REFERENCE_ROOT``)::

    RVC_BACKEND=numpy python tests/golden/make_golden_partial.py

Functions covered (the ones only the reference's own code pins exactly):

* ``SynthesizerTrn._make_noise`` -- nz [1,h,P] drawn before ns [1,P*upp,1]
  from one ``RandomState(seed)`` (``runtime/models/vits.py:2337-2350``),
  including the ``RVC_FIXED_SEED`` substitution for ``seed=None``;
* ``SynthesizerTrn.infer(seed=...)`` end to end (``:2352-2402``);
* ``SynthesizerTrn._phase_offsets`` (``:2404-2414``);
* ``prep_dec`` for full and partial synthesis (``:2478-2500``, with
  ``_partial_prep`` ``:2416-2476`` and ``_full_prep``);
* ``decode_batch(preps)`` over chunks of unequal lengths (``:2502-2522``);
* ``infer(skip_head=..., return_length=...)`` (``:2524-2531``).

The geometry is the reduced-width tiny one (same structure as RVC v2 40k),
so the reference's numpy decoder finishes in seconds.  Weights are not stored:
tests regenerate them from ``(geometry, seed)`` and check the recorded
SHA-256 digest.  Nothing here runs on the GPU box.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from make_golden import _import_reference, _save, _synth, syn  # noqa: E402

WSEED = 8
P = 64
# (skip_head, return_length): head inside the left pads (zs = 0, flow_head = 0),
# in the middle, and reaching the end (ze clipped to P)
PARTS = [(4, 20), (30, 12), (50, 14)]


def main():
    vits = _import_reference()
    geom = syn.GEOM_TINY
    w = syn.make_weights(geom, seed=WSEED)
    s = _synth(vits, w, sr=geom.sr)
    inp = syn.make_synth_inputs(geom, P, seed=61)
    phone, pitch, nsff0, sid = inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"]
    out = {"digest": np.array(syn.weights_digest(w)), "wseed": np.array(WSEED),
           "phone": phone, "pitch": pitch, "nsff0": nsff0, "sid": sid,
           "seed": np.array(123), "parts": np.array(PARTS, dtype=np.int64)}

    nz, ns = s._make_noise(phone, 123)
    out["nz"], out["ns"] = nz, ns
    saved = vits._FIXED_SEED
    vits._FIXED_SEED = "77"  # what RVC_FIXED_SEED=77 sets at import time
    try:
        fz, fs = s._make_noise(phone, None)
    finally:
        vits._FIXED_SEED = saved
    out["fixed77_nz"], out["fixed77_ns"] = fz, fs

    out["wave"] = s.infer(phone, pitch, nsff0, sid, seed=123)
    out["phase_offsets"] = s._phase_offsets(nsff0)

    preps = [s.prep_dec(phone, pitch, nsff0, sid, seed=123)]
    for i, (head, length) in enumerate(PARTS):
        out[f"part{i}_wave"] = s.infer(phone, pitch, nsff0, sid, seed=123, skip_head=head,
                                       return_length=length)
        p = s.prep_dec(phone, pitch, nsff0, sid, seed=123, skip_head=head, return_length=length)
        for k in ("z_seg", "nsff0_seg", "ns_seg", "off"):
            out[f"part{i}_{k}"] = np.asarray(p[k])
        out[f"part{i}_s0"] = np.array(p["s0"])
        out[f"part{i}_n_out"] = np.array(p["n_out"])
        preps.append(p)
    out["full_z"] = np.asarray(preps[0]["z_seg"])
    out["full_g"] = np.asarray(preps[0]["g"])
    waves = s.decode_batch(preps)
    for i, wv in enumerate(waves):
        out[f"batch{i}_wave"] = np.asarray(wv)
    _save("synth_partial_tiny.npz", **out)


if __name__ == "__main__":
    main()
