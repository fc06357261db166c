# -*- coding: utf-8 -*-
"""Write RMVPE golden vectors by running the reference's own numpy RMVPE.

Run ONLY in the build container, where the reference is mounted read-only at
``/root/reference`` (override with ``RVC_REFERENCE_ROOT``)::

    python tests/golden/make_golden_rmvpe.py

``RMVPE.__init__`` reads ``rmvpe.pt``; random-init weights
(``rvc_hip.synthetic.make_rmvpe_weights``) replace it, so the object is
assembled with ``__new__`` and the attributes ``__init__`` sets
(``runtime/models/rmvpe.py:557-592``: float32 weights, the HTK mel basis,
the padded cents table, the BatchNorm scale/shift cache) are filled in with
the reference's own functions.  The numpy paths are forced (conv2d on numpy,
host BiGRU).  Stored: inputs, log-mel, salience and f0 of two clips, the mel
basis, and ``RMVPE.decode`` on crafted salience (ties, edge bins, silent
frames).  Weights are regenerated from the seed and checked by digest.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "rvc-vulkan_amd"))

from rvc_hip import synthetic as syn  # noqa: E402

REF = os.environ.get("RVC_REFERENCE_ROOT", "/root/reference")
WSEED = 3
CLIPS = ((8000, 1), (4000, 2))


def crafted_salience(rng):
    s = rng.uniform(0.0, 0.5, size=(12, 360)).astype(np.float32)
    s[0, 0] = 0.9                      # argmax at the first bin (left padding)
    s[1, 359] = 0.9                    # argmax at the last bin (right padding)
    s[2, 100] = s[2, 200] = 0.95       # tie: the first maximum wins
    s[3] = 0.02                        # silent: max <= 0.03
    s[4] = 0.03                        # exactly at the threshold: silent
    s[5, 180] = 0.0301                 # just above the threshold
    s[5, s[5] > 0.0301] = 0.0
    s[6, 3] = 0.8                      # window partly in the padding
    s[7, 356] = 0.8
    s[8] = 0.0
    s[8, 50] = 0.5                     # single nonzero bin
    return s


def main():
    os.environ["RVC_BACKEND"] = "numpy"
    os.environ["RVC_RMVPE_CONV"] = "numpy"
    os.environ["RVC_RMVPE_GRU_GPU"] = "0"
    os.environ["RVC_RMVPE_NUMBA"] = "0"
    sys.path.insert(0, REF)
    from runtime.dsp.mel import mel_filter_bank  # noqa: PLC0415
    from runtime.models import rmvpe  # noqa: PLC0415

    w = syn.make_rmvpe_weights(WSEED)
    m = rmvpe.RMVPE.__new__(rmvpe.RMVPE)
    m.W = {k: v.astype(np.float32) for k, v in w.items()}
    m.mel_basis = mel_filter_bank(16000, 1024, 128, 30.0, 8000.0).astype(np.float32)
    m.cents_mapping = np.pad(20 * np.arange(360) + 1997.3794084376191, (4, 4)).astype(np.float32)
    m._bn_cache = {}
    for k in list(m.W):
        if k.endswith(".weight"):
            p = k[: -len(".weight")]
            if p + ".bias" in m.W and p + ".running_mean" in m.W and p + ".running_var" in m.W:
                m._bn_cache[p] = rmvpe._bn_scale_shift(m.W, p)
    m._load_time = 0.0
    m._unet_batch_flag = False

    out = {"weights_digest": np.array(syn.weights_digest(w)), "wseed": np.array(WSEED),
           "mel_basis": m.mel_basis}
    for i, (T, seed) in enumerate(CLIPS):
        x = syn.make_rmvpe_audio(T, seed)
        mel = m._extract_mel(x)
        hidden = m.mel2hidden(mel)
        f0 = m.decode(hidden[0], thred=0.03)
        out[f"x{i}"] = x
        out[f"mel{i}"] = mel[0]
        out[f"hidden{i}"] = hidden[0].astype(np.float32)
        out[f"f0_{i}"] = np.asarray(f0, dtype=np.float32)
        # infer_from_audio itself (single-threaded BLAS there: float32 sums
        # in another order, so equal to rounding, not bit for bit)
        np.testing.assert_allclose(m.infer_from_audio(x, thred=0.03), f0, rtol=1e-5)
    sal = crafted_salience(np.random.default_rng(9))
    out["dec_sal"] = sal
    out["dec_cents"] = np.asarray(m.to_local_average_cents(sal, thred=0.03), dtype=np.float32)
    out["dec_f0"] = np.asarray(m.decode(sal, thred=0.03), dtype=np.float32)
    path = os.path.join(HERE, "rmvpe.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: getattr(v, "shape", None) for k, v in out.items()})


if __name__ == "__main__":
    main()
