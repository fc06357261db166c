# -*- coding: utf-8 -*-
"""Write HuBERT golden vectors by running the reference's own numpy encoder.

Run ONLY in the build container, where the reference is mounted read-only at
``/root/reference`` (override with ``RVC_REFERENCE_ROOT``)::

    RVC_BACKEND=numpy python tests/golden/make_golden_hubert.py

``HubertEncoder.__init__`` reads ``pytorch_model.bin``; random-init weights
replace it here, so the loader's weight-norm step for the positional conv is
reproduced by calling the reference's own formula on the same arrays
(``runtime/models/hubert.py:510-522``) and the encoder object is assembled
with ``__new__``.  Inputs and outputs are stored; weights are regenerated
from ``(HUBERT_BASE, seed)`` and checked by SHA-256 digest.  Nothing here
runs on the GPU box and no reference source travels with the fixtures.
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
WSEED = 5


def _import_reference():
    os.environ["RVC_BACKEND"] = "numpy"
    sys.path.insert(0, REF)
    from runtime.models import hubert  # noqa: PLC0415

    return hubert


def _encoder(hubert, sd):
    """The object ``HubertEncoder.__init__`` would build, from a state dict:
    ``_load_and_prepare``'s steps on in-memory arrays."""
    o0 = sd["encoder.pos_conv_embed.conv.weight_g"]
    o1 = sd["encoder.pos_conv_embed.conv.weight_v"]
    norm = np.sqrt(np.sum(o1.astype(np.float64) ** 2, axis=(0, 1), keepdims=True))
    pos_w = (o0 * (o1 / norm.astype(np.float32))).astype(np.float32)
    layers = {
        "proj_ln": (sd["feature_projection.layer_norm.weight"], sd["feature_projection.layer_norm.bias"]),
        "proj": (sd["feature_projection.projection.weight"], sd["feature_projection.projection.bias"]),
        "enc_ln": (sd["encoder.layer_norm.weight"], sd["encoder.layer_norm.bias"]),
        "pos_conv": (pos_w, sd["encoder.pos_conv_embed.conv.bias"]),
        "final_proj": (sd["final_proj.weight"], sd["final_proj.bias"]),
        "conv": [(sd[f"feature_extractor.conv_layers.{i}.conv.weight"], None) for i in range(7)],
        "conv_gamma": sd["feature_extractor.conv_layers.0.layer_norm.weight"],
        "conv_beta": sd["feature_extractor.conv_layers.0.layer_norm.bias"],
        "enc_layers": [],
    }
    for i in range(12):
        p = f"encoder.layers.{i}."
        layers["enc_layers"].append({
            "attn": {nm: (sd[p + f"attention.{pn}.weight"], sd[p + f"attention.{pn}.bias"])
                     for nm, pn in (("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "out_proj"))},
            "ln1": (sd[p + "layer_norm.weight"], sd[p + "layer_norm.bias"]),
            "ff": {"wi": (sd[p + "feed_forward.intermediate_dense.weight"],
                          sd[p + "feed_forward.intermediate_dense.bias"]),
                   "wo": (sd[p + "feed_forward.output_dense.weight"], sd[p + "feed_forward.output_dense.bias"])},
            "ln2": (sd[p + "final_layer_norm.weight"], sd[p + "final_layer_norm.bias"]),
        })
    enc = hubert.HubertEncoder.__new__(hubert.HubertEncoder)
    enc.model_dir = ""
    enc._sd = sd
    enc._layers = layers
    enc._prof = None
    enc._prof_layers = None
    return enc


def main():
    hubert = _import_reference()
    sd = syn.make_hubert_weights(syn.HUBERT_BASE, seed=WSEED)
    enc = _encoder(hubert, sd)
    out = {"digest": np.array(syn.weights_digest(sd)), "wseed": np.array(WSEED)}
    for T in (1600, 4000):
        x = syn.make_hubert_input(T, seed=T)
        feats = enc._feature_extractor(x)               # [1, L, 512]
        proj = enc._feature_projection(feats)           # [1, L, 768]
        hs = enc._encoder(proj)                         # [13, 1, L, 768]
        out[f"T{T}_x"] = x
        out[f"T{T}_feats"] = feats
        out[f"T{T}_proj"] = proj
        out[f"T{T}_entry"] = hs[0]
        out[f"T{T}_layer1"] = hs[1]
        out[f"T{T}_v2"] = enc.encode(x, version=2)
        out[f"T{T}_v1"] = enc.encode(x, version=1)
        gl = np.linspace(-6, 6, 97, dtype=np.float32)
        out["gelu_x"] = gl
        out["gelu_y"] = hubert.gelu_erf(gl)
    path = os.path.join(HERE, "hubert_base.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
