# -*- coding: utf-8 -*-
"""Write golden vectors by running the reference's own numpy path.

Run ONLY in the build container, where the reference is mounted read-only at
``/root/reference`` (override with ``RVC_REFERENCE_ROOT``)::

    RVC_BACKEND=numpy python tests/golden/make_golden.py

It imports ``runtime.models.vits`` from the reference with the numpy backend
forced, feeds it the seeded random-init weights of
``rvc_hip.synthetic.make_weights`` and seeded inputs, and stores the inputs
and outputs as small ``.npz`` files next to this script.  Weights are not
stored: tests regenerate them from ``(geometry, seed)`` and check the SHA-256
digest recorded in each fixture.  Nothing here runs on the GPU box and no
reference source travels with the fixtures.

Functions covered (the ones that only the reference's own code pins exactly):
``_GeneratorNSF._sine_gen`` float32 rounding, ``VitsConfig`` derivations,
``_TextEncoder.encode`` (P <= 11 slice branch and P > 11 pad branch),
``_FlowBlock.reverse``, ``_GeneratorNSF.forward`` and
``SynthesizerTrn.infer_controlled`` end to end (reduced width and full width,
40k and 48k geometries).
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "rvc-vulkan_amd"))

from rvc_hip import synthetic as syn  # noqa: E402

REF = os.environ.get("RVC_REFERENCE_ROOT", "/root/reference")


def _import_reference():
    os.environ["RVC_BACKEND"] = "numpy"
    os.environ.pop("RVC_FIXED_SEED", None)
    sys.path.insert(0, REF)
    from runtime.models import vits  # noqa: PLC0415

    return vits


def _synth(vits, w, config=None, sr=None):
    """A ``SynthesizerTrn`` built from a weight dict (its ``__init__`` needs a
    checkpoint path, so the same attributes are set directly)."""
    s = vits.SynthesizerTrn.__new__(vits.SynthesizerTrn)
    s._w = w
    s.cfg = vits.VitsConfig(w, config, sr=sr)
    s.enc_p = vits._TextEncoder(w, s.cfg)
    s.flow = vits._FlowBlock(w, s.cfg)
    s.dec = vits._GeneratorNSF(w, s.cfg)
    s.register_persistent_weights()
    return s


def _save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


def golden_sine(vits):
    geom = syn.GEOM_40K
    w = syn.make_weights(syn.GEOM_TINY, seed=11)  # only l_linear is read
    s = _synth(vits, w, sr=geom.sr)
    rng = np.random.default_rng(5)
    P = 16
    f0 = syn.make_f0(P, rng)
    f0_const = np.full((1, P), 220.0, dtype=np.float32)
    _, ns = syn.make_noise(geom, P, seed=5)
    har = s.dec._sine_gen(f0, ns)
    har_const = s.dec._sine_gen(f0_const, ns)
    off = s._phase_offsets(f0)
    _save("sine_gen.npz", f0=f0, f0_const=f0_const, ns=ns, har=har,
          har_const=har_const, phase_offsets=off,
          digest=np.array(syn.weights_digest(w)), seed=np.array(11),
          sr=np.array(geom.sr), upp=np.array(s.cfg.upp))


def golden_config(vits):
    cases = {}
    for name, geom, cfg, sr in [
        ("40k_sr", syn.GEOM_40K, None, 40000),
        ("40k_cfg", syn.GEOM_40K, syn.GEOM_40K.config_array(), None),
        ("48k_noconfig", syn.GEOM_48K, None, None),
        ("48k_cfg", syn.GEOM_48K, syn.GEOM_48K.config_array(), None),
        ("tiny_sr", syn.GEOM_TINY, None, 40000),
    ]:
        w = syn.make_weights(geom, seed=1)
        c = vits.VitsConfig(w, cfg, sr=sr)
        cases[name] = {
            "config": cfg, "sr_arg": sr,
            "geom": {"phone_dim": geom.phone_dim, "hidden": geom.hidden,
                     "filter_channels": geom.filter_channels, "n_heads": geom.n_heads,
                     "n_layers": geom.n_layers, "gin": geom.gin, "n_spk": geom.n_spk,
                     "upsample_initial": geom.upsample_initial,
                     "upsample_rates": geom.upsample_rates,
                     "upsample_kernels": geom.upsample_kernels, "sr": geom.sr},
            "derived": {k: getattr(c, k) for k in (
                "phone_dim", "hidden", "filter", "n_layers", "k_channels", "n_heads",
                "upsample_initial", "upsample_rates", "upsample_kernels", "sr", "n_ups",
                "upp", "noise_strides", "resblock_kernel_sizes", "n_spk", "gin_channels")},
        }
    path = os.path.join(HERE, "vits_config.json")
    with open(path, "w") as f:
        json.dump(cases, f, indent=1, sort_keys=True)
    print(f"wrote {path}")


def golden_encoder_flow(vits):
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=3)
    s = _synth(vits, w, sr=geom.sr)
    out = {"digest": np.array(syn.weights_digest(w)), "seed": np.array(3)}
    for P in (5, 40):
        inp = syn.make_synth_inputs(geom, P, seed=100 + P)
        x = s.enc_p.embed(inp["phone"], inp["pitch"])
        x = x * math.sqrt(s.cfg.hidden)
        x = vits.nn.leaky_relu(x, 0.1)
        mask = vits.nn.generate_mask(P)
        h = s.enc_p.encode(x, mask)
        m, logs = s.enc_p.stats(h)
        out[f"P{P}_phone"] = inp["phone"]
        out[f"P{P}_pitch"] = inp["pitch"]
        out[f"P{P}_enc_in"] = x
        out[f"P{P}_enc_out"] = h
        out[f"P{P}_m"] = m
        out[f"P{P}_logs"] = logs
    P = 40
    rng = np.random.default_rng(7)
    z_p = rng.standard_normal((1, geom.hidden, P)).astype(np.float32)
    g = s._resolve_g(np.array([1], dtype=np.int64))
    z = s.flow.reverse(z_p, vits.nn.generate_mask(P), g)
    out["flow_zp"] = z_p
    out["flow_sid"] = np.array([1], dtype=np.int64)
    out["flow_z"] = np.ascontiguousarray(z)
    _save("enc_flow_40k.npz", **out)


def golden_end_to_end(vits, geom, geom_name, P, seed, wseed, use_config):
    w = syn.make_weights(geom, seed=wseed)
    cfg = geom.config_array() if use_config else None
    s = _synth(vits, w, config=cfg, sr=None if use_config else geom.sr)
    inp = syn.make_synth_inputs(geom, P, seed=seed)
    wave = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"],
                              inp["nz"], inp["ns"])
    dec_in = syn.make_dec_inputs(geom, P, seed=seed + 1)
    dec_wave = s.dec.forward(dec_in["z"], dec_in["f0"], dec_in["g"], dec_in["ns"])
    _save(f"synth_{geom_name}_P{P}.npz",
          digest=np.array(syn.weights_digest(w)), wseed=np.array(wseed),
          seed=np.array(seed), use_config=np.array(bool(use_config)),
          phone=inp["phone"], pitch=inp["pitch"], nsff0=inp["nsff0"], sid=inp["sid"],
          nz=inp["nz"], ns=inp["ns"], wave=wave,
          dec_z=dec_in["z"], dec_g=dec_in["g"], dec_f0=dec_in["f0"], dec_ns=dec_in["ns"],
          dec_wave=dec_wave)


def main():
    vits = _import_reference()
    golden_sine(vits)
    golden_config(vits)
    golden_encoder_flow(vits)
    golden_end_to_end(vits, syn.GEOM_TINY, "tiny", P=8, seed=21, wseed=2, use_config=False)
    golden_end_to_end(vits, syn.GEOM_40K, "40k", P=12, seed=31, wseed=4, use_config=True)
    golden_end_to_end(vits, syn.GEOM_48K, "48k", P=10, seed=41, wseed=6, use_config=True)


if __name__ == "__main__":
    main()
