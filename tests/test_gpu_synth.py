# -*- coding: utf-8 -*-
"""End-to-end parity of the device-resident synthesizer (GPU).

Against the reference's own outputs (golden vectors) and the numpy oracle on
identical seeded inputs and random-init weights: waveform max-abs <= 1e-3,
intermediates rel L2 <= 1e-4 (BASELINE.json north_star tolerances).  The
BASELINE shapes are checked against the oracle at full size -- config 2
(P = 1000: enc_p output, flow output and waveform; the attention's key-split
path), config 4 (48k, 8 chunks of P = 600 as one batch) -- with the oracle's
"taps" conv formulation (the same mathematics as the reference's einsum form
in another summation order, pinned against it on the CPU), plus the
size-independent properties: determinism, batch == per-chunk bit identity,
finiteness and |wave| <= 1."""

from __future__ import annotations

import math
import os

import numpy as np
import pytest

from conftest import GOLDEN, rel_l2
from oracle import nn_ref as nn
from oracle import vits_ref as V
from rvc_hip import synthetic as syn

pytestmark = pytest.mark.gpu

WAVE_TOL = 1e-3
OP_TOL = 1e-4
GEOMS = {"tiny": syn.GEOM_TINY, "40k": syn.GEOM_40K, "48k": syn.GEOM_48K}


def _hip_synth(w, config=None, sr=None):
    from rvc_hip import _hip
    from rvc_hip.synth import HipSynthesizer

    assert _hip.has_so, _hip.so_load_error
    return HipSynthesizer(w, config=config, sr=sr)


@pytest.mark.parametrize("name", ["synth_tiny_P8.npz", "synth_40k_P12.npz", "synth_48k_P10.npz"])
def test_golden_end_to_end(name):
    d = np.load(os.path.join(GOLDEN, name))
    geom = GEOMS[name.split("_")[1]]
    w = syn.make_weights(geom, seed=int(d["wseed"]))
    assert syn.weights_digest(w) == str(d["digest"])
    cfg = geom.config_array() if bool(d["use_config"]) else None
    s = _hip_synth(w, config=cfg, sr=None if cfg is not None else geom.sr)
    wave = s.infer_controlled(d["phone"], d["pitch"], d["nsff0"], d["sid"], d["nz"], d["ns"])
    assert wave.shape == d["wave"].shape
    assert np.abs(wave - d["wave"]).max() <= WAVE_TOL
    dw = s.dec_forward(d["dec_z"], d["dec_f0"], d["dec_g"], d["dec_ns"])
    assert np.abs(dw - d["dec_wave"]).max() <= WAVE_TOL


def test_golden_encoder_and_flow():
    d = np.load(os.path.join(GOLDEN, "enc_flow_40k.npz"))
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=int(d["seed"]))
    s = _hip_synth(w, sr=geom.sr)
    ref = V.Synthesizer(w, sr=geom.sr)
    H = geom.hidden
    for P in (5, 40):
        nz = np.zeros((1, H, P), np.float32)
        ns = np.zeros((1, P * geom.upp), np.float32)
        f0 = np.zeros((1, P), np.float32)
        s.infer_controlled(d[f"P{P}_phone"], d[f"P{P}_pitch"], f0, np.array([0]), nz, ns)
        assert rel_l2(s.read("enc_in", (1, H, P)), d[f"P{P}_enc_in"].transpose(0, 2, 1)) < OP_TOL
        assert rel_l2(s.read("enc_out", (1, H, P)), d[f"P{P}_enc_out"].transpose(0, 2, 1)) < OP_TOL
        st = s.read("stats", (1, 2 * H, P))
        assert rel_l2(st[:, :H], d[f"P{P}_m"]) < OP_TOL
        assert rel_l2(st[:, H:], d[f"P{P}_logs"]) < OP_TOL
        # flow in isolation: the oracle's reverse flow applied to the HIP z_p
        zp = s.read("z_p", (1, H, P))
        g = ref.resolve_g(np.array([0]))
        assert rel_l2(s.read("z", (1, H, P)), ref.flow.reverse(zp, np.ones((1, 1, P), np.float32), g)) < OP_TOL


def test_intermediates_vs_oracle_40k():
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=4)
    s = _hip_synth(w, sr=geom.sr)
    s.set_debug(True)
    ref = V.Synthesizer(w, sr=geom.sr)
    P = 40
    inp = syn.make_synth_inputs(geom, P, seed=77)
    wave = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    z, g = ref.enc_flow(inp["phone"], inp["pitch"], inp["sid"], inp["nz"])
    H = geom.hidden
    assert rel_l2(s.read("z", (1, H, P)), z) < OP_TOL
    # decoder stages from the HIP z (isolates the decoder from enc/flow drift)
    zh = s.read("z", (1, H, P))
    d = ref.dec
    har = d.sine_gen(inp["nsff0"], inp["ns"])
    assert rel_l2(s.read("har", (1, P * geom.upp)), har.reshape(1, -1)) < OP_TOL
    x = nn.conv1d(zh, w["dec.conv_pre.weight"], w["dec.conv_pre.bias"], padding=3) + \
        nn.conv1d(g, w["dec.cond.weight"], w["dec.cond.bias"])
    assert rel_l2(s.read("dec_pre", x.shape), x) < OP_TOL
    cfg = ref.cfg
    for i in range(cfg.n_ups):
        xh = s.read(f"dec_stage{i - 1}", x.shape) if i > 0 else x
        y = nn.leaky_relu(xh, 0.1)
        up = f"dec.ups.{i}"
        y = nn.conv_transpose1d(y, V.deweight_norm(w[up + ".weight_v"], w[up + ".weight_g"]), w[up + ".bias"],
                                stride=cfg.upsample_rates[i],
                                padding=(cfg.upsample_kernels[i] - cfg.upsample_rates[i]) // 2)
        y = y + nn.conv1d(har, w[f"dec.noise_convs.{i}.weight"], w[f"dec.noise_convs.{i}.bias"],
                          stride=cfg.noise_strides[i], padding=cfg.noise_strides[i] // 2)
        xs = None
        for j, k in enumerate((3, 7, 11)):
            o = V.resblock1(w, f"dec.resblocks.{3 * i + j}", k, y)
            xs = o if xs is None else xs + o
        x = xs / 3
        assert rel_l2(s.read(f"dec_stage{i}", x.shape), x) < OP_TOL, f"stage {i}"
    want = ref.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    assert np.abs(wave - want).max() <= WAVE_TOL


def test_config1_decoder_full_size():
    """40k GeneratorNSF alone, P=200 (2 s), B=1."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    s = _hip_synth(w, sr=geom.sr)
    inp = syn.make_dec_inputs(geom, 200, seed=1)
    wave = s.dec_forward(inp["z"], inp["f0"], inp["g"], inp["ns"])
    want = V.GeneratorNSF(w, V.VitsConfig(w, sr=geom.sr)).forward(inp["z"], inp["f0"], inp["g"], inp["ns"])
    assert wave.shape == (1, 1, 80000)
    assert np.abs(wave - want).max() <= WAVE_TOL


def test_decoder_P400_vs_oracle():
    """4 s decode (P=400): stages 1-3 run on the persistent MFMA kernel
    (ResBlock conv1 with leaky input, conv2 with the prefetched residual)."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=2)
    s = _hip_synth(w, sr=geom.sr)
    inp = syn.make_dec_inputs(geom, 400, seed=12)
    wave = s.dec_forward(inp["z"], inp["f0"], inp["g"], inp["ns"])
    want = V.GeneratorNSF(w, V.VitsConfig(w, sr=geom.sr)).forward(inp["z"], inp["f0"], inp["g"], inp["ns"])
    assert wave.shape == (1, 1, 160000)
    assert np.abs(wave - want).max() <= WAVE_TOL


def test_batch_equals_per_chunk_and_determinism():
    geom = syn.GEOM_48K
    w = syn.make_weights(geom, seed=6)
    s = _hip_synth(w, sr=geom.sr)
    P = 30
    ins = [syn.make_dec_inputs(geom, P, seed=50 + i) for i in range(3)]
    outs = s.dec.decode_batch([i["z"] for i in ins], ins[0]["g"], [i["f0"] for i in ins], [i["ns"] for i in ins])
    for i, o in zip(ins, outs):
        one = s.dec_forward(i["z"], i["f0"], ins[0]["g"], i["ns"])
        np.testing.assert_array_equal(o, one)
    again = s.dec_forward(ins[0]["z"], ins[0]["f0"], ins[0]["g"], ins[0]["ns"])
    np.testing.assert_array_equal(again, outs[0])


def test_full_size_10s_properties():
    """BASELINE config 2 size (P=1000): deterministic, finite, in tanh range,
    and the first second equal to a 1 s run of the same inputs up to the
    decoder's receptive-field boundary (attention is global, so the encoder
    is compared through the oracle at P=100 instead)."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    s = _hip_synth(w, sr=geom.sr)
    P = 1000
    inp = syn.make_synth_inputs(geom, P, seed=3)
    a = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    b = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    assert a.shape == (1, 1, 400000)
    np.testing.assert_array_equal(a, b)
    assert np.isfinite(a).all() and np.abs(a).max() <= 1.0
    assert 0.01 < float(a.std()) < 0.99
    # decoder-only locality: frames [0, 100) of a P=1000 decode equal a P=116 decode's first 100 frames
    d = syn.make_dec_inputs(geom, P, seed=4)
    full = s.dec_forward(d["z"], d["f0"], d["g"], d["ns"])
    Q = 116
    part = s.dec_forward(d["z"][:, :, :Q], d["f0"][:, :Q], d["g"], d["ns"][:, :Q * geom.upp])
    n = 100 * geom.upp
    # the sine phase of frame p depends only on frames < p, so the prefix is identical math
    assert np.abs(full[..., :n] - part[..., :n]).max() <= 1e-5


def test_end_to_end_1s_vs_oracle():
    """Full-width 40k synthesis of 1 s (P=100) against the oracle."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    s = _hip_synth(w, sr=geom.sr)
    inp = syn.make_synth_inputs(geom, 100, seed=9)
    wave = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    want = V.Synthesizer(w, sr=geom.sr).infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"],
                                                        inp["nz"], inp["ns"])
    assert np.abs(wave - want).max() <= WAVE_TOL
    assert math.isfinite(float(wave.sum()))


def _oracle_enc_out(ref, geom, phone, pitch):
    """enc_p output [1,H,P] of the oracle (runtime/models/vits.py:2566-2578)."""
    x = ref.enc_p.embed(phone, pitch) * math.sqrt(geom.hidden)
    x = nn.leaky_relu(x, 0.1)
    P = phone.shape[1]
    return ref.enc_p.encode(x, np.ones((1, 1, P), np.float32)).transpose(0, 2, 1)


def test_config2_full_size_vs_oracle():
    """BASELINE config 2 (40k, P = 1000, B = 1) against the oracle: the
    encoder output (its attention runs key-split at this length), the flow
    output and the 400 000-sample waveform."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    s = _hip_synth(w, sr=geom.sr)
    ref = V.Synthesizer(w, sr=geom.sr)
    P, H = 1000, geom.hidden
    inp = syn.make_synth_inputs(geom, P, seed=3)
    wave = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    enc_out = s.read("enc_out", (1, H, P))
    z = s.read("z", (1, H, P))
    assert rel_l2(enc_out, _oracle_enc_out(ref, geom, inp["phone"], inp["pitch"])) < OP_TOL
    with nn.conv_formulation("taps"):
        zr, g = ref.enc_flow(inp["phone"], inp["pitch"], inp["sid"], inp["nz"])
        assert rel_l2(z, zr) < OP_TOL
        want = ref.dec.forward(zr, inp["nsff0"], g, inp["ns"])
    assert wave.shape == want.shape == (1, 1, 400000)
    assert np.abs(wave - want).max() <= WAVE_TOL


def test_config4_48k_batch8_P600():
    """48k GeneratorNSF, 8 chunks of P = 600 as one batch.
    Every chunk equals its own single-chunk decode bit for bit; the batch is
    finite and in tanh range; chunk 5 against the oracle."""
    geom = syn.GEOM_48K
    w = syn.make_weights(geom, seed=6)
    s = _hip_synth(w, sr=geom.sr)
    P, B = 600, 8
    ins = [syn.make_dec_inputs(geom, P, seed=400 + i) for i in range(B)]
    z = np.concatenate([i["z"] for i in ins])
    f0 = np.concatenate([i["f0"] for i in ins])
    g = np.concatenate([i["g"] for i in ins])
    ns = np.concatenate([i["ns"].reshape(1, -1) for i in ins])
    batch = s.dec_forward(z, f0, g, ns)
    assert batch.shape == (B, 1, P * geom.upp) == (8, 1, 288000)
    assert np.isfinite(batch).all() and np.abs(batch).max() <= 1.0
    for i in range(B):
        one = s.dec_forward(ins[i]["z"], ins[i]["f0"], ins[i]["g"], ins[i]["ns"])
        np.testing.assert_array_equal(batch[i:i + 1], one)
    gen = V.GeneratorNSF(w, V.VitsConfig(w, sr=geom.sr))
    with nn.conv_formulation("taps"):
        want = gen.forward(ins[5]["z"], ins[5]["f0"], ins[5]["g"], ins[5]["ns"])
    assert np.abs(batch[5:6] - want).max() <= WAVE_TOL


def test_infer_batch_equals_per_chunk_at_key_split_lengths():
    """Two P = 256 chunks (attention key-split > 1 at this length) as a batch
    of 2 equal the same chunks run one by one, bit for bit: the split count
    and every tile depend on the chunk shape only, never on B."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=1)
    s = _hip_synth(w, sr=geom.sr)
    P = 256
    ins = [syn.make_synth_inputs(geom, P, seed=70 + i) for i in range(2)]
    cat = {k: np.concatenate([i[k] for i in ins]) for k in ("phone", "pitch", "nsff0", "sid", "nz", "ns")}
    both = s.infer_controlled(cat["phone"], cat["pitch"], cat["nsff0"], cat["sid"], cat["nz"], cat["ns"])
    for i, inp in enumerate(ins):
        one = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
        np.testing.assert_array_equal(both[i:i + 1], one)
