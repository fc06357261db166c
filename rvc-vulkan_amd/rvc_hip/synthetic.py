# -*- coding: utf-8 -*-
"""Seeded random-init weights and synthetic inputs for the RVC synthesis path.

There are no real checkpoints offline, so every parity test and the benchmark
run on random-init weights that follow the checkpoint key/shape schema the
reference consumes (``runtime/models/vits.py:166-277`` derives the geometry
from these shapes; key list at ``runtime/models/vits.py:2272-2334`` and
``:1426-1466``).

Init choices (the reference only says "random-init"; these keep activations
non-saturated so every op is exercised):

* weight-norm layers (``dec.ups``, ``dec.resblocks``, flow WN): ``weight_v``
  ~ N(0, sigma) and ``weight_g = ||v|| * U(0.8, 1.2)`` per output channel, so
  the de-weight-norm scaling is not the identity;
* plain convs / linears: U(+-1/sqrt(fan_in)) for weight and bias;
* ``emb_rel_k/v`` ~ N(0, kc^-0.5); LayerNorm gamma ~ 1 + 0.1 N, beta ~ 0.1 N;
* flow ``post`` is random (upstream zero-inits it, which would make the flow
  an identity and leave it unexercised).

The RNG is numpy's PCG64 (``default_rng``); a given ``(geometry, seed)``
always yields the same float32 arrays.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "Geometry",
    "GEOM_40K",
    "GEOM_48K",
    "GEOM_TINY",
    "make_weights",
    "make_f0",
    "make_dec_inputs",
    "make_synth_inputs",
    "make_noise",
    "weights_digest",
    "HubertGeometry",
    "HUBERT_BASE",
    "make_hubert_weights",
    "make_hubert_input",
]


class Geometry:
    """Architecture hyper-parameters of one RVC v2 synthesizer variant."""

    def __init__(self, *, phone_dim=768, hidden=192, filter_channels=768,
                 n_heads=2, n_layers=6, window=10, gin=256, n_spk=4,
                 upsample_initial=512, upsample_rates=(10, 10, 2, 2),
                 upsample_kernels=(16, 16, 4, 4), sr=40000,
                 n_flows=4, wn_layers=3, wn_kernel=5):
        self.phone_dim = phone_dim
        self.hidden = hidden
        self.filter_channels = filter_channels
        self.n_heads = n_heads
        self.n_layers = n_layers
        self.window = window
        self.gin = gin
        self.n_spk = n_spk
        self.upsample_initial = upsample_initial
        self.upsample_rates = list(upsample_rates)
        self.upsample_kernels = list(upsample_kernels)
        self.sr = sr
        self.n_flows = n_flows
        self.wn_layers = wn_layers
        self.wn_kernel = wn_kernel

    @property
    def upp(self) -> int:
        return int(math.prod(self.upsample_rates))

    @property
    def kc(self) -> int:
        return self.hidden // self.n_heads

    def noise_strides(self):
        n = len(self.upsample_rates)
        return [int(math.prod(self.upsample_rates[i + 1:])) if i < n - 1 else 1
                for i in range(n)]

    def stage_channels(self):
        return [self.upsample_initial // (2 ** (i + 1))
                for i in range(len(self.upsample_rates))]

    def config_array(self):
        """The checkpoint ``config`` list layout (``runtime/models/vits.py:174-177``)."""
        return [1025, 32, self.hidden, self.hidden, self.filter_channels,
                self.n_heads, self.n_layers, 3, 0.0, "1", [3, 7, 11],
                [[1, 3, 5], [1, 3, 5], [1, 3, 5]], list(self.upsample_rates),
                self.upsample_initial, list(self.upsample_kernels), self.n_spk,
                self.gin, self.sr]


GEOM_40K = Geometry()
GEOM_48K = Geometry(upsample_rates=(12, 10, 2, 2), upsample_kernels=(24, 20, 4, 4),
                    sr=48000)
# Reduced widths with the same structure: odd channel counts exercise every
# masking path of the kernels (stage channels 32/16/8/4).
GEOM_TINY = Geometry(phone_dim=64, hidden=48, filter_channels=96, n_heads=2,
                     n_layers=2, gin=32, n_spk=3, upsample_initial=64)


RB_GAIN = 1.0
UP_GAIN = 1.5


def _uniform(rng, shape, fan_in):
    bound = 1.0 / math.sqrt(fan_in)
    return rng.uniform(-bound, bound, size=shape).astype(np.float32)


def _wn_pair(rng, shape, sigma):
    v = (rng.standard_normal(shape) * sigma).astype(np.float32)
    norm = np.sqrt((v.astype(np.float64) ** 2).reshape(shape[0], -1).sum(1))
    g = (norm * rng.uniform(0.8, 1.2, size=shape[0])).astype(np.float32)
    return v, g.reshape(shape[0], 1, 1)


def make_weights(geom: Geometry = GEOM_40K, seed: int = 0, rb_gain: float = RB_GAIN,
                 up_gain: float = UP_GAIN) -> dict:
    """Random-init float32 weight dict keyed like an RVC v2 checkpoint.

    Decoder weight-norm layers use ``v ~ N(0, gain / sqrt(fan_in))`` (fan_in =
    C*k for ResBlock convs, C_in*K/stride taps per output for the
    upsamplers) so every stage carries signal of order one into ``tanh``.
    """
    rng = np.random.default_rng(seed)
    w: dict = {}
    H, F, G = geom.hidden, geom.filter_channels, geom.gin
    kc = geom.kc
    w["emb_g.weight"] = rng.standard_normal((geom.n_spk, G)).astype(np.float32)
    # ---- enc_p ----
    w["enc_p.emb_phone.weight"] = _uniform(rng, (H, geom.phone_dim), geom.phone_dim)
    w["enc_p.emb_phone.bias"] = _uniform(rng, (H,), geom.phone_dim)
    w["enc_p.emb_pitch.weight"] = rng.standard_normal((256, H)).astype(np.float32)
    for i in range(geom.n_layers):
        base = f"enc_p.encoder.attn_layers.{i}"
        for name in ("conv_q", "conv_k", "conv_v", "conv_o"):
            w[f"{base}.{name}.weight"] = _uniform(rng, (H, H, 1), H)
            w[f"{base}.{name}.bias"] = _uniform(rng, (H,), H)
        for name in ("emb_rel_k", "emb_rel_v"):
            w[f"{base}.{name}"] = (rng.standard_normal((1, 2 * geom.window + 1, kc))
                                   * kc ** -0.5).astype(np.float32)
        for nl in ("norm_layers_1", "norm_layers_2"):
            b2 = f"enc_p.encoder.{nl}.{i}"
            w[f"{b2}.gamma"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
            w[f"{b2}.beta"] = (0.1 * rng.standard_normal(H)).astype(np.float32)
        fb = f"enc_p.encoder.ffn_layers.{i}"
        w[f"{fb}.conv_1.weight"] = _uniform(rng, (F, H, 3), H * 3)
        w[f"{fb}.conv_1.bias"] = _uniform(rng, (F,), H * 3)
        w[f"{fb}.conv_2.weight"] = _uniform(rng, (H, F, 3), F * 3)
        w[f"{fb}.conv_2.bias"] = _uniform(rng, (H,), F * 3)
    w["enc_p.proj.weight"] = _uniform(rng, (2 * H, H, 1), H)
    w["enc_p.proj.bias"] = _uniform(rng, (2 * H,), H)
    # ---- flow ----
    half = H // 2
    for f in range(geom.n_flows):
        idx = 2 * f
        base = f"flow.flows.{idx}"
        w[f"{base}.pre.weight"] = _uniform(rng, (H, half, 1), half)
        w[f"{base}.pre.bias"] = _uniform(rng, (H,), half)
        w[f"{base}.post.weight"] = _uniform(rng, (half, H, 1), H)
        w[f"{base}.post.bias"] = _uniform(rng, (half,), H)
        c_out = 2 * H * geom.wn_layers
        v, g = _wn_pair(rng, (c_out, G, 1), 1.0 / math.sqrt(G))
        w[f"{base}.enc.cond_layer.weight_v"], w[f"{base}.enc.cond_layer.weight_g"] = v, g
        w[f"{base}.enc.cond_layer.bias"] = _uniform(rng, (c_out,), G)
        for i in range(geom.wn_layers):
            fan = H * geom.wn_kernel
            v, g = _wn_pair(rng, (2 * H, H, geom.wn_kernel), 1.0 / math.sqrt(fan))
            w[f"{base}.enc.in_layers.{i}.weight_v"] = v
            w[f"{base}.enc.in_layers.{i}.weight_g"] = g
            w[f"{base}.enc.in_layers.{i}.bias"] = _uniform(rng, (2 * H,), fan)
            rs = 2 * H if i < geom.wn_layers - 1 else H
            v, g = _wn_pair(rng, (rs, H, 1), 1.0 / math.sqrt(H))
            w[f"{base}.enc.res_skip_layers.{i}.weight_v"] = v
            w[f"{base}.enc.res_skip_layers.{i}.weight_g"] = g
            w[f"{base}.enc.res_skip_layers.{i}.bias"] = _uniform(rng, (rs,), H)
    # ---- dec (GeneratorNSF) ----
    U = geom.upsample_initial
    w["dec.conv_pre.weight"] = _uniform(rng, (U, H, 7), H * 7)
    w["dec.conv_pre.bias"] = _uniform(rng, (U,), H * 7)
    w["dec.cond.weight"] = _uniform(rng, (U, G, 1), G)
    w["dec.cond.bias"] = _uniform(rng, (U,), G)
    w["dec.m_source.l_linear.weight"] = rng.uniform(-1, 1, size=(1, 1)).astype(np.float32)
    w["dec.m_source.l_linear.bias"] = rng.uniform(-1, 1, size=(1,)).astype(np.float32)
    strides = geom.noise_strides()
    chans = geom.stage_channels()
    c_in = U
    for i, (r, k) in enumerate(zip(geom.upsample_rates, geom.upsample_kernels)):
        c_out = chans[i]
        v, g = _wn_pair(rng, (c_in, c_out, k), up_gain / math.sqrt(c_in * k / r))
        w[f"dec.ups.{i}.weight_v"], w[f"dec.ups.{i}.weight_g"] = v, g
        w[f"dec.ups.{i}.bias"] = _uniform(rng, (c_out,), c_in * k)
        kn = 2 * strides[i] if i < len(strides) - 1 else 1
        w[f"dec.noise_convs.{i}.weight"] = _uniform(rng, (c_out, 1, kn), kn)
        w[f"dec.noise_convs.{i}.bias"] = _uniform(rng, (c_out,), kn)
        for j, kr in enumerate((3, 7, 11)):
            base = f"dec.resblocks.{3 * i + j}"
            for layer in ("convs1", "convs2"):
                for q in range(3):
                    v, g = _wn_pair(rng, (c_out, c_out, kr), rb_gain / math.sqrt(c_out * kr))
                    w[f"{base}.{layer}.{q}.weight_v"] = v
                    w[f"{base}.{layer}.{q}.weight_g"] = g
                    w[f"{base}.{layer}.{q}.bias"] = _uniform(rng, (c_out,), c_out * kr)
        c_in = c_out
    w["dec.conv_post.weight"] = _uniform(rng, (1, chans[-1], 7), chans[-1] * 7)
    return w


def weights_digest(w: dict) -> str:
    """Order-independent SHA-256 over keys, shapes and raw bytes."""
    import hashlib

    h = hashlib.sha256()
    for k in sorted(w):
        a = np.ascontiguousarray(w[k])
        h.update(k.encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def make_f0(P: int, rng, lo: float = 80.0, hi: float = 400.0,
            unvoiced_frac: float = 0.2) -> np.ndarray:
    """f0 [1,P] ~ U(lo,hi) with >= ``unvoiced_frac`` of frames zeroed in runs.

    Run lengths are U[3,12] frames placed by the seeded RNG until the
    zeroed fraction reaches the target (BASELINE config 1 input spec).
    """
    f0 = rng.uniform(lo, hi, size=(1, P)).astype(np.float32)
    target = int(math.ceil(unvoiced_frac * P))
    zeroed = np.zeros(P, dtype=bool)
    guard = 0
    while zeroed.sum() < target and guard < 10 * P + 10:
        n = int(rng.integers(3, 13))
        s = int(rng.integers(0, max(1, P)))
        zeroed[s:s + n] = True
        guard += 1
    f0[0, zeroed] = 0.0
    return f0


def make_noise(geom: Geometry, P: int, seed: int, batch: int = 1):
    """(nz, ns) drawn like ``SynthesizerTrn._make_noise``: nz [1,H,P] first,
    then ns [1,P*upp,1], both float64 ``standard_normal`` cast to float32
    (``runtime/models/vits.py:2337-2350``)."""
    rng = np.random.RandomState(seed)
    nz = rng.standard_normal((1, geom.hidden, P)).astype(np.float32)
    ns = rng.standard_normal((1, P * geom.upp, 1)).astype(np.float32)
    return nz, ns


def make_dec_inputs(geom: Geometry, P: int, seed: int):
    """BASELINE config 1 inputs: z [1,H,P], g [1,gin,1], f0 [1,P], ns."""
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((1, geom.hidden, P)).astype(np.float32)
    g = rng.standard_normal((1, geom.gin, 1)).astype(np.float32)
    f0 = make_f0(P, rng)
    _, ns = make_noise(geom, P, seed)
    return {"z": z, "g": g, "f0": f0, "ns": ns}


def make_synth_inputs(geom: Geometry, P: int, seed: int):
    """BASELINE config 2 inputs: phone [1,P,D], pitch int64 [1,P] in [1,255],
    nsff0 [1,P], sid [1], and nz/ns from ``RandomState(seed)`` in that order."""
    rng = np.random.default_rng(seed)
    phone = rng.standard_normal((1, P, geom.phone_dim)).astype(np.float32)
    pitch = rng.integers(1, 256, size=(1, P)).astype(np.int64)
    nsff0 = make_f0(P, rng)
    sid = np.array([0], dtype=np.int64)
    nz, ns = make_noise(geom, P, seed)
    return {"phone": phone, "pitch": pitch, "nsff0": nsff0, "sid": sid,
            "nz": nz, "ns": ns}


# ---------------------------------------------------------------------------
# HuBERT-base
# ---------------------------------------------------------------------------

class HubertGeometry:
    """HuBERT-base hyper-parameters as the reference fixes them
    (``runtime/models/hubert.py:9-44``): 7 conv layers of 512 channels,
    kernels [10,3,3,3,3,2,2] / strides [5,2,2,2,2,2,2], GroupNorm on layer 0,
    hidden 768, 12 layers, 12 heads, FFN 3072, pos-conv k128 in 16 groups."""

    def __init__(self, *, conv_dim=512, conv_kernels=(10, 3, 3, 3, 3, 2, 2), hidden=768, n_layers=12,
                 ffn=3072, pos_kernel=128, pos_groups=16, final_dim=256):
        self.conv_dim = conv_dim
        self.conv_kernels = list(conv_kernels)
        self.conv_strides = [5] + [2] * (len(conv_kernels) - 1)
        self.hidden = hidden
        self.n_layers = n_layers
        self.ffn = ffn
        self.pos_kernel = pos_kernel
        self.pos_groups = pos_groups
        self.final_dim = final_dim

    def frames(self, T: int) -> int:
        L = T
        for k, s in zip(self.conv_kernels, self.conv_strides):
            L = (L - k) // s + 1
        return L


HUBERT_BASE = HubertGeometry()


def make_hubert_weights(geom: HubertGeometry = HUBERT_BASE, seed: int = 0) -> dict:
    """Random-init float32 state dict with the transformers key names the
    reference reads (``runtime/models/hubert.py:510-558``).

    Convs: ``N(0, sqrt(2 / fan_in))`` (keeps the bias-free conv + GELU stack
    away from underflow); linears: ``U(+-1/sqrt(fan_in))`` weights and biases;
    norms: ``gamma ~ 1 + 0.1 N``, ``beta ~ 0.1 N``; the positional conv's
    ``weight_g`` is the per-tap norm of ``weight_v`` times ``U(0.8, 1.2)``."""
    rng = np.random.default_rng(seed)
    w: dict = {}
    C, H, F = geom.conv_dim, geom.hidden, geom.ffn

    def norm_pair(name, n):
        w[name + ".weight"] = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        w[name + ".bias"] = (0.1 * rng.standard_normal(n)).astype(np.float32)

    def linear(name, o, i):
        w[name + ".weight"] = _uniform(rng, (o, i), i)
        w[name + ".bias"] = _uniform(rng, (o,), i)

    c_in = 1
    for i, k in enumerate(geom.conv_kernels):
        w[f"feature_extractor.conv_layers.{i}.conv.weight"] = (
            rng.standard_normal((C, c_in, k)) * math.sqrt(2.0 / (c_in * k))).astype(np.float32)
        c_in = C
    norm_pair("feature_extractor.conv_layers.0.layer_norm", C)
    norm_pair("feature_projection.layer_norm", C)
    linear("feature_projection.projection", H, C)
    cpg = H // geom.pos_groups
    K = geom.pos_kernel
    v = (rng.standard_normal((H, cpg, K)) / math.sqrt(cpg * K)).astype(np.float32)
    tap_norm = np.sqrt((v.astype(np.float64) ** 2).sum(axis=(0, 1)))
    w["encoder.pos_conv_embed.conv.weight_v"] = v
    w["encoder.pos_conv_embed.conv.weight_g"] = (tap_norm * rng.uniform(0.8, 1.2, size=K)).astype(
        np.float32).reshape(1, 1, K)
    w["encoder.pos_conv_embed.conv.bias"] = _uniform(rng, (H,), cpg * K)
    norm_pair("encoder.layer_norm", H)
    for i in range(geom.n_layers):
        p = f"encoder.layers.{i}."
        for nm in ("q_proj", "k_proj", "v_proj", "out_proj"):
            linear(p + "attention." + nm, H, H)
        norm_pair(p + "layer_norm", H)
        linear(p + "feed_forward.intermediate_dense", F, H)
        linear(p + "feed_forward.output_dense", H, F)
        norm_pair(p + "final_layer_norm", H)
    linear("final_proj", geom.final_dim, H)
    return w


def make_hubert_input(T: int, seed: int) -> np.ndarray:
    """BASELINE config 3 input: x ~ N(0, 0.1) [1, T] at 16 kHz."""
    rng = np.random.default_rng(seed)
    return (0.1 * rng.standard_normal((1, T))).astype(np.float32)


# ---------------------------------------------------------------------- RMVPE
RMVPE_EN = (16, 32, 64, 128, 256)   # encoder level widths (E2E en_out_channels=16, 5 levels)
RMVPE_INTER = 512                   # intermediate width (4 levels)
RMVPE_GRU = 256                     # BiGRU hidden size
RMVPE_BINS = 360


def rmvpe_blocks():
    """(prefix, C_in, C_out) of every ConvBlockRes of ``E2E(4, 1, (2, 2))``
    in execution order, and (prefix, C_in, C_out) of the five decoder
    ConvTranspose2d layers (``runtime/models/rmvpe.py:643-690``)."""
    blocks, ups = [], []
    c = 1
    for i, o in enumerate(RMVPE_EN):
        for j in range(4):
            blocks.append((f"unet.encoder.layers.{i}.conv.{j}", c if j == 0 else o, o))
        c = o
    for i in range(4):
        for j in range(4):
            blocks.append((f"unet.intermediate.layers.{i}.conv.{j}", c if j == 0 else RMVPE_INTER, RMVPE_INTER))
        c = RMVPE_INTER
    for i in range(5):
        o = c // 2
        ups.append((f"unet.decoder.layers.{i}", c, o))
        for j in range(4):
            blocks.append((f"unet.decoder.layers.{i}.conv2.{j}", 2 * o if j == 0 else o, o))
        c = o
    return blocks, ups


def make_rmvpe_weights(seed: int = 0) -> dict:
    """Random-init float32 RMVPE state dict with the checkpoint's key names
    (``runtime/models/rmvpe.py:518-551, 643-690, 727-751``).

    Convs and linears: ``U(+-1/sqrt(fan_in))`` (PyTorch's default bound);
    BatchNorm: gamma ~ U(0.8, 1.2), beta and running_mean ~ U(-0.1, 0.1),
    running_var ~ U(0.8, 1.2), so each folded scale/shift differs from the
    identity; GRU: ``U(+-1/sqrt(hidden))`` as ``torch.nn.GRU`` initialises."""
    rng = np.random.default_rng(seed)
    w: dict = {}

    def bn(p, n):
        w[p + ".weight"] = rng.uniform(0.8, 1.2, n).astype(np.float32)
        w[p + ".bias"] = rng.uniform(-0.1, 0.1, n).astype(np.float32)
        w[p + ".running_mean"] = rng.uniform(-0.1, 0.1, n).astype(np.float32)
        w[p + ".running_var"] = rng.uniform(0.8, 1.2, n).astype(np.float32)

    bn("unet.encoder.bn", 1)
    blocks, ups = rmvpe_blocks()
    up_at = {p + ".conv2.0": (p, ci, co) for p, ci, co in ups}
    for p, ci, co in blocks:
        if p in up_at:
            q, uci, uco = up_at[p]
            w[q + ".conv1.0.weight"] = _uniform(rng, (uci, uco, 3, 3), uco * 9)
            bn(q + ".conv1.1", uco)
        w[p + ".conv.0.weight"] = _uniform(rng, (co, ci, 3, 3), ci * 9)
        bn(p + ".conv.1", co)
        w[p + ".conv.3.weight"] = _uniform(rng, (co, co, 3, 3), co * 9)
        bn(p + ".conv.4", co)
        if ci != co:
            w[p + ".shortcut.weight"] = _uniform(rng, (co, ci, 1, 1), ci)
            w[p + ".shortcut.bias"] = _uniform(rng, (co,), ci)
    w["cnn.weight"] = _uniform(rng, (3, RMVPE_EN[0], 3, 3), RMVPE_EN[0] * 9)
    w["cnn.bias"] = _uniform(rng, (3,), RMVPE_EN[0] * 9)
    H = RMVPE_GRU
    for sfx in ("", "_reverse"):
        w["fc.0.gru.weight_ih_l0" + sfx] = _uniform(rng, (3 * H, 3 * 128), H)
        w["fc.0.gru.weight_hh_l0" + sfx] = _uniform(rng, (3 * H, H), H)
        w["fc.0.gru.bias_ih_l0" + sfx] = _uniform(rng, (3 * H,), H)
        w["fc.0.gru.bias_hh_l0" + sfx] = _uniform(rng, (3 * H,), H)
    w["fc.1.weight"] = _uniform(rng, (RMVPE_BINS, 2 * H), 2 * H)
    w["fc.1.bias"] = _uniform(rng, (RMVPE_BINS,), 2 * H)
    return w


def make_rmvpe_audio(T: int, seed: int) -> np.ndarray:
    """16 kHz test signal: a 110-330 Hz glide plus its 2nd harmonic, noise
    at -30 dB and a silent gap (exercises the clamp of the log-mel)."""
    rng = np.random.default_rng(seed)
    t = np.arange(T) / 16000.0
    f = 110.0 + 220.0 * t / max(t[-1], 1e-9)
    ph = 2 * np.pi * np.cumsum(f) / 16000.0
    x = 0.3 * np.sin(ph) + 0.1 * np.sin(2 * ph) + 0.01 * rng.standard_normal(T)
    x[T // 3: T // 3 + T // 10] = 0.0
    return x.astype(np.float32)
