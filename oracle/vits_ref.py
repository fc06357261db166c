# -*- coding: utf-8 -*-
"""numpy restatement of the reference RVC synthesizer (numpy backend branch).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``runtime/models/vits.py`` with the numpy backend (no resident
weights, ``_weights.enabled`` False), i.e. the ``else`` branches:
``_TextEncoder.encode`` :962-1049, ``_FlowBlock._rc_reverse/_wn/reverse``
:1086-1145, :1255-1268, ``_ResBlock1.forward`` :1285-1311,
``_GeneratorNSF._sine_gen/forward`` :1468-1501, :2133-2231 and
``SynthesizerTrn.infer_controlled`` :2551-2595.  Evaluation order that
changes float32 rounding is kept (sequential float32 cumsum of the sine
phase, ``((o1+o2)+o3)/3`` ResBlock average, conv bias after the core).
"""

from __future__ import annotations

import math

import numpy as np

from . import nn_ref as nn

__all__ = [
    "VitsConfig",
    "deweight_norm",
    "get_relative_embeddings",
    "relative_to_absolute",
    "absolute_to_relative",
    "TextEncoder",
    "FlowBlock",
    "GeneratorNSF",
    "Synthesizer",
]

_UPP_48K = 480
# partial synthesis context (runtime/models/vits.py:141-152): decoder frames
# either side of the target segment, and the flow's receptive field
DEC_PAD = 16
FLOW_PAD = 24


class VitsConfig:
    """Geometry from weight shapes and/or the checkpoint ``config`` list
    (``runtime/models/vits.py:166-268``)."""

    def __init__(self, w: dict, config=None, sr=None):
        cfg = list(config) if config is not None else None
        self.phone_dim = int(w["enc_p.emb_phone.weight"].shape[1])
        self.hidden = int(w["enc_p.emb_phone.weight"].shape[0])
        self.filter = int(w["enc_p.encoder.ffn_layers.0.conv_1.weight"].shape[0])
        n = 0
        while f"enc_p.encoder.attn_layers.{n}.conv_q.weight" in w:
            n += 1
        self.n_layers = n
        self.k_channels = int(w["enc_p.encoder.attn_layers.0.emb_rel_k"].shape[2])
        self.n_heads = self.hidden // self.k_channels
        self.upsample_initial = int(w["dec.conv_pre.weight"].shape[0])
        n_ups_w = 0
        while f"dec.ups.{n_ups_w}.weight_v" in w:
            n_ups_w += 1
        ups_kernels_w = [int(w[f"dec.ups.{i}.weight_v"].shape[2]) for i in range(n_ups_w)]
        if cfg and len(cfg) > 12:
            self.upsample_rates = [int(r) for r in cfg[12]]
            self.upsample_initial = int(cfg[13])
            self.sr = int(sr) if sr else (int(cfg[17]) if len(cfg) > 17 else 48000)
            if len(cfg) > 14 and cfg[14] is not None and cfg[14] != "":
                self.upsample_kernels = [int(k) for k in cfg[14]]
            else:
                self.upsample_kernels = ups_kernels_w
        else:
            self.upsample_rates = self._infer_rates(w, n_ups_w)
            self.sr = int(sr) if sr else 48000
            if sr:
                rest = math.prod(self.upsample_rates[1:])
                self.upsample_rates[0] = int(self.sr // 100) // rest
            self.upsample_kernels = ups_kernels_w
        self.n_ups = len(self.upsample_rates) or n_ups_w
        self.upp = int(math.prod(self.upsample_rates))
        self.noise_strides = []
        for i in range(self.n_ups):
            k = int(w[f"dec.noise_convs.{i}.weight"].shape[2])
            self.noise_strides.append(k // 2 if i < self.n_ups - 1 else 1)
        self.resblock_kernel_sizes = [3, 7, 11]
        self.resblock_dilation_sizes = [[1, 3, 5], [1, 3, 5], [1, 3, 5]]
        self.n_spk = int(w["emb_g.weight"].shape[0])
        self.gin_channels = int(w["emb_g.weight"].shape[1])

    @staticmethod
    def _infer_rates(w, n_ups):
        """Rates from noise-conv kernels, first rate from upp=480
        (``runtime/models/vits.py:251-268``)."""
        strides = []
        for i in range(n_ups):
            k = int(w[f"dec.noise_convs.{i}.weight"].shape[2])
            strides.append(k // 2 if i < n_ups - 1 else 1)
        rates = [strides[i] // strides[i + 1] for i in range(n_ups - 1)]
        rates.insert(0, _UPP_48K // strides[0])
        return rates


def deweight_norm(w_v, w_g):
    """``W = v * (g / ||v||)``, norm over all but dim 0, clamped at 1e-12
    (``runtime/models/vits.py:416-442``)."""
    w_v = np.asarray(w_v)
    w_g = np.asarray(w_g)
    dtype = w_v.dtype if w_v.dtype in (np.float32, np.float64) else np.float32
    w_v = w_v.astype(dtype, copy=False)
    w_g = w_g.astype(dtype, copy=False)
    if w_g.ndim == 1:
        w_g = w_g.reshape(-1, 1, 1)
    norm = np.linalg.norm(w_v.reshape(w_v.shape[0], -1), ord=2, axis=1)
    norm = np.maximum(norm, 1e-12).astype(dtype, copy=False)
    return (w_v * (w_g.reshape(-1, 1, 1) / norm.reshape(-1, 1, 1))).astype(dtype, copy=False)


def get_relative_embeddings(emb_rel, length, window_size):
    """[1,2w+1,k] -> [1,2L-1,k]: zero-pad both ends when L > w+1, else slice
    (``runtime/models/vits.py:448-462``)."""
    pad = max(length - (window_size + 1), 0)
    start = max((window_size + 1) - length, 0)
    end = start + 2 * length - 1
    emb = np.pad(emb_rel, ((0, 0), (pad, pad), (0, 0))) if pad > 0 else emb_rel
    return emb[:, start:end, :]


def relative_to_absolute(x):
    """[b,h,l,2l-1] -> [b,h,l,l] by the pad/reshape trick
    (``runtime/models/vits.py:465-472``)."""
    b, h, n, _ = x.shape
    xp = np.pad(x, ((0, 0), (0, 0), (0, 0), (0, 1))).reshape(b, h, n * 2 * n)
    xp = np.pad(xp, ((0, 0), (0, 0), (0, n - 1))).reshape(b, h, n + 1, 2 * n - 1)
    return xp[:, :, :n, n - 1:]


def absolute_to_relative(x):
    """[b,h,l,l] -> [b,h,l,2l-1] (``runtime/models/vits.py:475-482``)."""
    b, h, n, _ = x.shape
    xp = np.pad(x, ((0, 0), (0, 0), (0, 0), (0, n - 1))).reshape(b, h, n * n + n * (n - 1))
    xp = np.pad(xp, ((0, 0), (0, 0), (n, 0))).reshape(b, h, n, 2 * n)
    return xp[:, :, :, 1:]


class TextEncoder:
    """enc_p: embed, 6 relative-position attention layers, proj
    (``runtime/models/vits.py:488-1059``, numpy branches)."""

    def __init__(self, w, cfg: VitsConfig):
        self.w = w
        self.cfg = cfg

    def embed(self, phone, pitch):
        """``linear(phone) + emb_pitch[pitch]`` (:499-538)."""
        w = self.w
        x = nn.linear(phone, w["enc_p.emb_phone.weight"], w["enc_p.emb_phone.bias"])
        if pitch is not None:
            x = x + nn.embedding(pitch, w["enc_p.emb_pitch.weight"])
        return x

    def encode(self, x, x_mask):
        """[1,P,h] -> [1,P,h] (:962-1049; mask all ones skips the where)."""
        w = self.w
        hdim = self.cfg.hidden
        heads, kc = self.cfg.n_heads, self.cfg.k_channels
        mask_all_one = bool(np.all(x_mask != 0.0))
        attn_mask = None if mask_all_one else (x_mask[..., None] * x_mask[..., None, :])
        x = (x * x_mask.transpose(0, 2, 1)).transpose(0, 2, 1)
        for i in range(self.cfg.n_layers):
            a = f"enc_p.encoder.attn_layers.{i}"
            q = nn.conv1d(x, w[f"{a}.conv_q.weight"], w[f"{a}.conv_q.bias"])
            k = nn.conv1d(x, w[f"{a}.conv_k.weight"], w[f"{a}.conv_k.bias"])
            v = nn.conv1d(x, w[f"{a}.conv_v.weight"], w[f"{a}.conv_v.bias"])
            P = x.shape[-1]
            qh = q.reshape(1, heads, kc, P).transpose(0, 1, 3, 2)
            kh = k.reshape(1, heads, kc, P).transpose(0, 1, 3, 2)
            vh = v.reshape(1, heads, kc, P).transpose(0, 1, 3, 2)
            qs = qh / math.sqrt(kc)
            scores = np.matmul(qs, np.ascontiguousarray(kh.swapaxes(-1, -2)))
            used_k = get_relative_embeddings(w[f"{a}.emb_rel_k"], P, window_size=10)
            rel = np.matmul(qs, np.ascontiguousarray(used_k[0].T))
            scores = scores + relative_to_absolute(rel)
            if attn_mask is not None:
                scores = np.where(attn_mask != 0, scores, -1e4)
            p_attn = nn.softmax(scores, axis=-1)
            out = np.matmul(p_attn, vh)
            used_v = get_relative_embeddings(w[f"{a}.emb_rel_v"], P, window_size=10)
            out = out + np.matmul(absolute_to_relative(p_attn), np.ascontiguousarray(used_v[0]))
            attn_out = out.transpose(0, 1, 3, 2).reshape(1, hdim, P)
            attn_out = nn.conv1d(attn_out, w[f"{a}.conv_o.weight"], w[f"{a}.conv_o.bias"])
            x = nn.layer_norm((x + attn_out).transpose(0, 2, 1),
                              w[f"enc_p.encoder.norm_layers_1.{i}.gamma"],
                              w[f"enc_p.encoder.norm_layers_1.{i}.beta"]).transpose(0, 2, 1)
            f = f"enc_p.encoder.ffn_layers.{i}"
            y = nn.conv1d(x, w[f"{f}.conv_1.weight"], w[f"{f}.conv_1.bias"], padding=1)
            y = nn.relu(y)
            y = nn.conv1d(y, w[f"{f}.conv_2.weight"], w[f"{f}.conv_2.bias"], padding=1)
            x = nn.layer_norm((x + y).transpose(0, 2, 1),
                              w[f"enc_p.encoder.norm_layers_2.{i}.gamma"],
                              w[f"enc_p.encoder.norm_layers_2.{i}.beta"]).transpose(0, 2, 1)
        x = x * x_mask
        return x.transpose(0, 2, 1)

    def stats(self, x):
        """proj 1x1 then split into (m, logs) (:1051-1059)."""
        s = nn.conv1d(x.transpose(0, 2, 1), self.w["enc_p.proj.weight"], self.w["enc_p.proj.bias"])
        h = self.cfg.hidden
        return s[:, :h, :], s[:, h:, :]


class FlowBlock:
    """Reverse ResidualCouplingBlock: Flip, RC(6), Flip, RC(4), ... RC(0)
    (``runtime/models/vits.py:1062-1145, 1255-1268``)."""

    rc_ids = (0, 2, 4, 6)

    def __init__(self, w, cfg: VitsConfig):
        self.w = w
        self.cfg = cfg

    def _dwn(self, idx, name):
        k = f"flow.flows.{idx}.{name}"
        return deweight_norm(self.w[k + ".weight_v"], self.w[k + ".weight_g"])

    def _wn(self, x, x_mask, g, idx):
        w = self.w
        hidden = self.cfg.hidden
        n_layers = 3
        if g is not None:
            g = nn.conv1d(g, self._dwn(idx, "enc.cond_layer"),
                          w[f"flow.flows.{idx}.enc.cond_layer.bias"])
        output = np.zeros_like(x)
        for i in range(n_layers):
            x_in = nn.conv1d(x, self._dwn(idx, f"enc.in_layers.{i}"),
                             w[f"flow.flows.{idx}.enc.in_layers.{i}.bias"],
                             dilation=1, padding=2)
            if g is not None:
                off = i * 2 * hidden
                g_l = g[:, off:off + 2 * hidden, :]
            else:
                g_l = np.zeros_like(x_in)
            acts = nn.tanh(x_in + g_l)[:, :hidden, :] * nn.sigmoid((x_in + g_l)[:, hidden:, :])
            rs = nn.conv1d(acts, self._dwn(idx, f"enc.res_skip_layers.{i}"),
                           w[f"flow.flows.{idx}.enc.res_skip_layers.{i}.bias"])
            if i < n_layers - 1:
                x = (x + rs[:, :hidden, :]) * x_mask
                output = output + rs[:, hidden:, :]
            else:
                output = output + rs
        return output * x_mask

    def _rc_reverse(self, z, x_mask, g, idx):
        w = self.w
        half = self.cfg.hidden // 2
        x0, x1 = z[:, :half, :], z[:, half:, :]
        h = nn.conv1d(x0, w[f"flow.flows.{idx}.pre.weight"], w[f"flow.flows.{idx}.pre.bias"]) * x_mask
        h = self._wn(h, x_mask, g, idx)
        m = nn.conv1d(h, w[f"flow.flows.{idx}.post.weight"], w[f"flow.flows.{idx}.post.bias"]) * x_mask
        x1 = (x1 - m) * x_mask
        return np.concatenate([x0, x1], axis=1)

    def reverse(self, z, x_mask, g):
        for idx in reversed(self.rc_ids):
            z = np.flip(z, axis=1)
            z = self._rc_reverse(z, x_mask, g, idx)
        return z


def resblock1(w, base, k, x):
    """ResBlock1: three ``x += conv_{k,1}(lrelu(conv_{k,d}(lrelu(x))))``
    groups, d = 1,3,5 (``runtime/models/vits.py:1285-1311``)."""
    for j, d in enumerate((1, 3, 5)):
        b1 = f"{base}.convs1.{j}"
        c1 = nn.leaky_relu(x, 0.1)
        c1 = nn.conv1d(c1, deweight_norm(w[b1 + ".weight_v"], w[b1 + ".weight_g"]),
                       w[b1 + ".bias"], dilation=d, padding=(k * d - d) // 2)
        c1 = nn.leaky_relu(c1, 0.1)
        b2 = f"{base}.convs2.{j}"
        c2 = nn.conv1d(c1, deweight_norm(w[b2 + ".weight_v"], w[b2 + ".weight_g"]),
                       w[b2 + ".bias"], padding=(k - 1) // 2)
        x = c2 + x
    return x


class GeneratorNSF:
    """NSF-HiFiGAN vocoder, numpy branch (``runtime/models/vits.py:1389-2231``)."""

    def __init__(self, w, cfg: VitsConfig):
        self.w = w
        self.cfg = cfg

    def sine_gen(self, f0, ns, seg_offsets=None):
        """SineGen (harmonic_num=0) + SourceModuleHnNSF -> har [1,1,P*upp]
        (:1468-1501).  float32 throughout; the phase cumsum is numpy's
        sequential float32 ``cumsum`` over frames."""
        w = self.w
        upp, sr = self.cfg.upp, self.cfg.sr
        f0r = f0[:, None].transpose(0, 2, 1)
        rad = f0r / sr * np.arange(1, upp + 1, dtype=np.float32)[None, None, :]
        if seg_offsets is None:
            rad2 = np.fmod(rad[..., -1:] + 0.5, 1.0) - 0.5
            acc = np.fmod(np.cumsum(rad2, axis=1), 1.0)
            rad = rad.copy()
            rad[:, 1:, :] += acc[:, :-1, :]
        else:
            rad = rad + np.asarray(seg_offsets, dtype=np.float32)
        rad = rad.reshape(1, -1, 1)
        sine = np.sin(2 * np.pi * rad) * 0.1
        uv = np.repeat((f0r > 0).astype(np.float32), upp, axis=1)
        noise_amp = uv * 0.003 + (1 - uv) * 0.1 / 3
        sine = sine * uv + noise_amp * ns
        lin = nn.linear(sine, w["dec.m_source.l_linear.weight"], w["dec.m_source.l_linear.bias"])
        return nn.tanh(lin).transpose(0, 2, 1)

    def forward(self, z, f0, g, ns, seg_offsets=None):
        """z [1,h,P], f0 [1,P], g [1,gin,1] or None, ns [1,P*upp,1] -> [1,1,P*upp]
        (:2133-2231, the ``_dec_batch`` False path)."""
        w, cfg = self.w, self.cfg
        har = self.sine_gen(f0, ns, seg_offsets=seg_offsets)
        x = nn.conv1d(z, w["dec.conv_pre.weight"], w["dec.conv_pre.bias"], padding=3)
        if g is not None:
            x = x + nn.conv1d(g, w["dec.cond.weight"], w["dec.cond.bias"])
        for i in range(cfg.n_ups):
            x = nn.leaky_relu(x, 0.1)
            up = f"dec.ups.{i}"
            wn = deweight_norm(w[up + ".weight_v"], w[up + ".weight_g"])
            x = nn.conv_transpose1d(x, wn, w[up + ".bias"], stride=cfg.upsample_rates[i],
                                    padding=(cfg.upsample_kernels[i] - cfg.upsample_rates[i]) // 2)
            src = nn.conv1d(har, w[f"dec.noise_convs.{i}.weight"], w[f"dec.noise_convs.{i}.bias"],
                            stride=cfg.noise_strides[i], padding=cfg.noise_strides[i] // 2)
            x = x + src
            xs = None
            for j, k in enumerate(cfg.resblock_kernel_sizes):
                o = resblock1(w, f"dec.resblocks.{3 * i + j}", k, x)
                xs = o if xs is None else xs + o
            x = xs / 3
        x = nn.leaky_relu(x, 0.01)
        x = nn.conv1d(x, w["dec.conv_post.weight"], None, padding=3)
        return nn.tanh(x)

    def decode_batch(self, z_list, g, f0_list, ns_list, off_list=None):
        """Multi-chunk decode = per-chunk forward loop in numpy mode
        (``runtime/models/vits.py:1847-1871``)."""
        off_list = off_list or [None] * len(z_list)
        return [self.forward(z, f0, g, ns, seg_offsets=off)
                for z, f0, ns, off in zip(z_list, f0_list, ns_list, off_list)]


class Synthesizer:
    """``SynthesizerTrn`` on a weight dict (``runtime/models/vits.py:2237-2595``)."""

    def __init__(self, w, config=None, sr=None):
        self.w = w
        self.cfg = VitsConfig(w, config, sr=sr)
        self.enc_p = TextEncoder(w, self.cfg)
        self.flow = FlowBlock(w, self.cfg)
        self.dec = GeneratorNSF(w, self.cfg)

    def resolve_g(self, sid):
        """``emb_g[sid]`` -> [1,gin,1] (:2268-2270)."""
        return nn.embedding(sid, self.w["emb_g.weight"])[0].reshape(1, -1, 1)

    def make_noise(self, P, seed, fixed_seed=""):
        """nz [1,h,P] then ns [1,P*upp,1] from one RandomState (:2337-2350);
        ``fixed_seed`` (the RVC_FIXED_SEED text) replaces ``seed=None``."""
        if seed is None and fixed_seed:
            seed = int(fixed_seed)
        rng = np.random.RandomState(seed) if seed is not None else np.random.RandomState()
        nz = rng.standard_normal((1, self.cfg.hidden, P)).astype(np.float32)
        ns = rng.standard_normal((1, P * self.cfg.upp, 1)).astype(np.float32)
        return nz, ns

    def infer(self, phone, pitch, nsff0, sid, seed, skip_head=None, return_length=None):
        """``infer`` (:2352-2402): full synthesis, or the partial synthesis of
        frames [skip_head, skip_head + return_length)."""
        nz, ns = self.make_noise(phone.shape[1], seed)
        if skip_head is None or return_length is None:
            return self.infer_controlled(phone, pitch, nsff0, sid, nz, ns)
        head, length = self._check_part(phone.shape[1], skip_head, return_length)
        p = self.partial_prep(phone, pitch, nsff0, sid, nz, ns, head, length)
        o = self.dec.forward(p["z_seg"], p["nsff0_seg"], p["g"], p["ns_seg"], seg_offsets=p["off"])
        return o[:, :, p["s0"]:p["s0"] + p["n_out"]]

    @staticmethod
    def _check_part(P, skip_head, return_length):
        head, length = int(skip_head), int(return_length)
        if head < 0 or head >= P or length <= 0 or head + length > P:
            raise ValueError(f"skip_head/return_length out of range: P={P}, head={head}, length={length}")
        return head, length

    def phase_offsets(self, nsff0):
        """``_phase_offsets`` (:2404-2414): the full run's per-frame
        fmod-cumsum phase [1,P,1]."""
        cfg = self.cfg
        f0r = nsff0[:, None].transpose(0, 2, 1)
        rad = f0r / cfg.sr * np.arange(1, cfg.upp + 1, dtype=np.float32)[None, None, :]
        rad2 = np.fmod(rad[..., -1:] + 0.5, 1.0) - 0.5
        return np.fmod(np.cumsum(rad2, axis=1), 1.0)

    def _enc_stats(self, phone, pitch, sid):
        cfg = self.cfg
        g = self.resolve_g(sid)
        x = self.enc_p.embed(phone, pitch)
        x = x * math.sqrt(cfg.hidden)
        x = nn.leaky_relu(x, 0.1)
        x_mask = np.ones((1, 1, phone.shape[1]), dtype=np.float32)
        m, logs = self.enc_p.stats(self.enc_p.encode(x, x_mask))
        return g, m * x_mask, logs * x_mask, x_mask

    def full_prep(self, phone, pitch, nsff0, sid, nz, ns):
        """``_full_prep``: the decoder inputs of ``infer_controlled``."""
        z, g = self.enc_flow(phone, pitch, sid, nz)
        P = phone.shape[1]
        return {"z_seg": z, "nsff0_seg": nsff0, "ns_seg": ns, "off": None, "g": g,
                "s0": 0, "n_out": P * self.cfg.upp}

    def partial_prep(self, phone, pitch, nsff0, sid, nz, ns, head, length):
        """``_partial_prep`` (:2416-2476): enc_p over every frame, the flow
        from ``flow_head = max(head - 24 - 16, 0)``, the decoder segment
        [zs, ze) = [head - 16, head + length + 16] clipped to [0, P), and the
        segment's phase offsets taken from the full run's fmod-cumsum."""
        upp = self.cfg.upp
        P = phone.shape[1]
        g, m, logs, x_mask = self._enc_stats(phone, pitch, sid)
        flow_head = max(head - FLOW_PAD - DEC_PAD, 0)
        z_p = (m[:, :, flow_head:] + np.exp(logs[:, :, flow_head:]) * nz[:, :, flow_head:] * 0.66666) \
            * x_mask[:, :, flow_head:]
        z = self.flow.reverse(z_p, x_mask[:, :, flow_head:], g)
        zs = max(head - DEC_PAD, 0)
        ze = min(P, head + length + DEC_PAD)
        z_seg = z[:, :, zs - flow_head:ze - flow_head]
        rad_acc = self.phase_offsets(nsff0)
        n_seg = ze - zs
        if zs == 0:
            off = np.zeros((1, n_seg, 1), dtype=np.float32)
            if n_seg > 1:
                off[:, 1:, :] = rad_acc[:, :n_seg - 1, :]
        else:
            off = rad_acc[:, zs - 1:zs - 1 + n_seg, :]
        return {"z_seg": z_seg * x_mask[:, :, zs:ze], "nsff0_seg": nsff0[:, zs:ze],
                "ns_seg": ns[:, zs * upp:ze * upp, :], "off": off, "g": g,
                "s0": (head - zs) * upp, "n_out": length * upp}

    def prep_dec(self, phone, pitch, nsff0, sid, seed, skip_head=None, return_length=None):
        """``prep_dec`` (:2478-2500)."""
        nz, ns = self.make_noise(phone.shape[1], seed)
        if skip_head is None or return_length is None:
            return self.full_prep(phone, pitch, nsff0, sid, nz, ns)
        head, length = self._check_part(phone.shape[1], skip_head, return_length)
        return self.partial_prep(phone, pitch, nsff0, sid, nz, ns, head, length)

    def decode_batch(self, preps):
        """``decode_batch(preps)`` (:2502-2522): every chunk's target segment,
        the speaker of the first prep for all of them."""
        if not preps:
            return []
        outs = self.dec.decode_batch([p["z_seg"] for p in preps], preps[0]["g"],
                                     [p["nsff0_seg"] for p in preps], [p["ns_seg"] for p in preps],
                                     [p["off"] for p in preps])
        return [o[:, :, p["s0"]:p["s0"] + p["n_out"]] for o, p in zip(outs, preps)]

    def enc_flow(self, phone, pitch, sid, nz):
        """Steps 1-7 of ``infer_controlled``: returns (z, g) fed to the decoder."""
        cfg = self.cfg
        P = phone.shape[1]
        g = self.resolve_g(sid)
        x = self.enc_p.embed(phone, pitch)
        x = x * math.sqrt(cfg.hidden)
        x = nn.leaky_relu(x, 0.1)
        x_mask = np.ones((1, 1, P), dtype=np.float32)
        h = self.enc_p.encode(x, x_mask)
        m, logs = self.enc_p.stats(h)
        m = m * x_mask
        logs = logs * x_mask
        z_p = (m + np.exp(logs) * nz * 0.66666) * x_mask
        z = self.flow.reverse(z_p, x_mask, g)
        return z * x_mask, g

    def infer_controlled(self, phone, pitch, nsff0, sid, nz, ns):
        """Full synthesis with injected noise (:2551-2595)."""
        z, g = self.enc_flow(phone, pitch, sid, nz)
        return self.dec.forward(z, nsff0, g, ns)
