# -*- coding: utf-8 -*-
"""numpy restatement of the reference HuBERT-base encoder (numpy backend).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``runtime/models/hubert.py`` with the numpy backend and without
numba (the branch this container and the GPU box take):

* ``gelu_erf`` -- ``0.5 x (1 + erf(x / sqrt 2))`` with erf by Abramowitz &
  Stegun 7.1.26 in float32 (``runtime/models/hubert.py:150-241``);
* ``_feature_extractor`` -- 7 valid convs without bias, strides 5, 2, ...,
  GroupNorm(512 groups) after conv 0, GELU after every conv (:658-697);
* ``_feature_projection`` -- LayerNorm(512), ``x @ W.T`` then ``+ b``
  (:775-802);
* ``_pos_conv_embed`` -- weight-norm over dims (0, 1) per tap, grouped conv
  k128 / pad 64 / 16 groups with bias, right column dropped, GELU
  (:510-522, :301-339, :838-858);
* ``_encoder`` -- ``h + pos``, LayerNorm, 12 post-LN layers (:928-968,
  :1262-1288): attention with q scaled after its bias, 12 heads x 64,
  ``np.matmul`` scores, max-subtracted softmax (:1315-1338, :243-258),
  ``h + attn``, LN, ``h + ffn``, LN with ffn = ``linear(gelu(linear))``
  (:1401-1451);
* ``encode`` -- version 2 returns the last hidden state [1, L, 768];
  version 1 applies ``final_proj`` to layer 9's output (:564-591).
"""

from __future__ import annotations

import numpy as np

from . import nn_ref as nn

__all__ = [
    "gelu_erf",
    "group_norm",
    "layer_norm_last",
    "grouped_conv1d",
    "pos_conv_weight",
    "HubertRef",
    "N_HEADS",
]

_F32 = np.float32
N_HEADS = 12
_A = (np.float32(0.254829592), np.float32(-0.284496736), np.float32(1.421413741),
      np.float32(-1.453152027), np.float32(1.061405429))
_P = np.float32(0.3275911)
_ONE = np.float32(1.0)
_HALF = np.float32(0.5)
_SQRT2_INV = np.float32(0.7071067811865476)


def _erf(x):
    """A&S 7.1.26 erf, float32 throughout (``runtime/models/hubert.py:194-202``)."""
    x32 = np.asarray(x, dtype=_F32)
    ax = np.abs(x32)
    t = _ONE / (_ONE + _P * ax)
    y = _ONE - (((((_A[4] * t + _A[3]) * t) + _A[2]) * t + _A[1]) * t + _A[0]) * t * np.exp(-ax * ax)
    return np.sign(x32) * y


def gelu_erf(x):
    """GELU with the A&S erf (``runtime/models/hubert.py:222-241``, numpy branch)."""
    x32 = np.asarray(x, dtype=_F32)
    return (_HALF * x32 * (_ONE + _erf(x32 * _SQRT2_INV))).astype(_F32)


def group_norm(x, gamma, beta, num_groups, eps=1e-5):
    """``nn.group_norm`` (``runtime/nn.py:415-436``): biased variance per group."""
    x = np.asarray(x)
    B, C = x.shape[0], x.shape[1]
    G = int(num_groups)
    spatial = x.shape[2:]
    xr = x.reshape(B, G, C // G, *spatial)
    axes = tuple(range(2, xr.ndim))
    mean = xr.mean(axis=axes, keepdims=True)
    var = xr.var(axis=axes, keepdims=True)
    xn = (xr - mean) / np.sqrt(var + eps)
    g = np.asarray(gamma).reshape(1, G, C // G, *([1] * len(spatial)))
    bt = np.asarray(beta).reshape(1, G, C // G, *([1] * len(spatial)))
    return (xn * g + bt).reshape(x.shape)


def layer_norm_last(x, gamma, beta, eps=1e-5):
    """``_layer_norm_np`` (``runtime/models/hubert.py:260-267``) -- the same
    formula as ``nn.layer_norm``'s numpy branch."""
    mean = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    xn = (x - mean) / np.sqrt(var + eps)
    return xn * gamma + beta


def grouped_conv1d(x, w, b, groups, stride=1, padding=0):
    """Per-group ``nn.conv1d`` then concat (``runtime/models/hubert.py:301-339``)."""
    x = np.asarray(x, dtype=_F32)
    w = np.asarray(w, dtype=_F32)
    O, Ci, _ = w.shape
    opg = O // groups
    parts = []
    for g in range(groups):
        parts.append(nn.conv1d(x[:, g * Ci:(g + 1) * Ci, :], w[g * opg:(g + 1) * opg],
                               b[g * opg:(g + 1) * opg] if b is not None else None,
                               stride=stride, padding=padding))
    return np.concatenate(parts, axis=1)


def pos_conv_weight(weight_g, weight_v):
    """weight_norm over dim 2: the L2 norm over dims (0, 1) per tap, computed
    in float64, then ``g * (v / norm)`` in float32
    (``runtime/models/hubert.py:510-522``)."""
    v = np.asarray(weight_v, dtype=_F32)
    g = np.asarray(weight_g, dtype=_F32)
    norm = np.sqrt(np.sum(v.astype(np.float64) ** 2, axis=(0, 1), keepdims=True))
    return (g * (v / norm.astype(_F32))).astype(_F32)


class HubertRef:
    """HuBERT-base encoder from a transformers-style state dict
    (keys as in ``runtime/models/hubert.py:524-558``)."""

    def __init__(self, sd: dict):
        self.sd = {k: np.asarray(v, dtype=_F32) for k, v in sd.items()}
        self.n_conv = 0
        while f"feature_extractor.conv_layers.{self.n_conv}.conv.weight" in self.sd:
            self.n_conv += 1
        self.n_layers = 0
        while f"encoder.layers.{self.n_layers}.attention.q_proj.weight" in self.sd:
            self.n_layers += 1
        self.pos_w = pos_conv_weight(self.sd["encoder.pos_conv_embed.conv.weight_g"],
                                     self.sd["encoder.pos_conv_embed.conv.weight_v"])

    def feature_extractor(self, x):
        """x [1, T] -> [1, L, 512] (``runtime/models/hubert.py:658-697``)."""
        h = np.asarray(x, _F32)[:, None, :]
        for i in range(self.n_conv):
            w = self.sd[f"feature_extractor.conv_layers.{i}.conv.weight"]
            h = nn.conv1d(h, w, None, stride=5 if i == 0 else 2, padding=0)
            if i == 0:
                h = group_norm(h, self.sd["feature_extractor.conv_layers.0.layer_norm.weight"],
                               self.sd["feature_extractor.conv_layers.0.layer_norm.bias"],
                               num_groups=h.shape[1], eps=1e-5)
            h = gelu_erf(h)
        return h.transpose(0, 2, 1)

    def feature_projection(self, h):
        """LayerNorm(512) -> ``x @ W.T`` -> ``+ b`` (``runtime/models/hubert.py:775-802``)."""
        h = nn.layer_norm(h, self.sd["feature_projection.layer_norm.weight"],
                          self.sd["feature_projection.layer_norm.bias"], eps=1e-5)
        out = nn.linear(h, self.sd["feature_projection.projection.weight"], None)
        return out + self.sd["feature_projection.projection.bias"].reshape(1, -1)

    def pos_conv_embed(self, h):
        """``runtime/models/hubert.py:838-858``: [1, L, C] -> [1, L, C]."""
        L = h.shape[1]
        x = h.transpose(0, 2, 1)
        groups = x.shape[1] // self.pos_w.shape[1]
        K = self.pos_w.shape[2]
        y = grouped_conv1d(x, self.pos_w, self.sd["encoder.pos_conv_embed.conv.bias"], groups=groups,
                           stride=1, padding=K // 2)
        y = y[:, :, :L]
        return gelu_erf(y).transpose(0, 2, 1)

    def attention(self, h, i):
        """``_attn_numpy`` (``runtime/models/hubert.py:1315-1338``)."""
        p = f"encoder.layers.{i}.attention."
        C = h.shape[-1]
        D = C // N_HEADS
        scale = D ** -0.5
        q = nn.linear(h, self.sd[p + "q_proj.weight"], self.sd[p + "q_proj.bias"]) * scale
        k = nn.linear(h, self.sd[p + "k_proj.weight"], self.sd[p + "k_proj.bias"])
        v = nn.linear(h, self.sd[p + "v_proj.weight"], self.sd[p + "v_proj.bias"])
        B, T, _ = q.shape
        qh = q.reshape(B, T, N_HEADS, D).transpose(0, 2, 1, 3)
        kh = k.reshape(B, T, N_HEADS, D).transpose(0, 2, 1, 3)
        vh = v.reshape(B, T, N_HEADS, D).transpose(0, 2, 1, 3)
        scores = np.matmul(qh, np.ascontiguousarray(kh.swapaxes(-1, -2)))
        m = scores.max(axis=-1, keepdims=True)
        e = np.exp(scores - m)
        w = e / e.sum(axis=-1, keepdims=True)
        ctx = np.matmul(w, np.ascontiguousarray(vh))
        ctx = ctx.transpose(0, 2, 1, 3).reshape(B, T, C)
        return nn.linear(ctx, self.sd[p + "out_proj.weight"], self.sd[p + "out_proj.bias"])

    def layer(self, h, i):
        """Post-LN layer (``runtime/models/hubert.py:1262-1288``, numpy FFN
        ``:1447-1451``)."""
        p = f"encoder.layers.{i}."
        h = h + self.attention(h, i)
        h = layer_norm_last(h, self.sd[p + "layer_norm.weight"], self.sd[p + "layer_norm.bias"], eps=1e-5)
        f = nn.linear(h, self.sd[p + "feed_forward.intermediate_dense.weight"],
                      self.sd[p + "feed_forward.intermediate_dense.bias"])
        f = nn.linear(gelu_erf(f), self.sd[p + "feed_forward.output_dense.weight"],
                      self.sd[p + "feed_forward.output_dense.bias"])
        h = h + f
        return layer_norm_last(h, self.sd[p + "final_layer_norm.weight"], self.sd[p + "final_layer_norm.bias"],
                               eps=1e-5)

    def encoder(self, h, upto=None):
        """``runtime/models/hubert.py:928-968`` (numpy branch); returns the
        hidden states [entry, layer 1, ..., layer n]."""
        h = h + self.pos_conv_embed(h)
        h = layer_norm_last(h, self.sd["encoder.layer_norm.weight"], self.sd["encoder.layer_norm.bias"], eps=1e-5)
        outs = [h]
        n = self.n_layers if upto is None else upto
        for i in range(n):
            h = self.layer(h, i)
            outs.append(h)
        return outs

    def encode(self, x, version=2):
        """``runtime/models/hubert.py:564-591``."""
        h = self.feature_projection(self.feature_extractor(x))
        if version == 1:
            hs = self.encoder(h, upto=9)
            return nn.linear(hs[9], self.sd["final_proj.weight"], self.sd["final_proj.bias"])
        return self.encoder(h)[-1]
