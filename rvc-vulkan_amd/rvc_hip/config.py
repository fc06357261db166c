# -*- coding: utf-8 -*-
"""Synthesizer geometry from a checkpoint weight dict (host logic).

Same derivation rules as the reference's ``VitsConfig``
(``runtime/models/vits.py:166-268``): encoder sizes from weight shapes; the
upsample rates from the checkpoint ``config`` list when it has them, else
inferred from the noise-conv kernels with the 48k total upsampling of 480,
where an explicit ``sr`` re-derives the first rate so that
``prod(rates) == sr // 100``; ResBlock kernels [3,7,11] and dilations
[1,3,5] are fixed.
"""

from __future__ import annotations

import math

__all__ = ["VitsConfig"]

_UPP_48K = 480


class VitsConfig:
    def __init__(self, w: dict, config=None, sr: int | None = None):
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
        n_ups = 0
        while f"dec.ups.{n_ups}.weight_v" in w:
            n_ups += 1
        kernels_from_w = [int(w[f"dec.ups.{i}.weight_v"].shape[2]) for i in range(n_ups)]
        if cfg and len(cfg) > 12:
            self.upsample_rates = [int(r) for r in cfg[12]]
            self.upsample_initial = int(cfg[13])
            self.sr = int(sr) if sr else (int(cfg[17]) if len(cfg) > 17 else 48000)
            if len(cfg) > 14 and cfg[14] is not None and cfg[14] != "":
                self.upsample_kernels = [int(k) for k in cfg[14]]
            else:
                self.upsample_kernels = kernels_from_w
        else:
            strides = [int(w[f"dec.noise_convs.{i}.weight"].shape[2]) // 2 if i < n_ups - 1 else 1
                       for i in range(n_ups)]
            rates = [strides[i] // strides[i + 1] for i in range(n_ups - 1)]
            rates.insert(0, _UPP_48K // strides[0])
            self.upsample_rates = rates
            self.sr = int(sr) if sr else 48000
            if sr:
                rest = math.prod(self.upsample_rates[1:])
                self.upsample_rates[0] = int(self.sr // 100) // rest
            self.upsample_kernels = kernels_from_w
        self.n_ups = len(self.upsample_rates) or n_ups
        self.upp = int(math.prod(self.upsample_rates))
        self.noise_strides = [int(w[f"dec.noise_convs.{i}.weight"].shape[2]) // 2 if i < self.n_ups - 1 else 1
                              for i in range(self.n_ups)]
        self.resblock_kernel_sizes = [3, 7, 11]
        self.resblock_dilation_sizes = [[1, 3, 5], [1, 3, 5], [1, 3, 5]]
        self.n_spk = int(w["emb_g.weight"].shape[0])
        self.gin_channels = int(w["emb_g.weight"].shape[1])

    def __repr__(self):
        fields = ("sr", "phone_dim", "hidden", "filter", "n_heads", "n_layers", "n_spk", "gin_channels",
                  "upsample_rates", "upsample_kernels")
        return "VitsConfig<" + " ".join(f"{k}:{getattr(self, k)}" for k in fields) + ">"
