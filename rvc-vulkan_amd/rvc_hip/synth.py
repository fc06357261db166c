# -*- coding: utf-8 -*-
"""Device-resident RVC synthesizer on the HIP backend.

``HipSynthesizer`` has the inference surface of the reference's
``SynthesizerTrn`` (``runtime/models/vits.py:2237-2595``) -- ``infer``,
``infer_controlled``, ``decode_batch`` -- plus ``dec_forward`` for the
decoder alone (``_GeneratorNSF.forward``, ``:2133-2231``).  Construction
uploads every weight once into a ``rvc_synth`` session (the analogue of
``register_persistent_weights``, ``:2272-2334``); each call then runs
enc_p + flow + GeneratorNSF as one stream of HIP kernels with a single
upload of the inputs and a single download of the waveform.

Batching: ``phone`` / ``z`` may carry a leading batch of B independent
chunks of equal length; they run as one batched launch sequence.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _hip
from .config import VitsConfig
from .hip_ops import HipContext, get_context

__all__ = ["HipSynthesizer"]

_F32P = ctypes.POINTER(ctypes.c_float)
_I64P = ctypes.POINTER(ctypes.c_int64)

READABLE = ("enc_in", "enc_out", "stats", "z_p", "z", "g", "har", "dec_pre")


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i64(a):
    a = np.asarray(a)
    if not np.issubdtype(a.dtype, np.integer):
        raise TypeError(f"expected an integer array, got dtype={a.dtype}")
    return np.ascontiguousarray(a, dtype=np.int64)


class HipSynthesizer:
    """RVC v2 synthesizer with every weight resident on one MI355X."""

    def __init__(self, w: dict, config=None, sr: int | None = None, ctx: HipContext | None = None,
                 geometry=None, precision: int = 0):
        """``config`` / ``sr`` derive the geometry like the reference's
        ``VitsConfig``; ``geometry`` (any object with ``upsample_rates``,
        ``upsample_kernels`` and ``sr``, e.g. a reference ``VitsConfig``)
        overrides those three.  ``precision``: 0 fp32 (default); 1 the
        upsample ConvTranspose1d and the enc_p matmuls on bf16 MFMA with fp32
        accumulate; 2 also the decoder ResBlock convs."""
        self.cfg = VitsConfig(w, config, sr=sr)
        if geometry is not None:
            self.cfg.upsample_rates = [int(r) for r in geometry.upsample_rates]
            self.cfg.upsample_kernels = [int(k) for k in geometry.upsample_kernels]
            self.cfg.sr = int(geometry.sr)
            self.cfg.n_ups = len(self.cfg.upsample_rates)
            self.cfg.upp = int(np.prod(self.cfg.upsample_rates))
        self.ctx = ctx or get_context()
        self._lib = _hip.get_lib()
        self.handle = int(self._lib.rvc_synth_create(self.ctx.handle))
        if self.handle < 0:
            raise RuntimeError(f"rvc_synth_create failed: {_hip.last_error()}")
        self._w = w
        self.precision = int(precision)
        _hip._check(self._lib.rvc_synth_set_precision(self.handle, self.precision), "rvc_synth_set_precision")
        for key, arr in w.items():
            a = _f32(arr)
            shape = (ctypes.c_int64 * max(a.ndim, 1))(*(a.shape if a.ndim else (1,)))
            _hip._check(self._lib.rvc_synth_set_weight(self.handle, key.encode(), a.ctypes.data_as(_F32P),
                                                       shape, max(a.ndim, 1)), f"rvc_synth_set_weight({key})")
        c = self.cfg
        rates = (ctypes.c_int64 * c.n_ups)(*c.upsample_rates)
        kernels = (ctypes.c_int64 * c.n_ups)(*c.upsample_kernels)
        _hip._check(self._lib.rvc_synth_finalize(self.handle, c.sr, rates, kernels, c.n_ups),
                    "rvc_synth_finalize")

    # ------------------------------------------------------------------ lifecycle
    def close(self):
        if getattr(self, "handle", None) is not None and self.handle > 0:
            self._lib.rvc_synth_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            import sys

            if not sys.is_finalizing():
                self.close()
        except Exception:  # noqa: BLE001
            pass

    # ------------------------------------------------------------------ inference
    def make_noise(self, P: int, seed):
        """nz [1,hidden,P] then ns [1,P*upp,1] from one RandomState
        (``runtime/models/vits.py:2337-2350``)."""
        rng = np.random.RandomState(seed)
        nz = rng.standard_normal((1, self.cfg.hidden, P)).astype(np.float32)
        ns = rng.standard_normal((1, P * self.cfg.upp, 1)).astype(np.float32)
        return nz, ns

    def infer(self, phone, pitch, nsff0, sid, seed=None):
        nz, ns = self.make_noise(np.asarray(phone).shape[1], seed)
        return self.infer_controlled(phone, pitch, nsff0, sid, nz, ns)

    def infer_controlled(self, phone, pitch, nsff0, sid, nz, ns):
        """phone [B,P,D], pitch int [B,P], nsff0 [B,P], sid int [1] or [B],
        nz [B,hidden,P], ns [B,P*upp(,1)] -> wave [B,1,P*upp]."""
        phone = _f32(phone)
        if phone.ndim != 3 or phone.shape[2] != self.cfg.phone_dim:
            raise ValueError(f"phone must be [B,P,{self.cfg.phone_dim}], got {phone.shape}")
        B, P, _ = phone.shape
        pitch = _i64(pitch).reshape(B, P)
        nsff0 = _f32(nsff0).reshape(B, P)
        sid = _i64(sid).reshape(-1)
        if sid.size == 1 and B > 1:
            sid = np.repeat(sid, B)
        if sid.size != B:
            raise ValueError(f"sid must have 1 or B={B} entries")
        nz = _f32(nz).reshape(B, self.cfg.hidden, P)
        ns = _f32(ns).reshape(B, P * self.cfg.upp)
        wave = np.empty((B, 1, P * self.cfg.upp), dtype=np.float32)
        _hip._check(self._lib.rvc_synth_infer(
            self.handle, phone.ctypes.data_as(_F32P), pitch.ctypes.data_as(_I64P), nsff0.ctypes.data_as(_F32P),
            sid.ctypes.data_as(_I64P), nz.ctypes.data_as(_F32P), ns.ctypes.data_as(_F32P), B, P,
            wave.ctypes.data_as(_F32P)), "rvc_synth_infer")
        return wave

    def dec_forward(self, z, f0, g, ns):
        """GeneratorNSF only: z [B,hidden,P], f0 [B,P], g [B,gin(,1)], ns [B,P*upp(,1)]
        -> [B,1,P*upp]."""
        z = _f32(z)
        if z.ndim != 3 or z.shape[1] != self.cfg.hidden:
            raise ValueError(f"z must be [B,{self.cfg.hidden},P], got {z.shape}")
        B, _, P = z.shape
        f0 = _f32(f0).reshape(B, P)
        g = _f32(g).reshape(-1, self.cfg.gin_channels)
        if g.shape[0] == 1 and B > 1:
            g = np.ascontiguousarray(np.repeat(g, B, axis=0))
        if g.shape[0] != B:
            raise ValueError("g must have 1 or B rows")
        ns = _f32(ns).reshape(B, P * self.cfg.upp)
        wave = np.empty((B, 1, P * self.cfg.upp), dtype=np.float32)
        _hip._check(self._lib.rvc_synth_decode(
            self.handle, z.ctypes.data_as(_F32P), f0.ctypes.data_as(_F32P), g.ctypes.data_as(_F32P),
            ns.ctypes.data_as(_F32P), B, P, wave.ctypes.data_as(_F32P)), "rvc_synth_decode")
        return wave

    def decode_batch(self, z_list, g, f0_list, ns_list):
        """Multi-chunk decode (``runtime/models/vits.py:1847-1878``): chunks of
        equal length run as one batch, others one by one."""
        if not z_list:
            return []
        lens = {np.asarray(z).shape[-1] for z in z_list}
        if len(lens) == 1:
            z = np.concatenate([np.asarray(z, np.float32).reshape(1, self.cfg.hidden, -1) for z in z_list])
            f0 = np.concatenate([np.asarray(f, np.float32).reshape(1, -1) for f in f0_list])
            ns = np.concatenate([np.asarray(n, np.float32).reshape(1, -1) for n in ns_list])
            w = self.dec_forward(z, f0, g, ns)
            return [w[i:i + 1] for i in range(len(z_list))]
        return [self.dec_forward(z, f, g, n) for z, f, n in zip(z_list, f0_list, ns_list)]

    # ------------------------------------------------------------------ device-resident calls
    def infer_dev(self, phone_id, pitch_id, f0_id, sid_id, nz_id, ns_id, B, P, wave_id):
        """All arguments are engine buffer ids of resident inputs (pitch/sid int64)."""
        _hip._check(self._lib.rvc_synth_infer_dev(self.handle, phone_id, pitch_id, f0_id, sid_id, nz_id, ns_id,
                                                  B, P, wave_id), "rvc_synth_infer_dev")

    def decode_dev(self, z_id, f0_id, g_id, ns_id, B, P, wave_id):
        _hip._check(self._lib.rvc_synth_decode_dev(self.handle, z_id, f0_id, g_id, ns_id, B, P, wave_id),
                    "rvc_synth_decode_dev")

    # ------------------------------------------------------------------ introspection
    def read(self, name: str, shape):
        """Download a named intermediate of the last call (see ``READABLE``,
        plus ``dec_stage<i>`` after ``set_debug(True)``)."""
        out = np.empty(shape, dtype=np.float32)
        _hip._check(self._lib.rvc_synth_read(self.handle, name.encode(), out.ctypes.data_as(_F32P), out.size),
                    f"rvc_synth_read({name})")
        return out

    def set_debug(self, keep_stages: bool):
        _hip._check(self._lib.rvc_synth_set_debug(self.handle, int(bool(keep_stages))), "rvc_synth_set_debug")

    def set_timing(self, tag: str):
        _hip._check(self._lib.rvc_synth_set_timing(self.handle, tag.encode()), "rvc_synth_set_timing")

    def get_timing(self):
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        n = ctypes.c_int64()
        _hip._check(self._lib.rvc_synth_get_timing(self.handle, ctypes.byref(ms), ctypes.byref(n),
                                                   ctypes.byref(fl), ctypes.byref(by)), "rvc_synth_get_timing")
        return {"ms": ms.value, "launches": n.value, "flops": fl.value, "bytes": by.value}
