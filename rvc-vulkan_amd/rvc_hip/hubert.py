# -*- coding: utf-8 -*-
"""Device-resident HuBERT-base encoder on the HIP backend.

``HipHubert`` has the inference surface of the reference's ``HubertEncoder``
(``runtime/models/hubert.py:355-591``): ``encode(x, version=2)`` maps a
16 kHz waveform ``[1, T]`` (or ``[B, T]`` for B equal-length chunks) to
``[B, L, 768]`` (version 2, last hidden state) or ``[B, L, 256]`` (version 1,
``final_proj`` of layer 9).  The reference loads ``pytorch_model.bin``; here
the caller passes the state dict (transformers key names, float arrays), and
construction uploads every weight once into a ``rvc_hubert`` session.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _hip
from .hip_ops import HipContext, get_context

__all__ = ["HipHubert"]

_F32P = ctypes.POINTER(ctypes.c_float)


class HipHubert:
    """HuBERT-base with every weight resident on one MI355X."""

    def __init__(self, sd: dict, ctx: HipContext | None = None):
        self.ctx = ctx or get_context()
        self._lib = _hip.get_lib()
        self.handle = int(self._lib.rvc_hubert_create(self.ctx.handle))
        if self.handle < 0:
            raise RuntimeError(f"rvc_hubert_create failed: {_hip.last_error()}")
        for key, arr in sd.items():
            a = np.ascontiguousarray(np.asarray(arr, dtype=np.float32))
            shape = (ctypes.c_int64 * max(a.ndim, 1))(*(a.shape if a.ndim else (1,)))
            _hip._check(self._lib.rvc_hubert_set_weight(self.handle, key.encode(), a.ctypes.data_as(_F32P), shape,
                                                        max(a.ndim, 1)), f"rvc_hubert_set_weight({key})")
        _hip._check(self._lib.rvc_hubert_finalize(self.handle), "rvc_hubert_finalize")
        self.hidden = int(np.asarray(sd["feature_projection.projection.weight"]).shape[0])
        self.conv_dim = int(np.asarray(sd["feature_projection.projection.weight"]).shape[1])
        self.final_dim = int(np.asarray(sd["final_proj.weight"]).shape[0]) if "final_proj.weight" in sd else 0

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle > 0:
            self._lib.rvc_hubert_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            import sys

            if not sys.is_finalizing():
                self.close()
        except Exception:  # noqa: BLE001
            pass

    def frames(self, T: int) -> int:
        out = ctypes.c_int64()
        _hip._check(self._lib.rvc_hubert_frames(self.handle, int(T), ctypes.byref(out)), "rvc_hubert_frames")
        return int(out.value)

    def encode(self, x, version: int = 2) -> np.ndarray:
        """x [T] / [1,T] / [B,T] float32 -> [B, L, 768] (version 2) or
        [B, L, 256] (version 1); the reference's contract
        (``runtime/models/hubert.py:564-591``) with a batch of equal-length
        chunks allowed."""
        if version not in (1, 2):
            raise ValueError(f"version must be 1 or 2, got {version}")
        x = np.asarray(x, dtype=np.float32)
        if x.ndim == 1:
            x = x[None, :]
        if x.ndim != 2:
            raise ValueError(f"input must be [B, T], got {x.shape}")
        x = np.ascontiguousarray(x)
        B, T = x.shape
        L = self.frames(T)
        if L < 1:
            raise ValueError(f"input of {T} samples is shorter than the feature extractor's receptive field")
        od = self.hidden if version == 2 else self.final_dim
        out = np.empty((B, L, od), dtype=np.float32)
        _hip._check(self._lib.rvc_hubert_encode(self.handle, x.ctypes.data_as(_F32P), B, T, int(version),
                                                out.ctypes.data_as(_F32P)), "rvc_hubert_encode")
        return out

    def encode_batch(self, xs, version: int = 2) -> list:
        """The reference's ``encode_batch`` (``runtime/models/hubert.py:593-656``):
        a list of ``[1, T_i]`` (or ``[T_i]``) chunks of possibly different
        lengths -> a list of ``[1, L_i, D]``, each equal to ``encode`` of that
        chunk.  Chunks of equal length run as one batched call (bit-identical
        to running them one by one), in input order."""
        if version not in (1, 2):
            raise ValueError(f"version must be 1 or 2, got {version}")
        if isinstance(xs, np.ndarray):
            xs = [xs]
        xl = []
        for x in xs:
            x = np.asarray(x, dtype=np.float32)
            if x.ndim == 1:
                x = x[None, :]
            if x.ndim != 2 or x.shape[0] != 1:
                raise ValueError(f"each chunk must be [1, T], got {x.shape}")
            xl.append(x)
        out: list = [None] * len(xl)
        by_len: dict = {}
        for i, x in enumerate(xl):
            by_len.setdefault(x.shape[1], []).append(i)
        for idx in by_len.values():
            y = self.encode(np.concatenate([xl[i] for i in idx], axis=0), version)
            for j, i in enumerate(idx):
                out[i] = y[j:j + 1]
        return out

    def encode_dev(self, x_id: int, B: int, T: int, out_id: int, version: int = 2):
        _hip._check(self._lib.rvc_hubert_encode_dev(self.handle, int(x_id), int(B), int(T), int(version), int(out_id)),
                    "rvc_hubert_encode_dev")

    def read(self, name: str, shape):
        out = np.empty(shape, dtype=np.float32)
        _hip._check(self._lib.rvc_hubert_read(self.handle, name.encode(), out.ctypes.data_as(_F32P), out.size),
                    f"rvc_hubert_read({name})")
        return out

    def set_debug(self, keep: bool):
        _hip._check(self._lib.rvc_hubert_set_debug(self.handle, int(bool(keep))), "rvc_hubert_set_debug")

    def set_timing(self, tag: str):
        _hip._check(self._lib.rvc_hubert_set_timing(self.handle, tag.encode()), "rvc_hubert_set_timing")

    def get_timing(self):
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        n = ctypes.c_int64()
        _hip._check(self._lib.rvc_hubert_get_timing(self.handle, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(fl),
                                                    ctypes.byref(by)), "rvc_hubert_get_timing")
        return {"ms": ms.value, "launches": n.value, "flops": fl.value, "bytes": by.value}
