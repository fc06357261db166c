# -*- coding: utf-8 -*-
"""Device-resident RMVPE pitch extractor on the HIP backend.

``HipRMVPE`` has the inference surface of the reference's ``RMVPE``
(``runtime/models/rmvpe.py:554-952``): ``infer_from_audio(x, thred=0.03)``
maps 16 kHz mono audio ``[T]`` to f0 ``[1 + T // 160]`` in Hz (0 where
unvoiced), ``mel2hidden`` gives the salience ``[1, F, 360]`` and ``decode``
turns a salience into f0.  The reference loads ``rmvpe.pt``; here the caller
passes the state dict (checkpoint key names, float arrays) -- or uses
``rvc_hip.checkpoint.load_rmvpe(path)`` -- and construction uploads every
weight once into a ``rvc_rmvpe`` session (BatchNorm folded into the convs).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _hip
from .hip_ops import HipContext, get_context

__all__ = ["HipRMVPE"]

_F32P = ctypes.POINTER(ctypes.c_float)
HOP = 160
N_MELS = 128


class HipRMVPE:
    """RMVPE (``E2E(4, 1, (2, 2))``) with every weight resident on one MI355X."""

    def __init__(self, sd: dict, ctx: HipContext | None = None):
        self.ctx = ctx or get_context()
        self._lib = _hip.get_lib()
        self.handle = int(self._lib.rvc_rmvpe_create(self.ctx.handle))
        if self.handle < 0:
            raise RuntimeError(f"rvc_rmvpe_create failed: {_hip.last_error()}")
        for key, arr in sd.items():
            a = np.asarray(arr)
            if a.dtype.kind not in "fiu" or key.endswith("num_batches_tracked"):
                continue
            a = np.ascontiguousarray(a, dtype=np.float32)
            shape = (ctypes.c_int64 * max(a.ndim, 1))(*(a.shape if a.ndim else (1,)))
            _hip._check(self._lib.rvc_rmvpe_set_weight(self.handle, key.encode(), a.ctypes.data_as(_F32P), shape,
                                                        max(a.ndim, 1)), f"rvc_rmvpe_set_weight({key})")
        _hip._check(self._lib.rvc_rmvpe_finalize(self.handle), "rvc_rmvpe_finalize")
        self.n_bins = int(np.asarray(sd["fc.1.weight"]).shape[0])
        self.gru_hidden = int(np.asarray(sd["fc.0.gru.weight_hh_l0"]).shape[1])

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle > 0:
            self._lib.rvc_rmvpe_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            import sys

            if not sys.is_finalizing():
                self.close()
        except Exception:  # noqa: BLE001
            pass

    @staticmethod
    def frames(T: int) -> int:
        return 1 + int(T) // HOP

    @staticmethod
    def padded(F: int) -> int:
        return 32 * ((F - 1) // 32 + 1)

    def infer_from_audio(self, x, thred: float = 0.03) -> np.ndarray:
        """``[T]`` float32 16 kHz -> ``[F]`` float32 f0 (Hz); the reference's
        ``RMVPE.infer_from_audio`` (``runtime/models/rmvpe.py:927-952``)."""
        x = np.asarray(x, dtype=np.float32)
        if x.ndim != 1:
            raise ValueError(f"infer_from_audio needs 1-D audio, got {x.ndim}-D")
        x = np.ascontiguousarray(x)
        f0 = np.empty(self.frames(len(x)), dtype=np.float32)
        _hip._check(self._lib.rvc_rmvpe_infer(self.handle, x.ctypes.data_as(_F32P), len(x), float(thred),
                                              f0.ctypes.data_as(_F32P)), "rvc_rmvpe_infer")
        self._last_T = len(x)
        return f0

    def infer_dev(self, x_buf, T: int, f0_buf, thred: float = 0.03) -> None:
        """Device-resident form on engine buffers (audio [T] -> f0 [F])."""
        _hip._check(self._lib.rvc_rmvpe_infer_dev(self.handle, int(x_buf), int(T), float(thred), int(f0_buf)),
                    "rvc_rmvpe_infer_dev")
        self._last_T = int(T)

    def read(self, name: str, shape) -> np.ndarray:
        out = np.empty(shape, dtype=np.float32)
        _hip._check(self._lib.rvc_rmvpe_read(self.handle, name.encode(), out.ctypes.data_as(_F32P), out.size),
                    f"rvc_rmvpe_read({name})")
        return out

    def last_mel(self) -> np.ndarray:
        """log-mel ``[128, F]`` of the last call (``RMVPE._extract_mel``)."""
        return self.read("mel", (N_MELS, self.frames(self._last_T)))

    def last_hidden(self) -> np.ndarray:
        """Salience ``[1, F, 360]`` of the last call (``RMVPE.mel2hidden``)."""
        F = self.frames(self._last_T)
        s = self.read("salience", (self.n_bins, self.padded(F)))
        return np.ascontiguousarray(s.T[:F])[None]

    def mel2hidden_from_audio(self, x) -> np.ndarray:
        self.infer_from_audio(x)
        return self.last_hidden()

    def set_timing(self, tag: str) -> None:
        _hip._check(self._lib.rvc_rmvpe_set_timing(self.handle, tag.encode()), "rvc_rmvpe_set_timing")

    def timing(self) -> dict:
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        n = ctypes.c_int64()
        _hip._check(self._lib.rvc_rmvpe_get_timing(self.handle, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(fl),
                                                   ctypes.byref(by)), "rvc_rmvpe_get_timing")
        return {"ms": ms.value, "launches": n.value, "flops": fl.value, "bytes": by.value}
