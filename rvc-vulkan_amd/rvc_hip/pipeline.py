# -*- coding: utf-8 -*-
"""The conversion glue around synthesis on the HIP backend.

Mirrors the steps of the reference's ``runtime/pipeline.py`` that sit either
side of ``SynthesizerTrn.infer`` and ``runtime/retrieval.py``'s brute-force
search, with the same names, argument meaning and array contracts:

* ``search_l2(query, db, k=8)`` (``runtime/retrieval.py:35-83``) and
  ``HipFeatureIndex`` (the ``FeatureIndex`` search surface,
  ``runtime/retrieval.py:100-160``): the index stays resident on the GPU;
* ``HipPipeline._vc_prepare`` / ``vc`` (``runtime/pipeline.py:488-695``):
  retrieval blend, 2x feature interpolation, pitch alignment and the protect
  mask on the device, then synthesis;
* ``change_rms(data1, data2, sr1, sr2, rate)`` (``runtime/pipeline.py:164-188``)
  and ``HipPipeline.to_int16`` (``runtime/pipeline.py:1208-1213``).

Retrieval follows the reference's ``FeatureIndex`` branch (brute force over
every index row).  The inverted-file branch (``IVFIndex``, nprobe buckets,
``runtime/pipeline.py:66-161, 524-545``) is an approximation of it that this
backend does not reproduce: passing an index with ``vectors_by_rows`` raises
``NotImplementedError``.  Nothing here computes on the CPU except index
bookkeeping and the pitch alignment (a pad / truncate of int arrays).
"""

from __future__ import annotations

import ctypes
from time import time as ttime

import numpy as np

from . import _hip
from .hip_ops import HipContext, get_context

__all__ = ["K_SEARCH", "HipVcGlue", "HipFeatureIndex", "HipPipeline", "search_l2", "change_rms"]

K_SEARCH = 8  # runtime/pipeline.py:55
_F32P = ctypes.POINTER(ctypes.c_float)
_I64P = ctypes.POINTER(ctypes.c_int64)


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


class HipVcGlue:
    """One ``rvc_vc`` session: an optional resident index plus the glue ops."""

    def __init__(self, ctx: HipContext | None = None):
        self.ctx = ctx or get_context()
        self._lib = _hip.get_lib()
        self.handle = int(self._lib.rvc_vc_create(self.ctx.handle))
        if self.handle < 0:
            raise RuntimeError(f"rvc_vc_create failed: {_hip.last_error()}")
        self.ntotal = 0
        self.dim = 0

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle > 0:
            self._lib.rvc_vc_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            import sys

            if not sys.is_finalizing():
                self.close()
        except Exception:  # noqa: BLE001
            pass

    def set_index(self, vectors):
        v = _f32(vectors)
        if v.ndim != 2 or v.shape[0] < 1 or v.shape[1] < 1:
            raise ValueError(f"index vectors must be a non-empty [N, D] array, got {v.shape}")
        _hip._check(self._lib.rvc_vc_set_index(self.handle, v.ctypes.data_as(_F32P), v.shape[0], v.shape[1]),
                    "rvc_vc_set_index")
        self.ntotal, self.dim = int(v.shape[0]), int(v.shape[1])

    def search(self, query, k: int = K_SEARCH):
        """(scores [F, min(k, N)] float32 ascending, indices [F, min(k, N)] int64)."""
        q = _f32(query)
        if q.ndim != 2 or q.shape[1] != self.dim:
            raise ValueError(f"query must be [F, {self.dim}], got {q.shape}")
        if self.ntotal == 0:
            raise ValueError("search: no index vectors")
        k = min(int(k), self.ntotal)
        if k > K_SEARCH:
            raise ValueError(f"search: k <= {K_SEARCH} supported, got {k}")
        F = q.shape[0]
        scores = np.full((F, k), np.inf, dtype=np.float32)
        inds = np.full((F, k), -1, dtype=np.int64)
        if F:
            _hip._check(self._lib.rvc_vc_search(self.handle, q.ctypes.data_as(_F32P), F, k,
                                                scores.ctypes.data_as(_F32P), inds.ctypes.data_as(_I64P)),
                        "rvc_vc_search")
        return scores, inds

    def prepare(self, feats, index_rate: float, pitchf=None, protect: float = 0.5):
        """feats [F, D] -> [2F, D]: retrieval blend (index_rate != 0 and an
        index set), 2x interpolation, protect mask with pitchf [2F] (or none)."""
        x = _f32(feats)
        if x.ndim != 2:
            raise ValueError(f"feats must be [F, D], got {x.shape}")
        F, D = x.shape
        out = np.empty((2 * F, D), dtype=np.float32)
        if F == 0:
            return out
        pf = None
        if pitchf is not None:
            pf = _f32(pitchf).reshape(-1)
            if pf.shape[0] != 2 * F:
                raise ValueError(f"pitchf must hold {2 * F} frames, got {pf.shape[0]}")
        _hip._check(self._lib.rvc_vc_prepare(self.handle, x.ctypes.data_as(_F32P), F, D, float(index_rate),
                                             pf.ctypes.data_as(_F32P) if pf is not None else None,
                                             float(protect), out.ctypes.data_as(_F32P)), "rvc_vc_prepare")
        return out

    def prepare_dev(self, feats_id: int, F: int, D: int, index_rate: float, pitchf_id: int, protect: float,
                    out_id: int):
        _hip._check(self._lib.rvc_vc_prepare_dev(self.handle, int(feats_id), int(F), int(D), float(index_rate),
                                                 int(pitchf_id), float(protect), int(out_id)), "rvc_vc_prepare_dev")

    def change_rms(self, data1, data2, sr1, sr2, rate):
        a = _f32(data1).reshape(-1)
        b = _f32(data2).reshape(-1)
        out = np.empty_like(b)
        if b.shape[0] == 0:
            return out
        _hip._check(self._lib.rvc_vc_change_rms(self.handle, a.ctypes.data_as(_F32P), a.shape[0], int(sr1),
                                                b.ctypes.data_as(_F32P), b.shape[0], int(sr2), float(rate),
                                                out.ctypes.data_as(_F32P)), "rvc_vc_change_rms")
        return out

    def change_rms_dev(self, d1_id, n1, sr1, d2_id, n2, sr2, rate, out_id):
        _hip._check(self._lib.rvc_vc_change_rms_dev(self.handle, int(d1_id), int(n1), int(sr1), int(d2_id), int(n2),
                                                    int(sr2), float(rate), int(out_id)), "rvc_vc_change_rms_dev")

    def to_int16(self, audio):
        x = _f32(audio).reshape(-1)
        out = np.empty(x.shape[0], dtype=np.int16)
        if x.shape[0]:
            _hip._check(self._lib.rvc_vc_to_int16(self.handle, x.ctypes.data_as(_F32P), x.shape[0],
                                                  out.ctypes.data_as(ctypes.POINTER(ctypes.c_int16))),
                        "rvc_vc_to_int16")
        return out

    def set_timing(self, tag: str):
        _hip._check(self._lib.rvc_vc_set_timing(self.handle, tag.encode()), "rvc_vc_set_timing")

    def get_timing(self):
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        n = ctypes.c_int64()
        _hip._check(self._lib.rvc_vc_get_timing(self.handle, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(fl),
                                                ctypes.byref(by)), "rvc_vc_get_timing")
        return {"ms": ms.value, "launches": n.value, "flops": fl.value, "bytes": by.value}


class HipFeatureIndex:
    """The search surface of the reference's ``FeatureIndex``
    (``runtime/retrieval.py:100-160``) with the vectors resident on the GPU:
    ``ntotal``, ``dim``, ``metric``, ``search(query, k)``, ``reconstruct`` /
    ``reconstruct_n`` (host copies)."""

    def __init__(self, vectors, ctx: HipContext | None = None):
        self._vectors = _f32(vectors)
        self.metric = "L2"
        self._glue = HipVcGlue(ctx)
        self._glue.set_index(self._vectors)

    @property
    def ntotal(self) -> int:
        return int(self._vectors.shape[0])

    @property
    def dim(self) -> int:
        return int(self._vectors.shape[1])

    def search(self, query, k: int = K_SEARCH):
        return self._glue.search(query, k)

    def reconstruct(self, i: int):
        return self._vectors[i].copy()

    def reconstruct_n(self, start: int, n: int):
        return self._vectors[start:start + n].copy()


def search_l2(query, db, k: int = K_SEARCH, chunk: int = 4096):
    """``runtime/retrieval.py:35-83`` on the GPU (``chunk`` is accepted for the
    signature; the device searches every row in one pass)."""
    del chunk
    db = _f32(db)
    if db.ndim != 2 or db.shape[0] == 0:
        raise ValueError(f"db must be a non-empty [N, D] array, got {db.shape}")
    glue = HipVcGlue()
    try:
        glue.set_index(db)
        return glue.search(query, k)
    finally:
        glue.close()


def change_rms(data1, data2, sr1, sr2, rate):
    """``runtime/pipeline.py:164-188``: ``data2`` scaled by the RMS envelopes,
    ``rms1^(1-rate) * max(rms2, 1e-6)^(rate-1)``."""
    glue = HipVcGlue()
    try:
        return glue.change_rms(data1, data2, sr1, sr2, rate)
    finally:
        glue.close()


class HipPipeline:
    """The per-chunk conversion path of the reference's ``Pipeline``
    (``runtime/pipeline.py:368-695``) on the GPU.  ``tgt_sr`` and ``x_pad``
    as in the reference's constructor (``runtime/pipeline.py:386-406``)."""

    def __init__(self, tgt_sr: int, x_pad: int = 1, ctx: HipContext | None = None):
        self.sr = 16000
        self.window = 160
        self.x_pad = int(x_pad)
        self.t_pad = self.sr * self.x_pad
        self.t_pad_tgt = int(tgt_sr) * self.x_pad
        self.glue = HipVcGlue(ctx)
        self._index_key = None

    def _resident(self, index, index_vectors):
        """Make the FeatureIndex's vectors the session's resident index (once
        per distinct array)."""
        if index is not None and getattr(index, "vectors_by_rows", None) is not None and index_vectors is None:
            raise NotImplementedError("inverted-file (IVFIndex) retrieval is not provided by the HIP backend; "
                                      "pass a FeatureIndex or index_vectors for brute-force retrieval")
        if str(getattr(index, "metric", "L2")).upper() == "IP":
            raise NotImplementedError("retrieval needs an L2 index (the (1/score)^2 weights are L2 semantics)")
        vecs = index_vectors if index_vectors is not None else getattr(index, "_vectors", None)
        if vecs is None:
            raise ValueError("retrieval needs the index vectors")
        key = (id(vecs), np.shape(vecs))
        if key != self._index_key:
            self.glue.set_index(vecs)
            self._index_key = key
            self._index_ref = vecs

    def _vc_prepare(self, model, sid, audio0, pitch, pitchf, times, index, index_vectors, index_rate, version,
                    protect, feats=None, retrieval_mode="ivf", brute_mix=0.0):
        """``runtime/pipeline.py:488-614`` (FeatureIndex retrieval): returns
        ``{"feats" [1, 2L, D], "pitch", "pitchf", "sid_arr"}``."""
        if brute_mix != 0.0:
            raise NotImplementedError("brute_mix mixes IVF and brute-force retrieval; only brute force is provided")
        audio0 = np.asarray(audio0, dtype=np.float32)
        t0 = ttime()
        if audio0.ndim == 2:
            audio0 = audio0.mean(-1)
        if audio0.ndim != 1:
            raise ValueError(f"audio0 must be 1-D, got {audio0.ndim}-D")
        if feats is None:
            feats = model.encode(audio0[None, :], version=int(str(version).lstrip("v")))
        feats = _f32(feats)
        if feats.ndim != 3 or feats.shape[0] != 1:
            raise ValueError(f"feats must be [1, L, D], got {feats.shape}")
        L = feats.shape[1]
        use_index = index is not None and index_rate != 0 and getattr(index, "ntotal", 0) > 0
        if use_index:
            self._resident(index, index_vectors)
        protect_on = protect < 0.5 and pitch is not None and pitchf is not None
        if pitch is not None and pitchf is not None:
            pitch = np.asarray(pitch)
            pitchf = np.asarray(pitchf, dtype=np.float32)
            n, m = 2 * L, pitch.shape[1]
            if m < n:
                pitch = np.concatenate([pitch, np.repeat(pitch[:, -1:], n - m, axis=1)], axis=1)
                pitchf = np.concatenate([pitchf, np.repeat(pitchf[:, -1:], n - m, axis=1)], axis=1)
            elif m > n:
                pitch = pitch[:, :n]
                pitchf = pitchf[:, :n]
        out = self.glue.prepare(feats[0], index_rate if use_index else 0.0,
                                pitchf[0] if protect_on else None, protect)
        if times is not None:
            times[0] += ttime() - t0
        return {"feats": out[None], "pitch": pitch, "pitchf": pitchf, "sid_arr": np.asarray([sid], dtype=np.int64)}

    def vc(self, model, net_g, sid, audio0, pitch, pitchf, times, index, index_vectors, index_rate, version, protect,
           feats=None, retrieval_mode="ivf", brute_mix=0.0):
        """``runtime/pipeline.py:616-695``: prepare, then ``net_g.infer``;
        returns the flat waveform (t_pad not trimmed, as in the reference)."""
        prep = self._vc_prepare(model, sid, audio0, pitch, pitchf, times, index, index_vectors, index_rate, version,
                                protect, feats=feats, retrieval_mode=retrieval_mode, brute_mix=brute_mix)
        if prep["pitch"] is None or prep["pitchf"] is None:
            raise NotImplementedError("only f0-conditioned models (if_f0=True) are supported, as in the reference")
        audio1 = net_g.infer(prep["feats"], prep["pitch"], prep["pitchf"], prep["sid_arr"])
        return np.asarray(audio1, dtype=np.float32).reshape(-1)

    def change_rms(self, data1, data2, sr1, sr2, rate):
        return self.glue.change_rms(data1, data2, sr1, sr2, rate)

    def to_int16(self, audio):
        """``runtime/pipeline.py:1208-1213``."""
        return self.glue.to_int16(audio)
