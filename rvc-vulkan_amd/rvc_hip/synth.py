# -*- coding: utf-8 -*-
"""Device-resident RVC synthesizer on the HIP backend.

``HipSynthesizer`` has the inference surface of the reference's
``SynthesizerTrn`` (``runtime/models/vits.py:2237-2595``) -- ``infer`` (full
and partial synthesis), ``infer_controlled``, ``prep_dec``,
``decode_batch(preps)`` -- and its ``dec`` attribute that of
``_GeneratorNSF`` (``forward(z, f0, g, ns, seg_offsets)``,
``decode_batch(z_list, g, f0_list, ns_list, off_list)``, ``:1847-2231``).
Construction uploads every weight once into a ``rvc_synth`` session (the
analogue of ``register_persistent_weights``, ``:2272-2334``); each call then
runs enc_p + flow + GeneratorNSF as one stream of HIP kernels with a single
upload of the inputs and a single download of the waveform.

Batching: ``phone`` / ``z`` may carry a leading batch of B independent
chunks of equal length; they run as one batched launch sequence.  Chunks of
unequal length (``decode_batch``) run as one batch per length, queued on one
stream in a single call.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _hip
from .config import VitsConfig
from .hip_ops import HipContext, get_context

__all__ = ["HipSynthesizer", "HipDeferred"]

_F32P = ctypes.POINTER(ctypes.c_float)
_I64P = ctypes.POINTER(ctypes.c_int64)

# RVC_FIXED_SEED=<int>: ``infer`` / ``prep_dec`` calls without a seed use it
# (read at import, as runtime/models/vits.py:56 does)
_FIXED_SEED = os.environ.get("RVC_FIXED_SEED", "").strip()
# partial-synthesis context frames (runtime/models/vits.py:141-152)
_DEC_PAD = 16
_FLOW_PAD = 24

READABLE = ("enc_in", "enc_out", "stats", "z_p", "z", "g", "har", "dec_pre")


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _i64(a):
    a = np.asarray(a)
    if not np.issubdtype(a.dtype, np.integer):
        raise TypeError(f"expected an integer array, got dtype={a.dtype}")
    return np.ascontiguousarray(a, dtype=np.int64)


class HipGenerator:
    """The ``_GeneratorNSF`` call surface of a ``HipSynthesizer``
    (``runtime/models/vits.py:1847-2231``)."""

    def __init__(self, synth: "HipSynthesizer"):
        self._s = synth

    def forward(self, z, f0, g, ns, seg_offsets=None):
        """z [1,hidden,P], f0 [1,P], g [1,gin,1] or None, ns [1,P*upp,1],
        seg_offsets [1,P,1] or None -> [1,1,P*upp] (``:2133-2231``)."""
        return self._s.decode_chunks([z], g, [f0], [ns], [seg_offsets])[0]

    def decode_batch(self, z_list, g, f0_list, ns_list, off_list=None):
        """Chunks of any lengths, one speaker g (``:1847-1878``); each result
        equals ``forward`` of that chunk bit for bit."""
        return self._s.decode_chunks(z_list, g, f0_list, ns_list, off_list)


class HipDeferred:
    """The holder ``infer(..., _defer=True)`` returns (the reference's
    ``_DecCollector``, ``runtime/models/vits.py:1314-1360``): the synthesis
    is queued on the GPU; ``collect()`` waits for it and returns the waveform,
    ``abort()`` waits and drops it.  Either ends the holder; a second call
    raises ``RuntimeError``.  A holder dropped without either is aborted.
    It keeps the resident phone buffer alive until the call is ended."""

    __slots__ = ("_s", "_ticket", "_shape", "_keep", "_done")

    def __init__(self, synth, ticket, shape, keep):
        self._s = synth
        self._ticket = ticket
        self._shape = shape
        self._keep = keep
        self._done = False

    def collect(self):
        if self._done:
            raise RuntimeError("HipDeferred: already collected or aborted")
        self._done = True
        wave = np.empty(self._shape, dtype=np.float32)
        try:
            _hip._check(self._s._lib.rvc_synth_collect(self._s.handle, self._ticket, wave.ctypes.data_as(_F32P)),
                        "rvc_synth_collect")
        finally:
            self._keep = None
        return wave

    def abort(self):
        if self._done:
            return
        self._done = True
        try:
            self._s._lib.rvc_synth_abort(self._s.handle, self._ticket)
        finally:
            self._keep = None

    def __del__(self):
        try:
            import sys

            if not sys.is_finalizing() and not self._done and self._s.handle:
                self.abort()
        except Exception:  # noqa: BLE001
            pass


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
        self.dec = HipGenerator(self)

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
        (``runtime/models/vits.py:2337-2350``); ``seed=None`` takes
        RVC_FIXED_SEED when it is set, else fresh entropy."""
        if seed is None and _FIXED_SEED:
            seed = int(_FIXED_SEED)
        rng = np.random.RandomState(seed) if seed is not None else np.random.RandomState()
        nz = rng.standard_normal((1, self.cfg.hidden, P)).astype(np.float32)
        ns = rng.standard_normal((1, P * self.cfg.upp, 1)).astype(np.float32)
        return nz, ns

    def infer(self, phone, pitch, nsff0, sid, seed=None, skip_head=None, return_length=None, phone_gpu=None,
              _defer: bool = False):
        """``SynthesizerTrn.infer`` (``:2352-2402``): full synthesis, or with
        ``skip_head`` / ``return_length`` the waveform of frames
        [skip_head, skip_head + return_length) from the partial path.
        ``phone_gpu`` / ``_defer`` as in ``infer_controlled``; the partial
        path ignores ``_defer`` and returns the waveform, as the reference's
        does."""
        P = np.asarray(phone).shape[1]
        nz, ns = self.make_noise(P, seed)
        if skip_head is None or return_length is None:
            return self.infer_controlled(phone, pitch, nsff0, sid, nz, ns, phone_gpu=phone_gpu, _defer=_defer)
        head, length = self._check_part(P, skip_head, return_length)
        p = self._partial_prep(phone, pitch, nsff0, sid, nz, ns, head, length)
        o = self.dec.forward(p["z_seg"], p["nsff0_seg"], p["g"], p["ns_seg"], seg_offsets=p["off"])
        return o[:, :, p["s0"]:p["s0"] + p["n_out"]]

    def infer_controlled(self, phone, pitch, nsff0, sid, nz, ns, phone_gpu=None, _defer: bool = False):
        """phone [B,P,D], pitch int [B,P], nsff0 [B,P], sid int [1] or [B],
        nz [B,hidden,P], ns [B,P*upp(,1)] -> wave [B,1,P*upp].

        ``phone_gpu``: a resident ``hip_ops.PersistentBuffer`` of this
        session's context holding ``phone`` ([1,P,D] or [P,D] floats); the
        encoder reads it instead of uploading ``phone`` (the reference's
        ``phone_gpu``, ``runtime/models/vits.py:2352-2402``).  A freed
        buffer, one of another context or one too small is ignored and
        ``phone`` is uploaded.  ``_defer=True`` queues the synthesis and
        returns a holder whose ``collect()`` waits and returns the waveform
        (``abort()`` drops it), so the host can prepare the next chunk while
        the GPU runs this one (``:2551-2595``, ``runtime/pipeline.py:
        1010-1080``); up to 8 calls may be outstanding."""
        phone, pitch, nsff0, sid, nz = self._enc_inputs(phone, pitch, nsff0, sid, nz)
        B, P, _ = phone.shape
        ns = _f32(ns).reshape(B, P * self.cfg.upp)
        buf = 0
        if phone_gpu is not None and getattr(phone_gpu, "valid", False) and getattr(phone_gpu, "_ctx", None) is \
                self.ctx and int(getattr(phone_gpu, "nbytes", 0)) >= phone.nbytes:
            buf = int(phone_gpu.id)
        if not _defer and not buf:
            wave = np.empty((B, 1, P * self.cfg.upp), dtype=np.float32)
            _hip._check(self._lib.rvc_synth_infer(
                self.handle, phone.ctypes.data_as(_F32P), pitch.ctypes.data_as(_I64P),
                nsff0.ctypes.data_as(_F32P), sid.ctypes.data_as(_I64P), nz.ctypes.data_as(_F32P),
                ns.ctypes.data_as(_F32P), B, P, wave.ctypes.data_as(_F32P)), "rvc_synth_infer")
            return wave
        ticket = int(self._lib.rvc_synth_submit(
            self.handle, None if buf else phone.ctypes.data_as(_F32P), buf, pitch.ctypes.data_as(_I64P),
            nsff0.ctypes.data_as(_F32P), sid.ctypes.data_as(_I64P), nz.ctypes.data_as(_F32P),
            ns.ctypes.data_as(_F32P), B, P))
        if ticket < 0:
            raise RuntimeError(f"rvc_synth_submit failed: {_hip.last_error()}")
        holder = HipDeferred(self, ticket, (B, 1, P * self.cfg.upp), phone_gpu if buf else None)
        return holder if _defer else holder.collect()

    def _enc_inputs(self, phone, pitch, nsff0, sid, nz):
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
        return phone, pitch, nsff0, sid, nz

    def _enc_flow(self, phone, pitch, nsff0, sid, nz, flow_head=0, want_phase=False):
        """enc_p over all P frames and the flow over [flow_head, P) on the GPU
        -> (z [B,hidden,P-flow_head], g [B,gin], phase offsets [B,P] or None)."""
        phone, pitch, nsff0, sid, nz = self._enc_inputs(phone, pitch, nsff0, sid, nz)
        B, P, _ = phone.shape
        z = np.empty((B, self.cfg.hidden, P - flow_head), dtype=np.float32)
        g = np.empty((B, self.cfg.gin_channels), dtype=np.float32)
        ph = np.empty((B, P), dtype=np.float32) if want_phase else None
        _hip._check(self._lib.rvc_synth_prep(
            self.handle, phone.ctypes.data_as(_F32P), pitch.ctypes.data_as(_I64P), nsff0.ctypes.data_as(_F32P),
            sid.ctypes.data_as(_I64P), nz.ctypes.data_as(_F32P), B, P, int(flow_head), z.ctypes.data_as(_F32P),
            g.ctypes.data_as(_F32P), ph.ctypes.data_as(_F32P) if ph is not None else None), "rvc_synth_prep")
        return z, g, ph

    def phase_offsets(self, nsff0):
        """``_phase_offsets`` (``:2404-2414``) computed on the GPU: the full
        run's per-frame fmod-cumsum phase of nsff0 [B,P] -> [B,P,1]."""
        nsff0 = _f32(nsff0)
        nsff0 = nsff0.reshape(nsff0.shape[0] if nsff0.ndim > 1 else 1, -1)
        B, P = nsff0.shape
        out = np.empty((B, P), dtype=np.float32)
        _hip._check(self._lib.rvc_synth_phase_offsets(self.handle, nsff0.ctypes.data_as(_F32P), B, P,
                                                      out.ctypes.data_as(_F32P)), "rvc_synth_phase_offsets")
        return out.reshape(B, P, 1)

    @staticmethod
    def _check_part(P, skip_head, return_length):
        head, length = int(skip_head), int(return_length)
        if head < 0 or head >= P or length <= 0 or head + length > P:
            raise ValueError(f"skip_head/return_length out of range: P={P}, head={head}, length={length}")
        return head, length

    def _full_prep(self, phone, pitch, nsff0, sid, nz, ns):
        z, g, _ = self._enc_flow(phone, pitch, nsff0, sid, nz)
        P = z.shape[-1]
        return {"z_seg": z, "nsff0_seg": _f32(nsff0).reshape(1, P), "ns_seg": _f32(ns).reshape(1, -1, 1),
                "off": None, "g": g.reshape(1, -1, 1), "s0": 0, "n_out": P * self.cfg.upp}

    def _partial_prep(self, phone, pitch, nsff0, sid, nz, ns, head, length):
        """``_partial_prep`` (``:2416-2476``): enc_p over every frame, the
        flow from max(head - 40, 0), the decoder segment head -/+ 16 frames
        clipped to [0, P), and the segment's phase offsets taken from the
        full run's cumulative phase."""
        upp = self.cfg.upp
        P = np.asarray(phone).shape[1]
        flow_head = max(head - _FLOW_PAD - _DEC_PAD, 0)
        z, g, rad_acc = self._enc_flow(phone, pitch, nsff0, sid, nz, flow_head=flow_head, want_phase=True)
        zs = max(head - _DEC_PAD, 0)
        ze = min(P, head + length + _DEC_PAD)
        n_seg = ze - zs
        rad_acc = rad_acc.reshape(1, P, 1)
        if zs == 0:
            off = np.zeros((1, n_seg, 1), dtype=np.float32)
            if n_seg > 1:
                off[:, 1:, :] = rad_acc[:, :n_seg - 1, :]
        else:
            off = np.ascontiguousarray(rad_acc[:, zs - 1:zs - 1 + n_seg, :])
        return {"z_seg": np.ascontiguousarray(z[:, :, zs - flow_head:ze - flow_head]),
                "nsff0_seg": _f32(nsff0).reshape(1, P)[:, zs:ze].copy(),
                "ns_seg": _f32(ns).reshape(1, -1, 1)[:, zs * upp:ze * upp, :].copy(),
                "off": off, "g": g.reshape(1, -1, 1), "s0": (head - zs) * upp, "n_out": length * upp}

    def prep_dec(self, phone, pitch, nsff0, sid, seed=None, skip_head=None, return_length=None):
        """``SynthesizerTrn.prep_dec`` (``:2478-2500``): enc_p + flow (+ phase
        offsets for a partial segment) on the GPU, no decoder; the dict
        ``decode_batch`` takes."""
        P = np.asarray(phone).shape[1]
        nz, ns = self.make_noise(P, seed)
        if skip_head is None or return_length is None:
            return self._full_prep(phone, pitch, nsff0, sid, nz, ns)
        head, length = self._check_part(P, skip_head, return_length)
        return self._partial_prep(phone, pitch, nsff0, sid, nz, ns, head, length)

    def decode_batch(self, preps):
        """``SynthesizerTrn.decode_batch`` (``:2502-2522``): the decoders of
        several ``prep_dec`` chunks (lengths may differ) in one call, the
        first chunk's speaker for all; returns each chunk's target segment."""
        if not preps:
            return []
        outs = self.dec.decode_batch([p["z_seg"] for p in preps], preps[0]["g"],
                                     [p["nsff0_seg"] for p in preps], [p["ns_seg"] for p in preps],
                                     [p["off"] for p in preps])
        return [o[:, :, p["s0"]:p["s0"] + p["n_out"]] for o, p in zip(outs, preps)]

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

    def decode_chunks(self, z_list, g, f0_list, ns_list, off_list=None):
        """Decoder over chunks of any lengths in one call (``rvc_synth_decode_chunks``):
        z [1,hidden,P_i] (or [hidden,P_i]), f0 [1,P_i], ns [1,P_i*upp(,1)],
        off [1,P_i(,1)] or None, one speaker g [1,gin(,1)] or None -> list of
        [1,1,P_i*upp]."""
        n = len(z_list)
        if n == 0:
            return []
        off_list = list(off_list) if off_list is not None else [None] * n
        if not (len(f0_list) == len(ns_list) == len(off_list) == n):
            raise ValueError("z_list, f0_list, ns_list and off_list must have one entry per chunk")
        H, upp = self.cfg.hidden, self.cfg.upp
        zs, fs, nss, offs, Ps = [], [], [], [], []
        for z, f, nsv, o in zip(z_list, f0_list, ns_list, off_list):
            z = _f32(z)
            if z.ndim == 3 and z.shape[0] != 1:
                raise ValueError(f"each chunk's z must be [1,{H},P], got {z.shape}")
            z = z.reshape(H, -1) if z.size % H == 0 else None
            if z is None:
                raise ValueError(f"z must hold {H} channels")
            P = z.shape[1]
            zs.append(z)
            fs.append(_f32(f).reshape(P))
            nss.append(_f32(nsv).reshape(P * upp))
            offs.append(None if o is None else _f32(o).reshape(P))
            Ps.append(P)
        waves = [np.empty((1, 1, P * upp), dtype=np.float32) for P in Ps]
        arr = ctypes.POINTER(ctypes.c_float) * n
        zp = arr(*[a.ctypes.data_as(_F32P) for a in zs])
        fp = arr(*[a.ctypes.data_as(_F32P) for a in fs])
        np_ = arr(*[a.ctypes.data_as(_F32P) for a in nss])
        op = arr(*[a.ctypes.data_as(_F32P) if a is not None else _F32P() for a in offs])
        wp = arr(*[a.ctypes.data_as(_F32P) for a in waves])
        Pa = np.asarray(Ps, dtype=np.int64)
        gv = None
        if g is not None:
            gv = _f32(g).reshape(-1)
            if gv.size != self.cfg.gin_channels:
                raise ValueError(f"g must hold one speaker embedding of {self.cfg.gin_channels} values")
        _hip._check(self._lib.rvc_synth_decode_chunks(
            self.handle, n, zp, fp, np_, op, Pa.ctypes.data_as(_I64P),
            gv.ctypes.data_as(_F32P) if gv is not None else None, wp), "rvc_synth_decode_chunks")
        return waves

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
