# -*- coding: utf-8 -*-
"""numpy restatement of the conversion glue around synthesis.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``runtime/retrieval.py`` (``search_l2``) and ``runtime/pipeline.py``
(``_vc_prepare``'s feature path with a ``FeatureIndex``, ``change_rms`` and
its helpers, the int16 peak normalisation) and ``runtime/nn.py``
(``interpolate_linear``), in float32 with the same expression order, under
numpy 2 promotion rules (python scalars are weak: a float32 array times a
python float stays float32).

Pinning: ``search_l2`` against a float64 brute-force ranking;
``interpolate_linear`` and ``interp_linear_size`` against
``torch.nn.functional.interpolate(mode="linear", align_corners=False)``;
``rms_curve`` against a float64 frame loop; ``vc_prepare``, ``change_rms``
and ``to_int16`` end to end against golden vectors written by the
reference's own code (``tests/golden/make_golden_pipeline.py``;
``tests/test_oracle_pipeline.py``).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "K_SEARCH",
    "search_l2",
    "feature_blend",
    "interpolate_linear",
    "align_pitch",
    "vc_prepare",
    "rms_curve",
    "interp_linear_size",
    "change_rms",
    "to_int16",
]

K_SEARCH = 8  # runtime/pipeline.py:55


def search_l2(query, db, k=K_SEARCH):
    """Brute-force L2 neighbours (``runtime/retrieval.py:35-83``):
    ``dist = (q2 + d2) - 2 q.d``, clamped at 0, the ``min(k, N)`` smallest per
    row in ascending order.  The reference's chunked argpartition leaves the
    order of exactly equal distances unspecified; here the lower row comes
    first (a stable sort)."""
    query = np.asarray(query, dtype=np.float32)
    db = np.asarray(db, dtype=np.float32)
    F = query.shape[0]
    N = db.shape[0]
    k = min(k, N)
    q2 = np.einsum("fd,fd->f", query, query)
    d2 = np.einsum("nd,nd->n", db, db)
    dist = q2[:, None] + d2[None, :] - 2.0 * (query @ db.T)
    np.maximum(dist, 0.0, out=dist)
    order = np.argsort(dist, axis=1, kind="stable")[:, :k]
    scores = np.take_along_axis(dist, order, axis=1).astype(np.float32)
    return scores, order.astype(np.int64)[:, :k].reshape(F, k)


def feature_blend(feats, vectors, scores, inds, index_rate):
    """``runtime/pipeline.py:546-566`` (FeatureIndex branch, ``brute_mix`` 0):
    ``w = (1/score)^2``, rows normalised by ``max(sum, 1e-12)``, the weighted
    sum of the neighbours, mixed in at ``index_rate``.  feats ``[L, D]``."""
    feats = np.asarray(feats, dtype=np.float32)
    blk = np.asarray(vectors, dtype=np.float32)[inds]
    w = np.square(1.0 / scores)
    w /= np.maximum(w.sum(axis=1, keepdims=True), 1e-12)
    brute_blend = np.sum(blk * w[:, :, None], axis=1)
    ivf_blend = brute_blend
    blend = (1.0 - 0.0) * ivf_blend + 0.0 * brute_blend
    return blend * index_rate + feats * (1 - index_rate)


def interpolate_linear(x, scale_factor=2):
    """``runtime/nn.py:734-758`` along the last axis (align_corners=False)."""
    x = np.asarray(x)
    L_in = x.shape[-1]
    L_out = int(L_in * scale_factor)
    if L_out == L_in:
        return x.copy()
    src = (np.arange(L_out, dtype=np.float64) + 0.5) / float(scale_factor) - 0.5
    src = np.clip(src, 0.0, L_in - 1)
    lo = np.floor(src).astype(np.int64)
    hi = np.minimum(lo + 1, L_in - 1)
    frac = (src - lo).astype(x.dtype) if x.dtype != np.float64 else src - lo
    return x[..., lo] * (1.0 - frac) + x[..., hi] * frac


def align_pitch(pitch, pitchf, n):
    """Pad with the last frame or truncate to ``n`` frames
    (``runtime/pipeline.py:581-593``)."""
    m = pitch.shape[1]
    if m < n:
        pitch = np.concatenate([pitch, np.repeat(pitch[:, -1:], n - m, axis=1)], axis=1)
        pitchf = np.concatenate([pitchf, np.repeat(pitchf[:, -1:], n - m, axis=1)], axis=1)
    elif m > n:
        pitch = pitch[:, :n]
        pitchf = pitchf[:, :n]
    return pitch, pitchf


def vc_prepare(feats, pitch, pitchf, vectors=None, index_rate=0.0, protect=0.5):
    """``Pipeline._vc_prepare`` feature path (``runtime/pipeline.py:488-614``)
    with a ``FeatureIndex`` of ``vectors`` (or none), feats given: retrieval
    blend on ``[L, D]``, 2x interpolation, pitch alignment to the interpolated
    length, protect mask.  feats ``[1, L, D]``, pitch int64 / pitchf float32
    ``[1, P]``.  Returns ``(feats [1, 2L, D], pitch, pitchf)``."""
    feats = np.asarray(feats, dtype=np.float32)
    if protect < 0.5 and pitch is not None and pitchf is not None:
        feats0 = feats.copy()
    if vectors is not None and index_rate != 0 and len(vectors) > 0:
        npy = np.asarray(feats[0], dtype=np.float32)
        sc, ix = search_l2(npy, vectors, k=K_SEARCH)
        feats = feature_blend(npy, vectors, sc, ix, index_rate)[None, :, :]
    feats = interpolate_linear(feats.transpose(0, 2, 1), scale_factor=2).transpose(0, 2, 1)
    if protect < 0.5 and pitch is not None and pitchf is not None:
        feats0 = interpolate_linear(feats0.transpose(0, 2, 1), scale_factor=2).transpose(0, 2, 1)
    if pitch is not None and pitchf is not None:
        pitch, pitchf = align_pitch(pitch, pitchf, feats.shape[1])
    if protect < 0.5 and pitch is not None and pitchf is not None:
        pitchff = pitchf.copy()
        pitchff[pitchf > 0] = 1
        pitchff[pitchf < 1] = protect
        pitchff = pitchff[:, :, None]
        feats = feats * pitchff + feats0 * (1 - pitchff)
    return feats, pitch, pitchf


def rms_curve(x, sr):
    """``runtime/pipeline.py:191-206``: librosa ``feature.rms`` with
    frame ``sr//2*2``, hop ``sr//2``, centred zero padding; ``[1, frames]``."""
    frame_length = sr // 2 * 2
    hop = sr // 2
    pad = frame_length // 2
    xp = np.pad(x, (pad, pad), mode="constant")
    frames = np.lib.stride_tricks.sliding_window_view(xp, frame_length, axis=-1)[::hop, ...]
    rms = np.sqrt(np.mean(frames.astype(np.float32) ** 2, axis=-1))
    return rms[None, :].astype(np.float32)


def interp_linear_size(x, n_out):
    """``runtime/pipeline.py:209-232``: float64 linear interpolation onto
    exactly ``n_out`` points (align_corners=False), returned as float32."""
    x = np.asarray(x, dtype=np.float64)
    L_in = x.shape[-1]
    if n_out <= 0 or L_in == n_out:
        return np.asarray(x, dtype=np.float32)
    src = (np.arange(n_out, dtype=np.float64) + 0.5) * (L_in / n_out) - 0.5
    src = np.clip(src, 0.0, L_in - 1)
    lo = np.floor(src).astype(np.int64)
    hi = np.minimum(lo + 1, L_in - 1)
    frac = src - lo
    return (x[..., lo] * (1.0 - frac) + x[..., hi] * frac).astype(np.float32)


def change_rms(data1, data2, sr1, sr2, rate):
    """``runtime/pipeline.py:164-188``."""
    n_out = np.asarray(data2).shape[0]
    if n_out == 0:
        return np.asarray(data2, dtype=np.float32).copy()
    r1 = rms_curve(np.asarray(data1, dtype=np.float32), int(sr1))
    r2 = rms_curve(np.asarray(data2, dtype=np.float32), int(sr2))
    r1 = interp_linear_size(r1, n_out)
    r2 = interp_linear_size(r2, n_out)
    r2 = np.maximum(r2, np.float32(1e-6))
    ratio = np.power(r1, 1.0 - rate) * np.power(r2, rate - 1.0)
    return np.asarray(data2, dtype=np.float32) * ratio.reshape(-1)


def to_int16(audio):
    """``runtime/pipeline.py:1208-1213``: peak normalisation to int16."""
    audio = np.asarray(audio, dtype=np.float32)
    audio_max = np.abs(audio).max() / 0.99
    max_int16 = 32768.0
    if audio_max > 1:
        max_int16 /= audio_max
    return (audio * max_int16).astype(np.int16)
