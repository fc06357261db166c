# -*- coding: utf-8 -*-
"""numpy restatement of the reference op library (float32 semantics).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function follows the float32 branch the reference takes when the
backend is ``numpy``: ``runtime/nn.py`` routes float32 conv/LN/softmax/
linear through ``runtime/backend.py``, whose numpy branches are restated here
with the same evaluation order (bias added after the conv core, convT bias
inside, two-pass LayerNorm, max-subtracted softmax).
"""

from __future__ import annotations

import contextlib

import numpy as np

__all__ = [
    "conv1d",
    "conv_transpose1d",
    "layer_norm",
    "softmax",
    "leaky_relu",
    "relu",
    "sigmoid",
    "tanh",
    "linear",
    "embedding",
    "conv_formulation",
]

# How the conv1d core is evaluated.  "einsum" (default) is the reference's own
# formulation: a sliding-window view contracted against the zero-stuffed
# dilated kernel (``runtime/nn.py:89-135``); it is what the CPU baseline
# times.  "taps" sums one contiguous GEMM per tap, W[:, :, k] @ x[:, k*d :: s]:
# the same mathematics in another float32 summation order, about 50x faster on
# the decoder's shapes, for the parity tests at the full BASELINE sizes.  Both
# are pinned against the float64 loops and against each other.
_CONV_MODE = "einsum"


@contextlib.contextmanager
def conv_formulation(mode: str):
    """Evaluate conv1d cores with ``mode`` ("einsum" or "taps") inside the block."""
    global _CONV_MODE
    if mode not in ("einsum", "taps"):
        raise ValueError(f"unknown conv formulation {mode!r}")
    prev, _CONV_MODE = _CONV_MODE, mode
    try:
        yield
    finally:
        _CONV_MODE = prev


def _pads(padding):
    if isinstance(padding, (tuple, list)):
        return int(padding[0]), int(padding[1])
    return int(padding), int(padding)


def _conv1d_core(x, w, stride, pad_l, pad_r, dilation):
    """Conv core without bias: zero pad, zero-stuffed dilated kernel, a
    sliding-window view and one einsum contraction
    (``runtime/nn.py:89-135``)."""
    B, C, T = x.shape
    O, _, K = w.shape
    k_span = (K - 1) * dilation + 1
    n_out = (T + pad_l + pad_r - k_span) // stride + 1
    if n_out <= 0:
        return np.zeros((B, O, 0), dtype=x.dtype)
    if dilation > 1:
        w_span = np.zeros((O, C, k_span), dtype=w.dtype)
        w_span[:, :, ::dilation] = w
    else:
        w_span = w
    xp = np.pad(x, ((0, 0), (0, 0), (pad_l, pad_r)))
    if k_span > xp.shape[-1]:
        return np.zeros((B, O, n_out), dtype=x.dtype)
    if _CONV_MODE == "taps":
        return _conv1d_taps(xp, w, stride, dilation, n_out)
    win = np.lib.stride_tricks.sliding_window_view(xp, k_span, axis=-1)[:, :, ::stride, :]
    return np.einsum("bctk,ock->bot", win, w_span, optimize=True)


def _conv1d_taps(xp, w, stride, dilation, n_out):
    """Padded input ``xp`` [B,C,T'] -> sum over taps of contiguous GEMMs
    W[:, :, k] @ xp[b, :, k*d : k*d + (n_out-1)*s + 1 : s] (the "taps"
    formulation of ``conv_formulation``)."""
    B = xp.shape[0]
    O, _, K = w.shape
    out = np.zeros((B, O, n_out), dtype=np.result_type(xp.dtype, w.dtype))
    wk = [np.ascontiguousarray(w[:, :, k]) for k in range(K)]
    span = (n_out - 1) * stride + 1
    for b in range(B):
        for k in range(K):
            s0 = k * dilation
            out[b] += wk[k] @ np.ascontiguousarray(xp[b, :, s0:s0 + span:stride])
    return out


def conv1d(x, w, b=None, stride=1, padding=0, dilation=1):
    """``nn.conv1d`` float32 path: ``backend.conv1d(x, w, None, ...)`` then
    ``core + b`` (``runtime/nn.py:138-176``, ``runtime/backend.py:233-239``)."""
    x = np.asarray(x)
    w = np.asarray(w)
    pad_l, pad_r = _pads(padding)
    core = _conv1d_core(x, w, int(stride), pad_l, pad_r, int(dilation))
    if b is not None:
        core = core + np.asarray(b, dtype=core.dtype).reshape(1, -1, 1)
    return core


def conv_transpose1d(x, w, b=None, stride=1, padding=0, output_padding=0, dilation=1):
    """PyTorch ConvTranspose1d by per-tap matmul + strided scatter-add, bias
    added after all taps (``runtime/nn.py:293-346``; the matmul branch is the
    default, ``RVC_TRAIN_FWD_MATMUL`` unset)."""
    x = np.asarray(x)
    w = np.asarray(w)
    stride, padding = int(stride), int(padding)
    output_padding, dilation = int(output_padding), int(dilation)
    B, C_in, T = x.shape
    C_out, K = w.shape[1], w.shape[2]
    n_out = (T - 1) * stride - 2 * padding + dilation * (K - 1) + output_padding + 1
    if n_out <= 0:
        return np.zeros((B, C_out, 0), dtype=x.dtype)
    out = np.zeros((B, C_out, n_out), dtype=np.result_type(x.dtype, w.dtype))
    t = np.arange(T)
    for k in range(K):
        pos = t * stride - padding + k * dilation
        ok = np.nonzero((pos >= 0) & (pos < n_out))[0]
        if ok.size == 0:
            continue
        if _CONV_MODE == "taps":
            # the same per-tap product as one contiguous GEMM per batch item
            wkT = np.ascontiguousarray(w[:, :, k].T)
            lo, hi = int(ok[0]), int(ok[-1]) + 1  # ok is a contiguous run of t
            for bi in range(B):
                out[bi][:, pos[lo]:pos[hi - 1] + 1:stride] += wkT @ np.ascontiguousarray(x[bi, :, lo:hi])
            continue
        part = np.matmul(x[:, :, ok].transpose(0, 2, 1), w[:, :, k]).transpose(0, 2, 1)
        out[:, :, pos[ok]] += part
    if b is not None:
        out += np.asarray(b, dtype=out.dtype).reshape(1, -1, 1)
    return out


def layer_norm(x, gamma, beta, eps=1e-5):
    """Two-pass biased-variance LayerNorm over the last axis
    (``runtime/backend.py:286-295``)."""
    x = np.asarray(x)
    mean = x.mean(axis=-1, keepdims=True)
    var = x.var(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(gamma) + np.asarray(beta)


def softmax(x, axis=-1):
    """``exp(x - max) / sum`` (``runtime/backend.py:298-306``)."""
    x = np.asarray(x)
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def leaky_relu(x, negative_slope=0.1):
    """``where(x >= 0, x, slope*x)`` (``runtime/nn.py:507-517``, numba absent)."""
    x = np.asarray(x)
    return np.where(x >= 0, x, negative_slope * x)


def relu(x):
    """``maximum(x, 0)`` (``runtime/backend.py:226-230``)."""
    return np.maximum(np.asarray(x), 0.0)


def sigmoid(x):
    """Both-branch stable sigmoid (``runtime/nn.py:520-523``)."""
    x = np.asarray(x)
    return np.where(x >= 0, 1.0 / (1.0 + np.exp(-x)), np.exp(x) / (1.0 + np.exp(x)))


def tanh(x):
    return np.tanh(np.asarray(x))


def linear(x, w, b=None):
    """``x @ w.T`` through the 2-D matmul, then ``+ b``
    (``runtime/nn.py:534-556``, ``runtime/backend.py:205-209``)."""
    x = np.asarray(x)
    w = np.asarray(w)
    D = x.shape[-1]
    out = (x.reshape(-1, D) @ w.T).reshape(x.shape[:-1] + (w.shape[0],))
    if b is not None:
        out = out + np.asarray(b).reshape(1, -1)
    return out


def embedding(ids, table):
    """Row gather with Python-style negative indices (``runtime/nn.py:559-571``)."""
    ids = np.asarray(ids)
    table = np.asarray(table)
    V = table.shape[0]
    ids2 = np.where(ids < 0, ids + V, ids).astype(np.int64)
    return np.take(table, ids2, axis=0)
