# -*- coding: utf-8 -*-
"""float64 brute-force loop references for tiny inputs.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

These restate each op from its definition with explicit index loops, in the
style of the reference engine self-test's float64 references
(``engine/test_ffi.py:129-214``), so the numpy oracle (``oracle/nn_ref.py``,
``oracle/vits_ref.py``) is checked against something that shares none of its
vectorisation tricks (zero-stuffed dilated kernels, sliding windows, the
rel<->abs pad/reshape remaps).
"""

from __future__ import annotations

import math

import numpy as np


def conv1d(x, w, b=None, stride=1, pad_l=0, pad_r=0, dilation=1):
    """out[b,o,t] = bias[o] + sum_{c,k} w[o,c,k] * x[b,c,t*s - pad_l + k*d]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, C, T = x.shape
    O, _, K = w.shape
    n_out = (T + pad_l + pad_r - dilation * (K - 1) - 1) // stride + 1
    out = np.zeros((B, O, max(n_out, 0)))
    for bi in range(B):
        for o in range(O):
            for t in range(max(n_out, 0)):
                acc = 0.0 if b is None else float(b[o])
                for c in range(C):
                    for k in range(K):
                        i = t * stride - pad_l + k * dilation
                        if 0 <= i < T:
                            acc += w[o, c, k] * x[bi, c, i]
                out[bi, o, t] = acc
    return out


def conv_transpose1d(x, w, b=None, stride=1, padding=0, output_padding=0, dilation=1):
    """Scatter definition: out[b,o,t*s - p + k*d] += x[b,c,t] * w[c,o,k]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    B, C, T = x.shape
    _, O, K = w.shape
    n_out = (T - 1) * stride - 2 * padding + dilation * (K - 1) + output_padding + 1
    out = np.zeros((B, O, n_out))
    for bi in range(B):
        for c in range(C):
            for t in range(T):
                for k in range(K):
                    pos = t * stride - padding + k * dilation
                    if 0 <= pos < n_out:
                        out[bi, :, pos] += x[bi, c, t] * w[c, :, k]
    if b is not None:
        out += np.asarray(b, np.float64).reshape(1, -1, 1)
    return out


def layer_norm(x, gamma, beta, eps=1e-5):
    x = np.asarray(x, np.float64)
    out = np.empty_like(x)
    flat = x.reshape(-1, x.shape[-1])
    of = out.reshape(-1, x.shape[-1])
    for r in range(flat.shape[0]):
        row = flat[r]
        n = row.size
        mean = sum(row) / n
        var = sum((v - mean) ** 2 for v in row) / n
        for c in range(n):
            of[r, c] = (row[c] - mean) / math.sqrt(var + eps) * gamma[c] + beta[c]
    return out


def softmax(x):
    x = np.asarray(x, np.float64)
    out = np.empty_like(x)
    flat = x.reshape(-1, x.shape[-1])
    of = out.reshape(-1, x.shape[-1])
    for r in range(flat.shape[0]):
        m = max(flat[r])
        e = [math.exp(v - m) for v in flat[r]]
        s = sum(e)
        of[r] = [v / s for v in e]
    return out


def relpos_attention(q, k, v, emb_k, emb_v, window=10):
    """Windowed relative-position attention for one head, by definition.

    q, k, v: [P, D]; emb_k / emb_v: [2*window+1, D].
    score[t,s] = (q_t/sqrt(D)) . k_s + [|s-t|<=w] (q_t/sqrt(D)) . emb_k[s-t+w]
    out[t]     = sum_s p[t,s] v_s + sum_{|s-t|<=w} p[t,s] emb_v[s-t+w]
    (the banded form of ``runtime/models/vits.py:998-1014``, as stated in
    ``engine/shaders/banded_attn_qk.comp:1-11``).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    P, D = q.shape
    out = np.zeros((P, D))
    for t in range(P):
        qs = q[t] / math.sqrt(D)
        sc = np.zeros(P)
        for s in range(P):
            val = float(np.dot(qs, k[s]))
            r = s - t
            if -window <= r <= window:
                val += float(np.dot(qs, emb_k[r + window]))
            sc[s] = val
        m = sc.max()
        e = np.exp(sc - m)
        p = e / e.sum()
        for s in range(P):
            out[t] += p[s] * v[s]
            r = s - t
            if -window <= r <= window:
                out[t] += p[s] * emb_v[r + window]
    return out


def sine_source(f0, ns, w_lin, b_lin, sr, upp):
    """NSF source by its definition, float64: phase of sample u (1-based) in
    frame p = frac(sum_{q<p} f0[q]*upp/sr) + f0[p]*u/sr, har =
    tanh(w*(0.1*sin(2*pi*phase)*uv + amp*ns) + b)."""
    f0 = np.asarray(f0, np.float64).reshape(-1)
    ns = np.asarray(ns, np.float64).reshape(-1)
    P = f0.size
    out = np.zeros(P * upp)
    acc = 0.0
    for p in range(P):
        uv = 1.0 if f0[p] > 0 else 0.0
        amp = uv * 0.003 + (1 - uv) * 0.1 / 3
        for u in range(upp):
            ph = acc + f0[p] / sr * (u + 1)
            s = 0.1 * math.sin(2 * math.pi * ph) * uv + amp * ns[p * upp + u]
            out[p * upp + u] = math.tanh(w_lin * s + b_lin)
        step = f0[p] / sr * upp
        acc = math.fmod(acc + (math.fmod(step + 0.5, 1.0) - 0.5), 1.0)
    return out
