# -*- coding: utf-8 -*-
"""Pin the numpy oracle's ops against float64 loops, library routines and
mathematical identities (CPU only)."""

from __future__ import annotations

import numpy as np
import pytest
import scipy.signal

from conftest import rel_l2
from oracle import loops
from oracle import nn_ref as nn
from oracle import vits_ref as V

RNG = np.random.default_rng(1234)


def _r(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("mode", ["einsum", "taps"])
@pytest.mark.parametrize("B,C,O,T,K,s,pl,pr,d", [
    (1, 3, 4, 17, 3, 1, 1, 1, 1),
    (2, 2, 3, 20, 5, 1, 4, 4, 2),
    (1, 4, 2, 25, 7, 1, 9, 9, 3),
    (1, 1, 3, 40, 8, 4, 2, 2, 1),   # noise-conv shape: stride 4, k = 2*stride
    (1, 2, 2, 9, 3, 2, 0, 1, 1),    # asymmetric padding
    (1, 2, 2, 3, 5, 1, 0, 0, 1),    # kernel longer than input -> empty
])
def test_conv1d_matches_loops(B, C, O, T, K, s, pl, pr, d, mode):
    x, w, b = _r(B, C, T), _r(O, C, K), _r(O)
    with nn.conv_formulation(mode):
        got = nn.conv1d(x, w, b, stride=s, padding=(pl, pr), dilation=d)
    want = loops.conv1d(x, w, b, s, pl, pr, d)
    assert got.shape == want.shape
    if want.size:
        assert rel_l2(got, want) < 1e-6


def test_conv1d_matches_scipy_correlate():
    x, w = _r(1, 3, 64), _r(2, 3, 5)
    got = nn.conv1d(x, w, None, padding=2)
    want = np.stack([sum(scipy.signal.correlate(x[0, c].astype(np.float64), w[o, c].astype(np.float64),
                                                 mode="same") for c in range(3)) for o in range(2)])
    assert rel_l2(got[0], want) < 1e-6


@pytest.mark.parametrize("mode", ["einsum", "taps"])
@pytest.mark.parametrize("C,O,T,K,s,p,op,d", [
    (3, 2, 6, 16, 10, 3, 0, 1),   # dec.ups 0/1 geometry
    (4, 2, 9, 4, 2, 1, 0, 1),     # dec.ups 2/3 geometry
    (2, 3, 5, 24, 12, 6, 0, 1),   # 48k ups 0
    (2, 2, 7, 3, 2, 0, 1, 2),     # output_padding + dilation
])
def test_conv_transpose1d_matches_loops(C, O, T, K, s, p, op, d, mode):
    x, w, b = _r(2, C, T), _r(C, O, K), _r(O)
    with nn.conv_formulation(mode):
        got = nn.conv_transpose1d(x, w, b, stride=s, padding=p, output_padding=op, dilation=d)
    want = loops.conv_transpose1d(x, w, b, s, p, op, d)
    assert got.shape == want.shape
    assert rel_l2(got, want) < 1e-6


def test_conv_transpose1d_is_adjoint_of_strided_conv():
    # <convT(x), y> == <x, conv(y)> with the same weight, stride, padding.
    C, O, T, K, s, p = 3, 2, 11, 4, 2, 1
    x, w = _r(1, C, T), _r(C, O, K)
    yt = nn.conv_transpose1d(x, w, None, stride=s, padding=p)
    y = _r(*yt.shape)
    cy = loops.conv1d(y, w, None, s, p, p, 1)[:, :, :T]
    lhs = float((yt.astype(np.float64) * y).sum())
    rhs = float((x.astype(np.float64) * cy).sum())
    assert abs(lhs - rhs) < 1e-4 * max(1.0, abs(lhs))


def test_conv_formulations_agree_on_a_decoder_stage():
    """The "taps" formulation used by the full-size parity tests against the
    reference's einsum formulation on one 40k ResBlock group and one upsample
    shape (C = 32, k = 11, d = 5; ConvTranspose k16 s10)."""
    x, w = _r(2, 32, 3000), _r(32, 32, 11)
    a = nn.conv1d(x, w, None, padding=25, dilation=5)
    with nn.conv_formulation("taps"):
        b = nn.conv1d(x, w, None, padding=25, dilation=5)
    assert rel_l2(b, a) < 1e-6
    x, w = _r(2, 16, 300), _r(16, 8, 16)
    a = nn.conv_transpose1d(x, w, None, stride=10, padding=3)
    with nn.conv_formulation("taps"):
        b = nn.conv_transpose1d(x, w, None, stride=10, padding=3)
    assert rel_l2(b, a) < 1e-6
    with pytest.raises(ValueError):
        with nn.conv_formulation("fft"):
            pass


def test_layer_norm_softmax_match_loops():
    x, g, b = _r(5, 7), _r(7), _r(7)
    assert rel_l2(nn.layer_norm(x, g, b), loops.layer_norm(x, g, b)) < 1e-6
    s = nn.softmax(x * 4)
    assert rel_l2(s, loops.softmax(x * 4)) < 1e-6
    np.testing.assert_allclose(s.sum(-1), 1.0, rtol=1e-6)
    # shift invariance
    assert rel_l2(nn.softmax(x * 4 + 3.0), s) < 1e-6


def test_elementwise_definitions():
    x = np.array([-2.0, -0.0, 0.0, 1.5], dtype=np.float32)
    np.testing.assert_array_equal(nn.leaky_relu(x, 0.1), np.array([-0.2, -0.0, 0.0, 1.5], np.float32))
    np.testing.assert_allclose(nn.sigmoid(np.array([-80.0, 0.0, 80.0], np.float32)), [0.0, 0.5, 1.0], atol=1e-30)
    np.testing.assert_array_equal(nn.relu(x), np.maximum(x, 0))
    t = _r(6, 4)
    np.testing.assert_array_equal(nn.embedding(np.array([[0, -1]]), t), t[[0, 5]][None])
    x2, w2, b2 = _r(3, 5), _r(4, 5), _r(4)
    np.testing.assert_allclose(nn.linear(x2, w2, b2), x2.astype(np.float64) @ w2.T + b2, rtol=1e-5)


def test_deweight_norm_closed_form():
    v = _r(4, 3, 5)
    norm = np.sqrt((v.astype(np.float64) ** 2).reshape(4, -1).sum(1))
    g = (norm * np.array([0.5, 1, 2, 3])).astype(np.float32).reshape(4, 1, 1)
    W = V.deweight_norm(v, g)
    np.testing.assert_allclose(W, v * np.array([0.5, 1, 2, 3]).reshape(4, 1, 1), rtol=2e-6)
    # special case g = ||v|| -> W = v
    W1 = V.deweight_norm(v, norm.astype(np.float32))
    np.testing.assert_allclose(W1, v, rtol=2e-6)


@pytest.mark.parametrize("P", [1, 5, 11, 12, 40])
def test_relative_embedding_and_remaps_by_index(P):
    w = 10
    emb = _r(1, 2 * w + 1, 3)
    used = V.get_relative_embeddings(emb, P, w)
    assert used.shape == (1, 2 * P - 1, 3)
    for j in range(2 * P - 1):
        r = j - (P - 1)
        want = emb[0, r + w] if abs(r) <= w else np.zeros(3, np.float32)
        np.testing.assert_array_equal(used[0, j], want)
    X = _r(1, 2, P, 2 * P - 1)
    A = V.relative_to_absolute(X)
    for t in range(P):
        for s in range(P):
            assert A[0, 1, t, s] == X[0, 1, t, s - t + P - 1]
    Y = _r(1, 2, P, P)
    R = V.absolute_to_relative(Y)
    for t in range(P):
        for j in range(2 * P - 1):
            s = t + j - (P - 1)
            want = Y[0, 0, t, s] if 0 <= s < P else 0.0
            assert R[0, 0, t, j] == want


def test_attention_matches_banded_loops():
    from rvc_hip import synthetic as syn

    geom = syn.GEOM_TINY
    w = syn.make_weights(geom, seed=9)
    cfg = V.VitsConfig(w, sr=40000)
    P = 14
    kc = cfg.k_channels
    q, k, v = _r(1, cfg.hidden, P), _r(1, cfg.hidden, P), _r(1, cfg.hidden, P)
    a = "enc_p.encoder.attn_layers.0"
    # the oracle's attention core, pulled out of TextEncoder.encode
    qh = q.reshape(1, 2, kc, P).transpose(0, 1, 3, 2)
    kh = k.reshape(1, 2, kc, P).transpose(0, 1, 3, 2)
    vh = v.reshape(1, 2, kc, P).transpose(0, 1, 3, 2)
    qs = qh / np.sqrt(kc)
    sc = np.matmul(qs, kh.swapaxes(-1, -2))
    uk = V.get_relative_embeddings(w[f"{a}.emb_rel_k"], P, 10)
    sc = sc + V.relative_to_absolute(np.matmul(qs, uk[0].T))
    p = nn.softmax(sc)
    uv = V.get_relative_embeddings(w[f"{a}.emb_rel_v"], P, 10)
    out = np.matmul(p, vh) + np.matmul(V.absolute_to_relative(p), uv[0])
    for h in range(2):
        want = loops.relpos_attention(qh[0, h], kh[0, h], vh[0, h],
                                      w[f"{a}.emb_rel_k"][0], w[f"{a}.emb_rel_v"][0])
        assert rel_l2(out[0, h], want) < 1e-5


def test_sine_source_special_cases_and_loops():
    from rvc_hip import synthetic as syn

    w = syn.make_weights(syn.GEOM_TINY, seed=11)
    cfg = V.VitsConfig(w, sr=40000)
    gen = V.GeneratorNSF(w, cfg)
    wl = float(w["dec.m_source.l_linear.weight"][0, 0])
    bl = float(w["dec.m_source.l_linear.bias"][0])
    P, upp = 6, cfg.upp
    ns = _r(1, P * upp, 1)
    # f0 == 0 everywhere: har = tanh(w * (0.1/3) * ns + b)
    har0 = gen.sine_gen(np.zeros((1, P), np.float32), ns)
    np.testing.assert_allclose(har0.reshape(-1), np.tanh(wl * (0.1 / 3) * ns.reshape(-1).astype(np.float64) + bl),
                               atol=2e-6)
    # general f0 against the float64 definition
    rng = np.random.default_rng(3)
    f0 = syn.make_f0(P, rng)
    got = gen.sine_gen(f0, ns).reshape(-1)
    want = loops.sine_source(f0, ns, wl, bl, cfg.sr, upp)
    assert np.abs(got - want).max() < 2e-5
