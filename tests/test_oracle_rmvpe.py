# -*- coding: utf-8 -*-
"""Pins ``oracle/rmvpe_ref.py``: each op against an independent
implementation (numpy's window, ``torch.stft``, ``torch.nn.functional``
convolutions and pooling, ``torch.nn.GRU``, a float64 decode loop), and the
whole model against golden vectors written by the reference's own numpy
RMVPE (``tests/golden/make_golden_rmvpe.py``)."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import rmvpe_ref as R
from rvc_hip import synthetic as syn

torch = pytest.importorskip("torch")
F = torch.nn.functional

GOLD = os.path.join(os.path.dirname(__file__), "golden", "rmvpe.npz")


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


@pytest.fixture(scope="module")
def model(gold):
    w = syn.make_rmvpe_weights(int(gold["wseed"]))
    assert syn.weights_digest(w) == str(gold["weights_digest"])
    return R.Rmvpe(w)


def test_window_is_numpy_hanning():
    np.testing.assert_allclose(R.hann_sym(1024), np.hanning(1024), rtol=0, atol=1e-15)


def test_stft_mag_vs_torch():
    x = syn.make_rmvpe_audio(5000, 4).astype(np.float64)
    ref = torch.stft(torch.from_numpy(x), 1024, 160, 1024, window=torch.hann_window(1024, periodic=False,
                     dtype=torch.float64), center=True, pad_mode="reflect", return_complex=True).abs().numpy()
    got = R.stft_mag(x)
    assert got.shape == ref.shape == (513, R.n_frames(5000))
    np.testing.assert_allclose(got, ref.astype(np.float32), rtol=1e-6, atol=1e-9)


def test_mel_filter_bank(gold):
    fb = R.mel_filter_htk()
    np.testing.assert_allclose(fb.astype(np.float32), gold["mel_basis"], rtol=0, atol=1e-8)
    np.testing.assert_allclose(fb.sum(1), 1.0, atol=1e-12)
    # each triangle peaks at the FFT bin nearest its HTK centre frequency
    mel = lambda f: 1127.0 * np.log1p(f / 700.0)  # noqa: E731
    centres = 700.0 * np.expm1(np.linspace(mel(30.0), mel(8000.0), 130)[1:-1] / 1127.0)
    freqs = np.linspace(0, 8000, 513)
    for i in (0, 40, 127):
        near = np.argsort(np.abs(freqs - centres[i]))[:2]
        assert np.argmax(fb[i]) in near


def test_conv2d_and_transpose_vs_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 5, 7, 9)).astype(np.float32)
    w = rng.standard_normal((6, 5, 3, 3)).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    ref = F.conv2d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b), padding=1).numpy()
    np.testing.assert_allclose(R.conv2d(x, w, b, 1), ref, rtol=1e-5, atol=1e-5)
    w1 = rng.standard_normal((6, 5, 1, 1)).astype(np.float32)
    ref1 = F.conv2d(torch.from_numpy(x), torch.from_numpy(w1), torch.from_numpy(b)).numpy()
    np.testing.assert_allclose(R.conv2d(x, w1, b, 0), ref1, rtol=1e-5, atol=1e-5)
    wt = rng.standard_normal((5, 4, 3, 3)).astype(np.float32)
    reft = F.conv_transpose2d(torch.from_numpy(x), torch.from_numpy(wt), stride=2, padding=1,
                              output_padding=1).numpy()
    got = R.conv_transpose2d(x, wt)
    assert got.shape == reft.shape == (2, 4, 14, 18)
    # the reference pads the flipped-kernel conv symmetrically and zero-fills
    # the output-padding row and column (rmvpe.py:369-383), so its last row
    # and column miss the kh = 2 / kw = 2 taps torch adds there
    np.testing.assert_allclose(got[:, :, :-1, :-1], reft[:, :, :-1, :-1], rtol=1e-5, atol=1e-5)
    assert not got[:, :, -1, :].any() and not got[:, :, :, -1].any()
    assert np.abs(reft[:, :, -1, :]).max() > 0.1
    np.testing.assert_allclose(R.avg_pool2(x[:, :, :6, :8]),
                               F.avg_pool2d(torch.from_numpy(x[:, :, :6, :8]), 2).numpy(), rtol=1e-6, atol=1e-7)


def test_bigru_vs_torch():
    rng = np.random.default_rng(1)
    T, I, H = 19, 12, 8
    gru = torch.nn.GRU(I, H, batch_first=True, bidirectional=True)
    x = rng.standard_normal((T, I)).astype(np.float32)
    with torch.no_grad():
        ref = gru(torch.from_numpy(x)[None])[0][0].numpy()
    p = {k: v.detach().numpy() for k, v in gru.named_parameters()}
    got = R.bigru(x, p["weight_ih_l0"], p["weight_hh_l0"], p["bias_ih_l0"], p["bias_hh_l0"],
                  p["weight_ih_l0_reverse"], p["weight_hh_l0_reverse"], p["bias_ih_l0_reverse"],
                  p["bias_hh_l0_reverse"])
    assert got.shape == (T, 2 * H)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def _decode_loop(sal, thred=0.03):
    """float64 restatement of the local-average decode, one frame at a time."""
    cents = [0.0] * 4 + [20.0 * i + 1997.3794084376191 for i in range(360)] + [0.0] * 4
    out = []
    for row in np.asarray(sal, np.float64):
        c = int(np.argmax(row)) + 4
        pad = [0.0] * 4 + list(row) + [0.0] * 4
        num = sum(pad[j] * np.float64(np.float32(cents[j])) for j in range(c - 4, c + 5))
        den = sum(pad[j] for j in range(c - 4, c + 5))
        v = num / den if max(pad) > thred else 0.0
        out.append(v)
    return np.array(out)


def test_decode(gold):
    sal = gold["dec_sal"]
    np.testing.assert_array_equal(R.to_local_average_cents(sal), gold["dec_cents"])
    np.testing.assert_array_equal(R.decode(sal), gold["dec_f0"])
    np.testing.assert_allclose(R.to_local_average_cents(sal), _decode_loop(sal), rtol=1e-6)
    f0 = R.decode(sal)
    assert f0[3] == 0 and f0[4] == 0 and f0[5] > 0


@pytest.mark.parametrize("clip", [0, 1])
def test_end_to_end_vs_reference(gold, model, clip):
    x = gold[f"x{clip}"]
    mel = model.mel(x)
    assert rel_l2(mel, gold[f"mel{clip}"]) < 1e-6
    hidden = model.mel2hidden(mel[None])[0]
    assert hidden.shape == gold[f"hidden{clip}"].shape
    assert rel_l2(hidden, gold[f"hidden{clip}"]) < 1e-5
    f0 = R.decode(hidden)
    ref = gold[f"f0_{clip}"]
    srt = np.sort(gold[f"hidden{clip}"], axis=1)
    clear = (srt[:, -1] - srt[:, -2]) > 1e-4      # argmax not decided by rounding
    assert clear.mean() > 0.9
    np.testing.assert_allclose(f0[clear], ref[clear], rtol=1e-4)
