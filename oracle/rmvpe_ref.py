# -*- coding: utf-8 -*-
"""numpy restatement of RMVPE pitch extraction (16 kHz audio -> f0 per 10 ms).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``runtime/models/rmvpe.py`` (numpy path: ``RMVPE.infer_from_audio``
with ``_unet_batch_flag`` off and the host BiGRU), ``runtime/dsp/fft.py``
(``stft``), ``runtime/dsp/mel.py`` / ``runtime/dsp/utils.py`` (HTK mel
filter bank) and ``runtime/nn.py`` (``sigmoid``, ``linear``), in float32
where the reference is float32 and float64 where it is float64 (the STFT),
with the reference's expression order.

The model (``E2E(4, 1, (2, 2))``): log-mel [F, 128] -> input BatchNorm ->
5 encoder levels (4 ConvBlockRes each, AvgPool 2x2 after each level) ->
4 intermediate levels (4 ConvBlockRes, 256 -> 512 channels) -> 5 decoder
levels (ConvTranspose2d 3x3 s2 + BN + ReLU, concat with the encoder level,
4 ConvBlockRes) -> cnn Conv2d 16 -> 3 -> BiGRU(384, 256) -> Linear(512, 360)
-> sigmoid -> local-average cents -> Hz.

Pinning (``tests/test_oracle_rmvpe.py``): ``stft_mag`` against
``torch.stft`` (symmetric Hann, reflect padding); ``mel_filter_htk`` against
the golden filter bank the reference's own ``mel_filter_bank`` wrote, and
its closed-form properties (unit row sums, triangle peaks at the HTK
centres); ``conv2d`` / ``conv_transpose2d`` against
``torch.nn.functional``; ``bigru`` against ``torch.nn.GRU``
(bidirectional); ``decode`` against golden vectors of the reference's
``RMVPE.decode`` on crafted salience (ties, edge bins, silent frames) and a
float64 loop; ``infer_from_audio`` end to end (mel, salience, f0) against
golden vectors of the reference's own ``RMVPE`` on random-init weights
(``tests/golden/make_golden_rmvpe.py``).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "SR", "N_FFT", "HOP", "N_MELS", "FMIN", "FMAX", "MEL_CLAMP", "N_BINS_OUT",
    "hann_sym", "stft_mag", "mel_filter_htk", "log_mel", "n_frames",
    "bn_scale_shift", "conv2d", "conv_transpose2d", "avg_pool2", "conv_block_res",
    "Rmvpe", "bigru", "sigmoid", "cents_mapping", "to_local_average_cents", "decode",
]

SR, N_FFT, HOP, N_MELS = 16000, 1024, 160, 128        # rmvpe.py:57-62
FMIN, FMAX, MEL_CLAMP = 30.0, 8000.0, 1e-5            # rmvpe.py:63-65
N_BINS_OUT = 360                                      # rmvpe.py:567
_F32 = np.float32


# ------------------------------------------------------------------ mel
def hann_sym(n: int) -> np.ndarray:
    """``np.hanning(n)`` (symmetric Hann: 0.5 - 0.5 cos(2 pi k / (n - 1))),
    the window ``get_window("hann")`` returns (``runtime/dsp/fft.py:36-38``)."""
    k = np.arange(n, dtype=np.float64)
    return 0.5 - 0.5 * np.cos(2.0 * np.pi * k / (n - 1))


def n_frames(T: int) -> int:
    """STFT frame count with center padding: 1 + T // hop (``fft.py:102``)."""
    return 1 + T // HOP


def stft_mag(x: np.ndarray) -> np.ndarray:
    """|STFT| [513, F] float32 of a 1-D signal (``runtime/dsp/fft.py:59-113``
    with n_fft 1024, hop 160, symmetric Hann, center reflect padding; the FFT
    is float64, the magnitude cast to float32 as ``rmvpe.py:638``)."""
    x = np.asarray(x, dtype=np.float64)
    pad = N_FFT // 2
    if len(x) <= pad:
        raise ValueError("signal too short for reflect padding")
    xp = np.pad(x, (pad, pad), mode="reflect")
    F = 1 + (len(xp) - N_FFT) // HOP
    idx = np.arange(N_FFT)[None, :] + HOP * np.arange(F)[:, None]
    frames = xp[idx] * hann_sym(N_FFT)[None, :]
    return np.abs(np.fft.rfft(frames, axis=1).T).astype(_F32)


def mel_filter_htk(sr: int = SR, n_fft: int = N_FFT, n_mels: int = N_MELS, fmin: float = FMIN,
                   fmax: float = FMAX) -> np.ndarray:
    """HTK-scale triangular filters with unit row sums, float64
    [n_mels, n_fft/2+1] (``runtime/dsp/mel.py:68-122``; mel = 1127 ln(1 +
    f/700), ``runtime/dsp/utils.py:23-47``)."""
    n_bins = n_fft // 2 + 1
    freqs = np.linspace(0.0, sr / 2.0, n_bins)
    m_lo = 1127.0 * np.log1p(fmin / 700.0)
    m_hi = 1127.0 * np.log1p(fmax / 700.0)
    edges = 700.0 * np.expm1(np.linspace(m_lo, m_hi, n_mels + 2) / 1127.0)
    out = np.zeros((n_mels, n_bins))
    for i in range(n_mels):
        lo, c, hi = edges[i], edges[i + 1], edges[i + 2]
        rise = (freqs - lo) / (c - lo) if c > lo else np.zeros(n_bins)
        fall = (hi - freqs) / (hi - c) if hi > c else np.zeros(n_bins)
        tri = np.maximum(0.0, np.minimum(rise, fall))
        tot = tri.sum()
        out[i] = tri / tot if tot > 0 else tri
    return out


def log_mel(x: np.ndarray, basis32: np.ndarray) -> np.ndarray:
    """[128, F] float32 log-mel (``RMVPE._extract_mel``, ``rmvpe.py:632-640``)."""
    mel = basis32 @ stft_mag(x)
    return np.log(np.clip(mel, MEL_CLAMP, None)).astype(_F32)


# ------------------------------------------------------------------ U-Net ops
def bn_scale_shift(w: dict, prefix: str):
    """Inference BatchNorm as (scale, shift), float32 (``rmvpe.py:507-515``)."""
    g = w[prefix + ".weight"].astype(_F32)
    b = w[prefix + ".bias"].astype(_F32)
    rm = w[prefix + ".running_mean"].astype(_F32)
    rv = w[prefix + ".running_var"].astype(_F32)
    scale = g / np.sqrt(rv + 1e-5)
    return scale, b - rm * scale


def _bn(x, ss):
    s, t = ss
    shape = (1, -1) + (1,) * (x.ndim - 2)
    return x * s.reshape(shape) + t.reshape(shape)


def conv2d(x: np.ndarray, w: np.ndarray, b=None, pad: int = 1) -> np.ndarray:
    """Stride-1 conv2d, x [B, C, H, W], w [O, C, KH, KW], zero padding
    ``pad`` (``runtime/nn.py:200-260`` im2col + matmul semantics)."""
    B, C, H, W = x.shape
    O, _, KH, KW = w.shape
    OH, OW = H + 2 * pad - KH + 1, W + 2 * pad - KW + 1
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    cols = np.empty((B, C, KH, KW, OH, OW), dtype=x.dtype)
    for i in range(KH):
        for j in range(KW):
            cols[:, :, i, j] = xp[:, :, i:i + OH, j:j + OW]
    out = np.einsum("ok,bkp->bop", w.reshape(O, -1), cols.reshape(B, C * KH * KW, OH * OW), optimize=True)
    out = out.reshape(B, O, OH, OW)
    if b is not None:
        out = out + np.asarray(b, dtype=out.dtype).reshape(1, -1, 1, 1)
    return out


def conv_transpose2d(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """ConvTranspose2d 3x3, stride 2, padding 1, output_padding 1, no bias;
    w [C_in, C_out, 3, 3] (``rmvpe.py:319-384``: zero insertion between input
    samples, flipped kernel, plain conv with padding K-1-p, output padded to
    (H-1)*2 - 2 + 3 + 1 = 2H).  Because the padding is symmetric and the
    extra row / column is zero-filled, output row 2H-1 and column 2W-1 are 0
    (torch adds the kh = 2 / kw = 2 taps there); this is the reference's
    result and the one reproduced here."""
    B, C, H, W = x.shape
    Co = w.shape[1]
    xu = np.zeros((B, C, 2 * H - 1, 2 * W - 1), dtype=x.dtype)
    xu[:, :, ::2, ::2] = x
    wf = np.ascontiguousarray(w.transpose(1, 0, 2, 3)[:, :, ::-1, ::-1])
    y = conv2d(xu, wf, None, pad=1)
    out = np.zeros((B, Co, 2 * H, 2 * W), dtype=y.dtype)
    out[:, :, :y.shape[2], :y.shape[3]] = y
    return out


def avg_pool2(x: np.ndarray) -> np.ndarray:
    """AvgPool2d(2, 2) (``rmvpe.py:387-390``)."""
    B, C, H, W = x.shape
    return x.reshape(B, C, H // 2, 2, W // 2, 2).mean(axis=(3, 5))


def conv_block_res(x, w: dict, bn: dict, p: str):
    """ConvBlockRes: relu(BN(conv3x3)) twice plus the identity or 1x1
    shortcut (``rmvpe.py:518-551``; BN layers are ``conv.1`` / ``conv.4``)."""
    y = np.maximum(_bn(conv2d(x, w[p + ".conv.0.weight"], None, 1), bn[p + ".conv.1"]), 0.0)
    y = np.maximum(_bn(conv2d(y, w[p + ".conv.3.weight"], None, 1), bn[p + ".conv.4"]), 0.0)
    if p + ".shortcut.weight" in w:
        return y + conv2d(x, w[p + ".shortcut.weight"], w.get(p + ".shortcut.bias"), 0)
    return y + x


# ------------------------------------------------------------------ head
def sigmoid(x):
    """``runtime/nn.py:520-523``."""
    x = np.asarray(x)
    with np.errstate(over="ignore"):
        return np.where(x >= 0, 1.0 / (1.0 + np.exp(-x)), np.exp(x) / (1.0 + np.exp(x)))


def bigru(x, w_ih, w_hh, b_ih, b_hh, w_ih_r, w_hh_r, b_ih_r, b_hh_r):
    """Bidirectional single-layer GRU over x [T, in] (PyTorch gate order r,
    z, n; ``rmvpe.py:393-442`` host path): returns [T, 2H], forward first."""
    def run(xs, wi, wh, bi, bh):
        H = wh.shape[0] // 3
        gx_all = xs @ wi.T + bi
        h = np.zeros(H, dtype=_F32)
        out = np.empty((xs.shape[0], H), dtype=_F32)
        with np.errstate(over="ignore", invalid="ignore"):
            for t in range(xs.shape[0]):
                gx = gx_all[t]
                gh = h @ wh.T + bh
                r = sigmoid(gx[:H] + gh[:H])
                z = sigmoid(gx[H:2 * H] + gh[H:2 * H])
                n = np.tanh(gx[2 * H:] + r * gh[2 * H:])
                h = (1.0 - z) * n + z * h
                out[t] = h
        return out

    fwd = run(x, w_ih, w_hh, b_ih, b_hh)
    rev = run(x[::-1, :], w_ih_r, w_hh_r, b_ih_r, b_hh_r)[::-1, :]
    return np.concatenate([fwd, rev], axis=-1)


def cents_mapping() -> np.ndarray:
    """20 * arange(360) + 1997.379..., zero padded by 4 each side, float32
    (``rmvpe.py:565-566``)."""
    return np.pad(20 * np.arange(360) + 1997.3794084376191, (4, 4)).astype(_F32)


def to_local_average_cents(sal: np.ndarray, thred: float = 0.03) -> np.ndarray:
    """Per frame: argmax bin c, salience-weighted mean of the cents of bins
    c-4 .. c+4 (zero outside the table), 0 where max salience <= thred
    (``rmvpe.py:906-924``)."""
    sal = np.asarray(sal, dtype=_F32)
    F = sal.shape[0]
    center = np.argmax(sal, axis=1) + 4
    sp = np.pad(sal, ((0, 0), (4, 4)))
    cols = (center - 4)[:, None] + np.arange(9)[None, :]
    rows = np.arange(F)[:, None]
    ts = sp[rows, cols]
    tc = cents_mapping()[cols]
    out = np.sum(ts * tc, axis=1) / np.sum(ts, axis=1)
    out[np.max(sp, axis=1) <= thred] = 0
    return out


def decode(sal: np.ndarray, thred: float = 0.03) -> np.ndarray:
    """Salience [F, 360] -> f0 [F] Hz; cents 0 -> 10 Hz -> 0 (``rmvpe.py:899-904``)."""
    c = to_local_average_cents(sal, thred)
    f0 = 10 * (2 ** (c / 1200))
    f0[f0 == 10] = 0
    return f0


# ------------------------------------------------------------------ model
class Rmvpe:
    """The numpy RMVPE on a float32 state dict with the checkpoint's keys."""

    def __init__(self, w: dict):
        self.W = {k: np.asarray(v, dtype=_F32) for k, v in w.items()}
        self.basis = mel_filter_htk().astype(_F32)
        self.bn = {}
        for k in self.W:
            if k.endswith(".running_mean"):
                p = k[: -len(".running_mean")]
                self.bn[p] = bn_scale_shift(self.W, p)

    def mel(self, x):
        return log_mel(x, self.basis)

    def unet_cnn(self, x):
        """[1, 1, F', 128] -> [1, 3, F', 128] (``rmvpe.py:643-735``)."""
        W, bn = self.W, self.bn
        x = _bn(x, bn["unet.encoder.bn"])
        skips = []
        for i in range(5):
            for j in range(4):
                x = conv_block_res(x, W, bn, f"unet.encoder.layers.{i}.conv.{j}")
            skips.append(x)
            x = avg_pool2(x)
        for i in range(4):
            for j in range(4):
                x = conv_block_res(x, W, bn, f"unet.intermediate.layers.{i}.conv.{j}")
        for i in range(5):
            p = f"unet.decoder.layers.{i}"
            y = np.maximum(_bn(conv_transpose2d(x, W[p + ".conv1.0.weight"]), bn[p + ".conv1.1"]), 0.0)
            x = np.concatenate([y, skips[-1 - i]], axis=1)
            for j in range(4):
                x = conv_block_res(x, W, bn, f"{p}.conv2.{j}")
        return conv2d(x, W["cnn.weight"], W["cnn.bias"], 1)

    def hidden_from_cnn(self, c):
        """[1, 3, F', 128] -> salience [1, F', 360] (``rmvpe.py:735-751``)."""
        W = self.W
        x = c.transpose(0, 2, 1, 3).reshape(c.shape[0], c.shape[2], -1)
        g = "fc.0.gru."
        h = bigru(x[0], W[g + "weight_ih_l0"], W[g + "weight_hh_l0"], W[g + "bias_ih_l0"], W[g + "bias_hh_l0"],
                  W[g + "weight_ih_l0_reverse"], W[g + "weight_hh_l0_reverse"], W[g + "bias_ih_l0_reverse"],
                  W[g + "bias_hh_l0_reverse"])
        return sigmoid(h[None] @ W["fc.1.weight"].T + W["fc.1.bias"].reshape(1, -1))

    def mel2hidden(self, mel):
        """[1, 128, F] -> [1, F, 360]: frames zero padded to a multiple of 32
        (``rmvpe.py:861-876``)."""
        F = mel.shape[-1]
        pad = 32 * ((F - 1) // 32 + 1) - F
        if pad > 0:
            mel = np.pad(mel, ((0, 0), (0, 0), (0, pad)), mode="constant")
        x = mel.transpose(0, 2, 1)[:, None, ...]
        return self.hidden_from_cnn(self.unet_cnn(x))[:, :F, :]

    def infer_from_audio(self, x, thred: float = 0.03):
        """[T] float32 16 kHz -> f0 [F] (``rmvpe.py:927-952``)."""
        x = np.asarray(x, dtype=_F32)
        mel = self.mel(x)[None]
        hidden = self.mel2hidden(mel)
        return decode(hidden[0], thred)
