# -*- coding: utf-8 -*-
"""The bf16-MFMA variant on the GPU.

Kernel level: rvc_conv1d_bf16 / rvc_conv_t1d_bf16 against an exact emulation
-- inputs and weights rounded to bf16 (nearest even) on the CPU, then summed
in float64 -- at relative L2 <= 5e-6 (the products of two bf16 are exact in
fp32, so only the fp32 summation order differs); the same outputs must differ
from the unrounded fp32 result by bf16-sized amounts, which shows the rounding
really happened.

Synthesis level (the tolerance config 5 states): waveform
SNR = 10 log10(sum ref^2 / sum (y - ref)^2) >= 40 dB against the fp32 numpy
oracle at 1 s and at config 5's full size (4 independent seeds x 10 s,
batch 4), and against the fp32 HIP path at full size.  The bf16
upsamplers are also checked stage by stage against an exact emulation.  Mode 2 (ResBlocks also bf16) is
reported separately; its SNR is recorded, with a loose floor."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from conftest import rel_l2
from oracle import nn_ref as nn
from oracle import vits_ref as V
from rvc_hip import synthetic as syn

pytestmark = pytest.mark.gpu


def bf16_round(a):
    """float32 -> nearest-even bf16, returned as float32."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def snr_db(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return 10.0 * math.log10(float((ref * ref).sum()) / max(float(((y - ref) ** 2).sum()), 1e-300))


@pytest.fixture(scope="module")
def ctx():
    from rvc_hip import _hip, hip_ops

    assert _hip.has_so, _hip.so_load_error
    return hip_ops.get_context()


def _r(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def _call(ctx, name, *args):
    from rvc_hip import _hip

    rc = getattr(ctx._lib, name)(ctx.handle, *args)
    assert rc == 0, _hip.last_error()


@pytest.mark.parametrize("B,Ci,Co,T,K,pad,d", [
    (2, 40, 70, 300, 3, 2, 1),        # channel counts off the 8 / 32 grid
    (1, 192, 576, 1000, 1, 0, 1),     # enc_p q/k/v GEMM
    (1, 256, 128, 2000, 11, 25, 5),   # a ResBlock conv (k 11, dilation 5)
    (1, 32, 32, 5000, 7, 9, 3),       # narrow late stage
])
def test_conv1d_bf16_matches_exact_emulation(ctx, B, Ci, Co, T, K, pad, d):
    rng = np.random.default_rng(Ci + K)
    x, w, b = _r(rng, B, Ci, T), _r(rng, Co, Ci, K, scale=1 / np.sqrt(Ci * K)), _r(rng, Co)
    L_out = T + 2 * pad - d * (K - 1)
    xi, wi, bi, oi = ctx.upload(x), ctx.upload(w), ctx.upload(b), ctx.alloc(B * Co * L_out)
    _call(ctx, "rvc_conv1d_bf16", xi, wi, bi, oi, B, Ci, T, Co, K, 1, pad, pad, d)
    got = ctx.download(oi, (B, Co, L_out))
    emu = nn.conv1d(bf16_round(x).astype(np.float64), bf16_round(w).astype(np.float64), None, padding=pad,
                    dilation=d) + b.astype(np.float64)[None, :, None]
    assert rel_l2(got, emu) < 5e-6
    full = nn.conv1d(x, w, b, padding=pad, dilation=d)
    assert 1e-4 < rel_l2(got, full) < 2e-2


@pytest.mark.parametrize("Ci,Co,L,K,s,p", [(64, 32, 100, 16, 10, 3), (128, 64, 200, 4, 2, 1), (512, 256, 50, 16, 10, 3),
                                           (20, 12, 33, 24, 12, 6)])
def test_conv_t1d_bf16_matches_exact_emulation(ctx, Ci, Co, L, K, s, p):
    rng = np.random.default_rng(Ci * K)
    x, w, b = _r(rng, 1, Ci, L), _r(rng, Ci, Co, K, scale=1 / np.sqrt(Ci)), _r(rng, Co)
    L_out = (L - 1) * s - 2 * p + K
    xi, wi, bi, oi = ctx.upload(x), ctx.upload(w), ctx.upload(b), ctx.alloc(Co * L_out)
    _call(ctx, "rvc_conv_t1d_bf16", xi, wi, bi, oi, 1, Ci, L, Co, K, s, p, 0, 1)
    got = ctx.download(oi, (1, Co, L_out))
    emu = nn.conv_transpose1d(bf16_round(x).astype(np.float64), bf16_round(w).astype(np.float64), None, stride=s,
                              padding=p) + b.astype(np.float64)[None, :, None]
    assert rel_l2(got, emu) < 5e-6
    assert 1e-4 < rel_l2(got, nn.conv_transpose1d(x, w, b, stride=s, padding=p)) < 2e-2


def test_bf16_op_limits(ctx):
    from rvc_hip import _hip

    a = ctx.alloc(4096)
    assert ctx._lib.rvc_conv1d_bf16(ctx.handle, a, a, 0, a, 1, 4, 100, 4, 3, 2, 1, 1, 1) == -1  # stride 2
    assert "conv1d_bf16" in _hip.last_error()
    assert ctx._lib.rvc_conv_t1d_bf16(ctx.handle, a, a, 0, a, 1, 4, 50, 4, 3, 2, 1, 0, 2) == -1  # dilation 2


def _synth(w, geom, precision):
    from rvc_hip.synth import HipSynthesizer

    return HipSynthesizer(w, sr=geom.sr, precision=precision)


def test_precision_is_set_before_finalize(ctx):
    from rvc_hip import _hip

    geom = syn.GEOM_TINY
    s = _synth(syn.make_weights(geom, seed=1), geom, 1)
    assert s._lib.rvc_synth_set_precision(s.handle, 0) == -1
    assert "already finalized" in _hip.last_error()
    with pytest.raises(RuntimeError):
        _synth(syn.make_weights(geom, seed=1), geom, 3)


def _stack_inputs(geom, P, seeds):
    ins = [syn.make_synth_inputs(geom, P, seed=sd) for sd in seeds]
    cat = {k: np.concatenate([i[k] for i in ins], axis=0) for k in ("phone", "pitch", "nsff0", "nz", "ns")}
    cat["sid"] = np.concatenate([i["sid"] for i in ins], axis=0)
    return ins, cat


def test_config5_1s_snr_vs_oracle():
    """Mode 1 (config 5's split: ups + enc_p matmuls in bf16) against the fp32
    numpy oracle, 4 seeds as one batch of 1 s each."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    ins, cat = _stack_inputs(geom, 100, (21, 22, 23, 24))
    s1 = _synth(w, geom, 1)
    y = s1.infer_controlled(cat["phone"], cat["pitch"], cat["nsff0"], cat["sid"], cat["nz"], cat["ns"])
    ref = V.Synthesizer(w, sr=geom.sr)
    for b, i in enumerate(ins):
        want = ref.infer_controlled(i["phone"], i["pitch"], i["nsff0"], i["sid"], i["nz"], i["ns"])
        assert snr_db(y[b:b + 1], want) >= 40.0


def test_bf16_upsamplers_match_exact_emulation():
    """Mode 1's upsamplers run the output-stationary ConvTranspose on bf16
    operands, the noise conv fused in fp32.  Stage by stage, from the GPU's
    own stage input: leaky ReLU, operands rounded to bf16, the transposed
    convolution summed in float64, + bias + the fp32 noise conv, then the fp32
    ResBlocks; the GPU's stage output must match at rel L2 2e-5 (fp32
    summation order only) and differ from the unrounded fp32 result by
    bf16-sized amounts."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=4)
    s = _synth(w, geom, 1)
    s.set_debug(True)
    P = 40
    inp = syn.make_synth_inputs(geom, P, seed=77)
    s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    ref = V.Synthesizer(w, sr=geom.sr)
    cfg = ref.cfg
    U = w["dec.conv_pre.weight"].shape[0]
    har = s.read("har", (1, P * geom.upp))[:, None, :]
    L = P
    for i in range(cfg.n_ups):
        C = U >> (i + 1)
        xh = s.read(f"dec_stage{i - 1}" if i > 0 else "dec_pre", (1, U >> i, L))
        y = nn.leaky_relu(xh, 0.1)
        up = f"dec.ups.{i}"
        wt = V.deweight_norm(w[up + ".weight_v"], w[up + ".weight_g"])
        st, K = cfg.upsample_rates[i], cfg.upsample_kernels[i]
        pad = (K - st) // 2
        noise = nn.conv1d(har, w[f"dec.noise_convs.{i}.weight"], w[f"dec.noise_convs.{i}.bias"],
                          stride=cfg.noise_strides[i], padding=cfg.noise_strides[i] // 2)
        emu = nn.conv_transpose1d(bf16_round(y).astype(np.float64), bf16_round(wt).astype(np.float64), None,
                                  stride=st, padding=pad) + w[up + ".bias"].astype(np.float64)[None, :, None]
        full = nn.conv_transpose1d(y, wt, w[up + ".bias"], stride=st, padding=pad)
        outs = []
        for yy in (emu.astype(np.float32) + noise, full + noise):
            xs = None
            for j, k in enumerate((3, 7, 11)):
                o = V.resblock1(w, f"dec.resblocks.{3 * i + j}", k, yy)
                xs = o if xs is None else xs + o
            outs.append(xs / 3)
        L *= st
        got = s.read(f"dec_stage{i}", (1, C, L))
        assert rel_l2(got, outs[0]) < 2e-5, f"stage {i}"
        assert rel_l2(got, outs[1]) > 1e-4, f"stage {i}: no bf16 rounding visible"


def test_config5_full_size_vs_oracle():
    """BASELINE config 5 as stated: 4 independent seeds x 10 s as one batch of
    4, upsamplers and enc_p matmuls on bf16, each wave against the fp32 numpy
    oracle (taps formulation) at SNR >= 40 dB; the per-seed margin is
    printed."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    ins, cat = _stack_inputs(geom, 1000, (31, 32, 33, 34))
    y = _synth(w, geom, 1).infer_controlled(cat["phone"], cat["pitch"], cat["nsff0"], cat["sid"], cat["nz"],
                                           cat["ns"])
    ref = V.Synthesizer(w, sr=geom.sr)
    snrs = []
    with nn.conv_formulation("taps"):
        for b, i in enumerate(ins):
            want = ref.infer_controlled(i["phone"], i["pitch"], i["nsff0"], i["sid"], i["nz"], i["ns"])
            snrs.append(snr_db(y[b:b + 1], want))
    print("config 5 SNR vs oracle per seed: " + ", ".join(f"{v:.2f} dB (margin {v - 40.0:+.2f})" for v in snrs))
    assert min(snrs) >= 40.0


def test_config5_full_size_snr():
    """Config 5 at full size: 4 seeds x 10 s, batch 4.  Mode 1 against the fp32
    HIP path (itself within 1e-3 max-abs of the oracle): SNR >= 40 dB per seed.
    Mode 2 (ResBlocks too) is measured and only held to a 20 dB floor; its
    figure is the one reported separately."""
    geom = syn.GEOM_40K
    w = syn.make_weights(geom, seed=0)
    _, cat = _stack_inputs(geom, 1000, (31, 32, 33, 34))
    args = (cat["phone"], cat["pitch"], cat["nsff0"], cat["sid"], cat["nz"], cat["ns"])
    y0 = _synth(w, geom, 0).infer_controlled(*args)
    y1 = _synth(w, geom, 1).infer_controlled(*args)
    y2 = _synth(w, geom, 2).infer_controlled(*args)
    assert y1.shape == (4, 1, 400000)
    snr1 = [snr_db(y1[b], y0[b]) for b in range(4)]
    snr2 = [snr_db(y2[b], y0[b]) for b in range(4)]
    print(f"config 5 SNR vs fp32: mode 1 {min(snr1):.1f} dB, mode 2 {min(snr2):.1f} dB")
    assert min(snr1) >= 40.0
    assert min(snr2) >= 20.0
    assert np.isfinite(y2).all() and np.abs(y2).max() <= 1.0
