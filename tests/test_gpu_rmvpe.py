# -*- coding: utf-8 -*-
"""GPU parity of RMVPE (``rvc_rmvpe_*`` session, ``rvc_conv2d``, ``rvc_gru``)
against the oracle (``oracle/rmvpe_ref.py``) and the reference's golden
vectors.

Bar: per-op relative L2 <= 1e-4 in fp32 (log-mel, the cnn output feeding the
GRU, the GRU output, the salience); f0 within relative 1e-4 on every frame
whose salience argmax is not decided by rounding (top-2 gap > 1e-4 in the
oracle), and those frames must be at least 90 % of the clip.  The decode
kernel on identical salience matches the oracle to float32 rounding of powf."""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from oracle import rmvpe_ref as R

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rmvpe.npz")
OP_TOL = 1e-4


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def clear_frames(sal):
    s = np.sort(np.asarray(sal), axis=1)
    return (s[:, -1] - s[:, -2]) > 1e-4


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def weights(gold):
    from rvc_hip import synthetic as syn

    w = syn.make_rmvpe_weights(int(gold["wseed"]))
    assert syn.weights_digest(w) == str(gold["weights_digest"])
    return w


@pytest.fixture(scope="module")
def hr(weights):
    from rvc_hip import _hip

    if not _hip.has_so:
        pytest.fail(f"HIP backend missing: {_hip.so_load_error}")
    from rvc_hip.rmvpe import HipRMVPE

    m = HipRMVPE(weights)
    yield m
    m.close()


@pytest.fixture(scope="module")
def oracle(weights):
    return R.Rmvpe(weights)


@pytest.mark.parametrize("clip", [0, 1])
def test_rmvpe_golden(hr, gold, clip):
    x = gold[f"x{clip}"]
    print(f"rmvpe golden clip {clip} T={len(x)}", flush=True)
    f0 = hr.infer_from_audio(x)
    assert f0.shape == gold[f"f0_{clip}"].shape and f0.dtype == np.float32
    assert rel_l2(hr.last_mel(), gold[f"mel{clip}"]) < OP_TOL
    hid = hr.last_hidden()[0]
    assert hid.shape == gold[f"hidden{clip}"].shape
    assert rel_l2(hid, gold[f"hidden{clip}"]) < OP_TOL
    ok = clear_frames(gold[f"hidden{clip}"])
    assert ok.mean() > 0.9
    np.testing.assert_allclose(f0[ok], gold[f"f0_{clip}"][ok], rtol=1e-4)


def test_rmvpe_vs_oracle_3s(hr, oracle):
    """3 s clip: F = 301 frames padded to 320 (deep levels of 10 x 4 points,
    split-K convolutions); each stage against the oracle."""
    from rvc_hip import synthetic as syn

    x = syn.make_rmvpe_audio(48000, 7)
    print("rmvpe vs oracle T=48000", flush=True)
    f0 = hr.infer_from_audio(x)
    F = R.n_frames(len(x))
    Fp = 32 * ((F - 1) // 32 + 1)
    mel = oracle.mel(x)
    assert rel_l2(hr.last_mel(), mel) < OP_TOL
    melp = np.pad(mel[None], ((0, 0), (0, 0), (0, Fp - F)))
    cnn = oracle.unet_cnn(melp.transpose(0, 2, 1)[:, None])             # [1, 3, Fp, 128]
    gin = cnn.transpose(0, 2, 1, 3).reshape(Fp, -1).T                   # [384, Fp]
    assert rel_l2(hr.read("gru_in", gin.shape), gin) < OP_TOL
    sal = oracle.hidden_from_cnn(cnn)[0]                                  # [Fp, 360]
    got = hr.read("salience", (sal.shape[1], Fp)).T
    assert rel_l2(got, sal) < OP_TOL
    ok = clear_frames(sal[:F])
    assert ok.mean() > 0.9
    np.testing.assert_allclose(f0[ok], R.decode(sal[:F])[ok], rtol=1e-4)


def test_rmvpe_silence_and_short_input(hr, oracle):
    """All-zero audio (every log-mel clamped) and the shortest legal input."""
    for x in (np.zeros(3200, np.float32), (0.1 * np.random.default_rng(3).standard_normal(513)).astype(np.float32)):
        print(f"rmvpe T={len(x)}", flush=True)
        f0 = hr.infer_from_audio(x)
        ref = oracle.infer_from_audio(x)
        assert f0.shape == ref.shape
        sal = oracle.mel2hidden(oracle.mel(x)[None])[0]
        assert rel_l2(hr.last_hidden()[0], sal) < OP_TOL
        ok = clear_frames(sal)
        np.testing.assert_allclose(f0[ok], ref[ok], rtol=1e-4)
    from rvc_hip import _hip

    with pytest.raises(RuntimeError, match="512"):
        hr.infer_from_audio(np.zeros(512, np.float32))
    assert "512" in _hip.last_error()


def _ctx():
    from rvc_hip.hip_ops import get_context

    return get_context()


@pytest.mark.parametrize("B,C_in,H,W,C_out,k,pad,stride", [
    (1, 16, 64, 128, 16, 3, 1, 1),      # encoder level 0 shape
    (1, 1, 32, 128, 16, 3, 1, 1),       # the first conv (one input channel)
    (2, 40, 9, 13, 24, 3, 1, 1),        # ragged: odd extents, partial tiles
    (1, 512, 8, 4, 512, 3, 1, 1),       # intermediate level: split-K
    (1, 64, 16, 8, 96, 1, 0, 1),        # 1x1 shortcut
    (1, 32, 20, 16, 32, 2, 0, 2),       # 2x2 stride-2 pooling conv
])
def test_conv2d_export_vs_oracle(B, C_in, H, W, C_out, k, pad, stride):
    from rvc_hip import _hip

    ctx = _ctx()
    L = _hip.get_lib()
    rng = np.random.default_rng(C_in * 7 + H)
    x = rng.standard_normal((B, C_in, H, W)).astype(np.float32)
    w = (rng.standard_normal((C_out, C_in, k, k)) / np.sqrt(C_in * k * k)).astype(np.float32)
    b = rng.standard_normal(C_out).astype(np.float32)
    OH, OW = (H + 2 * pad - k) // stride + 1, (W + 2 * pad - k) // stride + 1
    if stride == 1:
        ref = R.conv2d(x, w, b, pad)
    else:
        full = R.conv2d(x, w, b, pad)
        ref = full[:, :, ::stride, ::stride][:, :, :OH, :OW]
    ids = [ctx.upload(x), ctx.upload(w), ctx.upload(b), ctx.alloc(B * C_out * OH * OW)]
    try:
        print(f"conv2d {B}x{C_in}x{H}x{W} -> {C_out} k{k} s{stride}", flush=True)
        _hip._check(L.rvc_conv2d(ctx.handle, ids[0], ids[1], ids[2], ids[3], B, C_in, H, W, C_out, k, k, pad, pad,
                                 stride, stride), "rvc_conv2d")
        got = ctx.download(ids[3], (B, C_out, OH, OW))
    finally:
        for i in ids:
            ctx.free(i)
    assert rel_l2(got, ref) < OP_TOL


def test_conv2d_export_rejects_unsupported():
    from rvc_hip import _hip

    ctx = _ctx()
    L = _hip.get_lib()
    ids = [ctx.alloc(4096) for _ in range(3)]
    try:
        assert L.rvc_conv2d(ctx.handle, ids[0], ids[1], 0, ids[2], 1, 1, 16, 16, 1, 5, 5, 2, 2, 1, 1) == -1
        assert "3x3" in _hip.last_error()
        assert L.rvc_conv2d(ctx.handle, ids[0], ids[1], 0, ids[2], 1, 1, 16, 16, 1, 3, 3, 1, 1, 1, 2) == -1
    finally:
        for i in ids:
            ctx.free(i)


@pytest.mark.parametrize("T,I,H", [(37, 24, 16), (200, 384, 256), (5, 8, 100)])
def test_gru_export_vs_oracle(T, I, H):
    """rvc_gru on the reference's layout: gate inputs [2T][3H] from
    x @ W_ih^T + b_ih of each direction, W_hh [2][3H][H], b_hh [2][3H]."""
    from rvc_hip import _hip

    ctx = _ctx()
    L = _hip.get_lib()
    rng = np.random.default_rng(T + H)
    bound = 1.0 / np.sqrt(H)
    p = {k: rng.uniform(-bound, bound, s).astype(np.float32) for k, s in (
        ("wi", (3 * H, I)), ("wh", (3 * H, H)), ("bi", (3 * H,)), ("bh", (3 * H,)),
        ("wir", (3 * H, I)), ("whr", (3 * H, H)), ("bir", (3 * H,)), ("bhr", (3 * H,)))}
    x = rng.standard_normal((T, I)).astype(np.float32)
    ref = R.bigru(x, p["wi"], p["wh"], p["bi"], p["bh"], p["wir"], p["whr"], p["bir"], p["bhr"])
    gx = np.concatenate([x @ p["wi"].T + p["bi"], x @ p["wir"].T + p["bir"]], axis=0).astype(np.float32)
    ids = [ctx.upload(gx), ctx.upload(np.stack([p["wh"], p["whr"]])), ctx.upload(np.stack([p["bh"], p["bhr"]])),
           ctx.alloc(T * 2 * H)]
    try:
        print(f"gru T={T} H={H}", flush=True)
        _hip._check(L.rvc_gru(ctx.handle, ids[0], ids[1], ids[2], ids[3], T, H), "rvc_gru")
        got = ctx.download(ids[3], (T, 2 * H))
    finally:
        for i in ids:
            ctx.free(i)
    assert rel_l2(got, ref) < OP_TOL
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5)


def test_rmvpe_timing_breakdown(hr):
    from rvc_hip import synthetic as syn

    x = syn.make_rmvpe_audio(16000, 2)
    hr.set_timing("rmvpe")
    hr.infer_from_audio(x)
    t = hr.timing()
    hr.set_timing("")
    assert t["launches"] > 100 and t["ms"] > 0 and t["flops"] > 1e9


@pytest.mark.parametrize("B,C_in,ih,iw,C_out,kh,kw,sh,sw,ph,pw,oph,opw", [
    (1, 8, 5, 7, 6, 3, 3, 2, 2, 1, 1, 1, 1),     # RMVPE's decoder shape
    (2, 16, 4, 4, 8, 2, 2, 2, 2, 0, 0, 0, 0),
    (1, 12, 6, 5, 10, 3, 3, 1, 1, 1, 1, 0, 0),
    (1, 8, 5, 6, 4, 3, 2, 2, 1, 1, 0, 1, 0),     # different strides per axis
    (1, 8, 4, 5, 8, 1, 1, 2, 2, 0, 0, 1, 1),     # phases no tap reaches: zeros
    (1, 40, 9, 3, 24, 3, 3, 2, 2, 0, 1, 1, 0),
])
def test_conv_t2d_export_vs_torch(B, C_in, ih, iw, C_out, kh, kw, sh, sw, ph, pw, oph, opw):
    import torch

    from rvc_hip import _hip

    ctx = _ctx()
    L = _hip.get_lib()
    rng = np.random.default_rng(C_in + kh * 10 + sh)
    x = rng.standard_normal((B, C_in, ih, iw)).astype(np.float32)
    w = (rng.standard_normal((C_in, C_out, kh, kw)) / np.sqrt(C_in * kh * kw)).astype(np.float32)
    ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(x), torch.from_numpy(w), stride=(sh, sw),
                                               padding=(ph, pw), output_padding=(oph, opw)).numpy()
    H, W = ref.shape[2], ref.shape[3]
    ids = [ctx.upload(x), ctx.upload(w), ctx.alloc(B * C_out * H * W)]
    try:
        print(f"conv_t2d {x.shape} k{kh}x{kw} s{sh}x{sw} p{ph}x{pw} op{oph}x{opw}", flush=True)
        _hip._check(L.rvc_conv_t2d(ctx.handle, ids[0], ids[1], ids[2], B, C_in, ih, iw, C_out, kh, kw, sh, sw, ph, pw,
                                   oph, opw, H, W), "rvc_conv_t2d")
        got = ctx.download(ids[2], ref.shape)
        assert L.rvc_conv_t2d(ctx.handle, ids[0], ids[1], ids[2], B, C_in, ih, iw, C_out, kh, kw, sh, sw, ph, pw,
                              oph, opw, H + 1, W) == -1
        assert "formula" in _hip.last_error()
    finally:
        for i in ids:
            ctx.free(i)
    assert rel_l2(got, ref) < OP_TOL


def test_insert_zeros_then_conv2d_is_the_reference_transpose():
    """RMVPE's vulkan route for ConvTranspose2d (rmvpe.py:268-316): zero
    insertion on the device, then conv2d with the flipped kernel and padding
    1 -- the reference's formulation, zero last row and column included."""
    from rvc_hip import _hip

    ctx = _ctx()
    L = _hip.get_lib()
    rng = np.random.default_rng(11)
    C_in, C_out, H, W = 24, 16, 6, 5
    x = rng.standard_normal((1, C_in, H, W)).astype(np.float32)
    w = (rng.standard_normal((C_in, C_out, 3, 3)) / np.sqrt(C_in * 9)).astype(np.float32)
    wf = np.ascontiguousarray(w.transpose(1, 0, 2, 3)[:, :, ::-1, ::-1])
    ids = [ctx.upload(x), ctx.alloc(C_in * (2 * H - 1) * (2 * W - 1)), ctx.upload(wf),
           ctx.alloc(C_out * (2 * H - 1) * (2 * W - 1))]
    try:
        _hip._check(L.rvc_insert_zeros_2x(ctx.handle, ids[0], ids[1], C_in, H, W), "rvc_insert_zeros_2x")
        xu = ctx.download(ids[1], (1, C_in, 2 * H - 1, 2 * W - 1))
        _hip._check(L.rvc_conv2d(ctx.handle, ids[1], ids[2], 0, ids[3], 1, C_in, 2 * H - 1, 2 * W - 1, C_out, 3, 3,
                                 1, 1, 1, 1), "rvc_conv2d")
        y = ctx.download(ids[3], (1, C_out, 2 * H - 1, 2 * W - 1))
    finally:
        for i in ids:
            ctx.free(i)
    ref_u = np.zeros_like(xu)
    ref_u[:, :, ::2, ::2] = x
    np.testing.assert_array_equal(xu, ref_u)
    ref = R.conv_transpose2d(x, w)
    assert rel_l2(y, ref[:, :, :2 * H - 1, :2 * W - 1]) < OP_TOL


def test_batched_2d_ops_match_single_ops():
    """rvc_batch_add_{conv2d,conv_t2d,gru} (ffi.zig:1196, :1246, :1377): one
    batch that chains conv2d -> conv_t2d (with a bias) and runs a BiGRU gives
    the single-op results, checked against torch and the oracle; a record the
    backend cannot run is refused when it is added, not at commit."""
    import torch

    from rvc_hip import _hip

    ctx = _ctx()
    L = _hip.get_lib()
    rng = np.random.default_rng(5)
    C0, C1, C2, H, W = 16, 24, 8, 7, 10
    x = rng.standard_normal((1, C0, H, W)).astype(np.float32)
    w1 = (rng.standard_normal((C1, C0, 3, 3)) / np.sqrt(C0 * 9)).astype(np.float32)
    b1 = rng.standard_normal(C1).astype(np.float32)
    w2 = (rng.standard_normal((C1, C2, 3, 3)) / np.sqrt(C1 * 9)).astype(np.float32)
    b2 = rng.standard_normal(C2).astype(np.float32)
    T, Hd = 23, 32
    bound = 1.0 / np.sqrt(Hd)
    gx = rng.uniform(-1, 1, (2 * T, 3 * Hd)).astype(np.float32)
    whh = rng.uniform(-bound, bound, (2, 3 * Hd, Hd)).astype(np.float32)
    bhh = rng.uniform(-bound, bound, (2, 3 * Hd)).astype(np.float32)
    y1_ref = R.conv2d(x, w1, b1, 1)
    y2_ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(y1_ref), torch.from_numpy(w2),
                                                  torch.from_numpy(b2), stride=2, padding=1,
                                                  output_padding=1).numpy()
    OH, OW = 2 * H, 2 * W
    # gate inputs handed over directly: the oracle's W_ih selects each direction's half of [T][6H]
    sel = np.eye(6 * Hd, dtype=np.float32)
    zb = np.zeros(3 * Hd, np.float32)
    g_ref = R.bigru(np.concatenate([gx[:T], gx[T:]], axis=1), sel[:3 * Hd], whh[0], zb, bhh[0], sel[3 * Hd:],
                    whh[1], zb, bhh[1])
    ids = {k: ctx.upload(v) for k, v in (("x", x), ("w1", w1), ("b1", b1), ("w2", w2), ("b2", b2), ("gx", gx),
                                         ("whh", whh), ("bhh", bhh))}
    ids["y1"] = ctx.alloc(C1 * H * W)
    ids["y2"] = ctx.alloc(C2 * OH * OW)
    ids["g"] = ctx.alloc(T * 2 * Hd)
    try:
        print("batched conv2d -> conv_t2d + gru", flush=True)
        _hip._check(L.rvc_batch_begin(ctx.handle), "rvc_batch_begin")
        _hip._check(L.rvc_batch_add_conv2d(ctx.handle, ids["x"], ids["w1"], ids["b1"], ids["y1"], 1, C0, H, W, C1,
                                           3, 3, 1, 1, 1, 1), "rvc_batch_add_conv2d")
        assert L.rvc_batch_add_conv2d(ctx.handle, ids["x"], ids["w1"], 0, ids["y1"], 1, C0, H, W, C1, 5, 5, 2, 2,
                                      1, 1) == -1
        assert "3x3" in _hip.last_error()
        _hip._check(L.rvc_batch_add_conv_t2d(ctx.handle, ids["y1"], ids["w2"], ids["b2"], ids["y2"], 1, C1, H, W,
                                             C2, 3, 3, 2, 2, 1, 1, 1, 1, OH, OW), "rvc_batch_add_conv_t2d")
        _hip._check(L.rvc_batch_add_gru(ctx.handle, ids["gx"], ids["whh"], ids["bhh"], ids["g"], T, Hd),
                    "rvc_batch_add_gru")
        _hip._check(L.rvc_batch_commit(ctx.handle), "rvc_batch_commit")
        y1 = ctx.download(ids["y1"], y1_ref.shape)
        y2 = ctx.download(ids["y2"], y2_ref.shape)
        g = ctx.download(ids["g"], (T, 2 * Hd))
        _hip._check(L.rvc_conv2d(ctx.handle, ids["x"], ids["w1"], ids["b1"], ids["y1"], 1, C0, H, W, C1, 3, 3, 1, 1,
                                 1, 1), "rvc_conv2d")
        _hip._check(L.rvc_gru(ctx.handle, ids["gx"], ids["whh"], ids["bhh"], ids["g"], T, Hd), "rvc_gru")
        y1s = ctx.download(ids["y1"], y1_ref.shape)
        gs = ctx.download(ids["g"], (T, 2 * Hd))
    finally:
        for i in ids.values():
            ctx.free(i)
    np.testing.assert_array_equal(y1, y1s)
    np.testing.assert_array_equal(g, gs)
    assert rel_l2(y1, y1_ref) < OP_TOL
    assert rel_l2(y2, y2_ref) < OP_TOL
    np.testing.assert_allclose(g, g_ref, rtol=0, atol=1e-5)
