# -*- coding: utf-8 -*-
"""The rest of the reference's C ABI on the GPU, called through ctypes like
the reference's loader does: batch op codes 10-13 and 15-17
(engine/src/ffi.zig:888-912), the segment records (ffi.zig:636-878),
rvc_rmsnorm, the batched transfers and the stats exports.

Checks: the numpy oracle (gelu_erf, group_norm, the relative-position helpers
of runtime/models/vits.py:448-482) and float64 closed forms; segments against
the same op computed whole.  Tolerance: relative L2 <= 1e-5 for the fp32
reductions here (the engine self-test's bar is 1e-4, engine/test_ffi.py:
103-105); exact equality where the arithmetic is one rounding."""

from __future__ import annotations

import ctypes
import os
import struct

import numpy as np
import pytest

from conftest import rel_l2
from oracle import hubert_ref as H
from oracle import nn_ref as nn
from oracle import vits_ref as V

pytestmark = pytest.mark.gpu

F32P = ctypes.POINTER(ctypes.c_float)


def bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


@pytest.fixture(scope="module")
def ctx():
    from rvc_hip import _hip, hip_ops

    assert _hip.has_so, _hip.so_load_error
    c = hip_ops.HipContext()
    yield c
    c.close()


class Rec:
    """Record ops through the raw ABI and commit them as one batch."""

    def __init__(self, ctx):
        from rvc_hip import _hip

        self.ctx, self.L, self.hip = ctx, ctx._lib, _hip
        assert self.L.rvc_batch_begin(ctx.handle) == 0

    def add(self, op, a=0, b=0, c=0, *p):
        p = list(p) + [0] * (11 - len(p))
        rc = self.L.rvc_batch_add(self.ctx.handle, op, a, b, c, *p)
        assert rc == 0, self.hip.last_error()

    def call(self, name, *args):
        rc = getattr(self.L, name)(self.ctx.handle, *args)
        assert rc == 0, self.hip.last_error()

    def commit(self):
        assert self.L.rvc_batch_commit(self.ctx.handle) == 0, self.hip.last_error()


def _r(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- 10, 11
def test_gelu_and_bias_add(ctx):
    rng = np.random.default_rng(10)
    x = _r(rng, 10007, scale=2.0)
    a = _r(rng, 37, 48)
    bias = _r(rng, 48)
    xi, ai, bi = ctx.upload(x), ctx.upload(a), ctx.upload(bias)
    oi = ctx.alloc(a.size)
    r = Rec(ctx)
    r.add(10, xi, 0, 0, x.size)
    r.add(11, ai, bi, oi, a.size, 48)
    r.commit()
    g = ctx.download(xi, x.shape)
    want = H.gelu_erf(x)
    assert np.abs(g - want).max() < 2e-6 * max(1.0, np.abs(want).max())
    np.testing.assert_array_equal(ctx.download(oi, a.shape), a + bias[None, :])


# ---------------------------------------------------------------- 12, 13
@pytest.mark.parametrize("Hh,T,D", [(2, 77, 96), (12, 50, 64), (3, 1, 5), (1, 130, 33)])
def test_attention_scores_and_context(ctx, Hh, T, D):
    rng = np.random.default_rng(Hh * 1000 + T)
    C = Hh * D + 3  # row stride wider than H*D
    q, k, v = _r(rng, T, C), _r(rng, T, C), _r(rng, T, C)
    qi, ki, vi = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    si = ctx.alloc(Hh * T * T)
    r = Rec(ctx)
    r.add(12, qi, ki, si, Hh, T, D, C)
    r.commit()
    qh = q[:, :Hh * D].reshape(T, Hh, D).transpose(1, 0, 2).astype(np.float64)
    kh = k[:, :Hh * D].reshape(T, Hh, D).transpose(1, 0, 2).astype(np.float64)
    vh = v[:, :Hh * D].reshape(T, Hh, D).transpose(1, 0, 2).astype(np.float64)
    s = ctx.download(si, (Hh, T, T))
    assert rel_l2(s, qh @ kh.transpose(0, 2, 1)) < 1e-5
    w = nn.softmax(s.astype(np.float32), axis=-1)
    wi = ctx.upload(w)
    out = np.full((T, C), 7.0, np.float32)
    oi = ctx.upload(out)
    r = Rec(ctx)
    r.add(13, wi, vi, oi, Hh, T, D, C)
    r.commit()
    got = ctx.download(oi, (T, C))
    want = (w.astype(np.float64) @ vh).transpose(1, 0, 2).reshape(T, Hh * D)
    assert rel_l2(got[:, :Hh * D], want) < 1e-5
    np.testing.assert_array_equal(got[:, Hh * D:], 7.0)  # columns past H*D untouched


# ---------------------------------------------------------------- 16, 17
@pytest.mark.parametrize("T", [5, 11, 12, 40, 130])
def test_banded_attention_equals_relpos_composition(ctx, T):
    """The banded ops against the reference's two-matmul numpy form
    scores = qs k^T + rel_to_abs(qs used_k^T), ctx = p v + abs_to_rel(p) used_v
    (runtime/models/vits.py:994-1016) with used = get_relative_embeddings
    (window 10; T <= 11 slices, T > 11 pads)."""
    rng = np.random.default_rng(T)
    Hh, D = 2, 96
    C = Hh * D
    q, k, v = _r(rng, T, C), _r(rng, T, C), _r(rng, T, C)
    emb_k, emb_v = _r(rng, 1, 21, D, scale=0.5), _r(rng, 1, 21, D, scale=0.5)
    used_k = np.ascontiguousarray(V.get_relative_embeddings(emb_k, T, 10)[0])
    used_v = np.ascontiguousarray(V.get_relative_embeddings(emb_v, T, 10)[0])
    assert used_k.shape == (2 * T - 1, D)
    qh = q.reshape(T, Hh, D).transpose(1, 0, 2)[None]
    kh = k.reshape(T, Hh, D).transpose(1, 0, 2)[None]
    vh = v.reshape(T, Hh, D).transpose(1, 0, 2)[None]
    want_s = np.matmul(qh, np.ascontiguousarray(kh.swapaxes(-1, -2))) + \
        V.relative_to_absolute(np.matmul(qh, np.ascontiguousarray(used_k.T)))
    qi, ki, vi, uki, uvi = (ctx.upload(a) for a in (q, k, v, used_k, used_v))
    si = ctx.alloc(Hh * T * T)
    r = Rec(ctx)
    r.add(16, qi, ki, uki, Hh, T, D, C, 0, 0, 0, 0, 0, si)
    r.commit()
    s = ctx.download(si, (Hh, T, T))
    assert rel_l2(s, want_s[0]) < 1e-5
    p = nn.softmax(want_s.astype(np.float32), axis=-1)
    want_o = np.matmul(p, vh) + np.matmul(V.absolute_to_relative(p), used_v)
    want_o = want_o[0].transpose(1, 0, 2).reshape(T, C)
    pi, oi = ctx.upload(np.ascontiguousarray(p[0])), ctx.alloc(T * C)
    r = Rec(ctx)
    r.add(17, pi, vi, uvi, Hh, T, D, C, 0, 0, 0, 0, 0, oi)
    r.commit()
    assert rel_l2(ctx.download(oi, (T, C)), want_o) < 1e-5


# ---------------------------------------------------------------- 15, rmsnorm
@pytest.mark.parametrize("G,Cpg,S", [(512, 1, 3999), (4, 3, 50), (1, 7, 1)])
def test_group_norm(ctx, G, Cpg, S):
    rng = np.random.default_rng(G + S)
    x = _r(rng, 1, G * Cpg, S, scale=3.0) + 1.5
    g, b = _r(rng, G * Cpg), _r(rng, G * Cpg)
    xi, gi, bi, oi = ctx.upload(x), ctx.upload(g), ctx.upload(b), ctx.alloc(x.size)
    r = Rec(ctx)
    r.add(15, xi, gi, bi, G, Cpg, S, bits(1e-5), 0, 0, 0, 0, 0, oi)
    r.commit()
    want = H.group_norm(x.astype(np.float64), g, b, G)
    assert rel_l2(ctx.download(oi, x.shape), want) < 1e-5


def test_rmsnorm(ctx):
    from rvc_hip import hip_ops

    rng = np.random.default_rng(3)
    x, g = _r(rng, 33, 768, scale=2.0), _r(rng, 768)
    got = hip_ops.rmsnorm(x, g, eps=1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6) * g
    assert rel_l2(got, want) < 1e-6
    with pytest.raises(ValueError):
        hip_ops.rmsnorm(x, g[:5])


# ---------------------------------------------------------------- segments
def test_elementwise_segments(ctx):
    rng = np.random.default_rng(4)
    a, b = _r(rng, 4000), _r(rng, 4000)
    ids = {n: ctx.upload(a) for n in ("add", "mul", "leaky", "gelu", "copy")}
    bi = ctx.upload(b)
    r = Rec(ctx)
    r.call("rvc_batch_add_add_seg", ids["add"], bi, 1000, 100, 2000)
    r.call("rvc_batch_add_mul_seg", ids["mul"], bi, 999, 3001, 7)
    r.call("rvc_batch_add_leaky_seg", ids["leaky"], 1500, 17, bits(0.1))
    r.call("rvc_batch_add_gelu_seg", ids["gelu"], 333, 3667)
    r.call("rvc_batch_add_copy_seg", ids["copy"], bi, 64, 0, 3936)
    r.commit()
    exp = {n: a.copy() for n in ids}
    exp["add"][100:1100] = a[100:1100] + b[2000:3000]
    exp["mul"][3001:4000] = a[3001:4000] * b[7:1006]
    seg = a[17:1517]
    exp["leaky"][17:1517] = np.where(seg >= 0, seg, np.float32(0.1) * seg)
    exp["copy"][0:64] = b[3936:4000]
    for n in ("add", "mul", "leaky", "copy"):
        np.testing.assert_array_equal(ctx.download(ids[n], a.shape), exp[n], err_msg=n)
    got = ctx.download(ids["gelu"], a.shape)
    np.testing.assert_array_equal(got[:3667], a[:3667])
    assert np.abs(got[3667:] - H.gelu_erf(a[3667:])).max() < 1e-5
    # a segment past the buffer end is rejected when recorded
    L = ctx._lib
    assert L.rvc_batch_begin(ctx.handle) == 0
    assert L.rvc_batch_add_add_seg(ctx.handle, bi, bi, 100, 3950, 0) == -1
    assert L.rvc_batch_discard(ctx.handle) == 0


@pytest.mark.parametrize("B,Ci,Co,T,K,s,pad,d,cuts", [
    (1, 64, 64, 1000, 7, 1, 9, 3, (0, 300, 700, 1000)),
    (2, 32, 48, 517, 3, 2, 1, 1, (0, 1, 100, 259)),
    (1, 2, 5, 301, 5, 3, 2, 1, (0, 50, 101)),     # stride 3: direct kernel
])
def test_conv1d_segments_assemble_the_full_conv(ctx, B, Ci, Co, T, K, s, pad, d, cuts):
    rng = np.random.default_rng(T + K)
    x, w, b = _r(rng, B, Ci, T), _r(rng, Co, Ci, K, scale=1 / np.sqrt(Ci * K)), _r(rng, Co)
    full = nn.conv1d(x, w, b, stride=s, padding=pad, dilation=d)
    Lo = full.shape[-1]
    assert cuts[-1] == Lo
    xi, wi, bi = ctx.upload(x), ctx.upload(w), ctx.upload(b)
    oi = ctx.upload(np.zeros((B, Co, Lo), np.float32))
    fi = ctx.alloc(full.size)
    r = Rec(ctx)
    r.add(2, xi, wi, bi, B, Ci, T, Co, K, s, pad, pad, d, fi)
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        r.call("rvc_batch_add_conv1d_seg", xi, wi, bi, B, Ci, T, Co, K, s, pad, pad, d, oi, hi - lo, lo, Lo)
    r.commit()
    whole = ctx.download(fi, full.shape)
    segs = ctx.download(oi, full.shape)
    assert rel_l2(whole, full) < 1e-4
    assert np.abs(segs - whole).max() <= 1e-6 * np.abs(whole).max()
    # asymmetric padding is rejected at record time
    L = ctx._lib
    assert L.rvc_batch_begin(ctx.handle) == 0
    assert L.rvc_batch_add_conv1d_seg(ctx.handle, xi, wi, bi, B, Ci, T, Co, K, s, pad, pad + 1, d, oi,
                                      1, 0, Lo) == -1
    assert L.rvc_batch_discard(ctx.handle) == 0


def _convt_windows(L, K, s, p, d, lo, hi):
    """The exact input range feeding output columns [lo, hi)."""
    i_min = max(0, -(-(lo + p - (K - 1) * d) // s))
    i_max = min(L - 1, (hi - 1 + p) // s)
    i_min = min(i_min, L - 1)
    return i_min, max(1, i_max - i_min + 1)


@pytest.mark.parametrize("B,Ci,Co,L,K,s,p,op,d,cuts", [
    (1, 64, 32, 50, 16, 10, 3, 0, 1, (0, 123, 124, 400, 500)),
    (2, 16, 8, 40, 4, 2, 1, 0, 1, (0, 33, 80)),
    (1, 3, 5, 20, 3, 2, 1, 1, 2, (0, 7, 30, 42)),   # dilation 2: gather kernel
])
def test_conv_t1d_segments_assemble_the_full_conv(ctx, B, Ci, Co, L, K, s, p, op, d, cuts):
    rng = np.random.default_rng(L * K)
    x, w, b = _r(rng, B, Ci, L), _r(rng, Ci, Co, K, scale=1 / np.sqrt(Ci)), _r(rng, Co)
    full = nn.conv_transpose1d(x, w, b, stride=s, padding=p, output_padding=op, dilation=d)
    Lo = full.shape[-1]
    assert cuts[-1] == Lo
    xi, wi, bi = ctx.upload(x), ctx.upload(w), ctx.upload(b)
    oi = ctx.upload(np.zeros(full.shape, np.float32))
    r = Rec(ctx)
    for lo, hi in zip(cuts[:-1], cuts[1:]):
        i0, n = _convt_windows(L, K, s, p, d, lo, hi)
        r.call("rvc_batch_add_conv_t1d_seg", xi, wi, bi, B, Ci, L, Co, K, s, p, op, d, oi,
               hi - lo, n, i0, lo, Lo, -1, -1, -1, -1)
    r.commit()
    assert rel_l2(ctx.download(oi, full.shape), full) < 1e-4


def test_conv_t1d_segment_window_and_views(ctx):
    """Only input columns inside [in_off, in_off + l_in_seg) contribute; the
    byte-offset views shift x / out (engine/src/engine.zig:2430-2468)."""
    rng = np.random.default_rng(11)
    B, Ci, Co, L, K, s, p = 1, 8, 4, 60, 16, 10, 3
    x, w, b = _r(rng, B, Ci, L), _r(rng, Ci, Co, K), _r(rng, Co)
    Lo = (L - 1) * s - 2 * p + (K - 1) + 1
    in_off, n_in, lo, n_out = 10, 20, 100, 200
    xw = x.copy()
    xw[:, :, :in_off] = 0
    xw[:, :, in_off + n_in:] = 0
    want = nn.conv_transpose1d(xw, w, b, stride=s, padding=p)[:, :, lo:lo + n_out]
    pre_x, pre_o = 7, 5
    xi = ctx.upload(np.concatenate([np.full(pre_x, 99, np.float32), x.ravel()]))
    wi, bi = ctx.upload(w), ctx.upload(b)
    oi = ctx.upload(np.zeros(pre_o + B * Co * Lo, np.float32))
    r = Rec(ctx)
    r.call("rvc_batch_add_conv_t1d_seg", xi, wi, bi, B, Ci, L, Co, K, s, p, 0, 1, oi,
           n_out, n_in, in_off, lo, Lo, 4 * pre_x, -1, -1, 4 * pre_o)
    r.commit()
    got = ctx.download(oi, (pre_o + B * Co * Lo,))
    np.testing.assert_array_equal(got[:pre_o], 0)
    got = got[pre_o:].reshape(B, Co, Lo)
    assert rel_l2(got[:, :, lo:lo + n_out], want) < 1e-5
    np.testing.assert_array_equal(got[:, :, :lo], 0)
    np.testing.assert_array_equal(got[:, :, lo + n_out:], 0)
    # a window past the input row, or a view offset that is not a float multiple, is rejected
    Lb = ctx._lib
    assert Lb.rvc_batch_begin(ctx.handle) == 0
    assert Lb.rvc_batch_add_conv_t1d_seg(ctx.handle, xi, wi, bi, B, Ci, L, Co, K, s, p, 0, 1, oi,
                                         n_out, 60, in_off, lo, Lo, -1, -1, -1, -1) == -1
    assert Lb.rvc_batch_add_conv_t1d_seg(ctx.handle, xi, wi, bi, B, Ci, L, Co, K, s, p, 0, 1, oi,
                                         n_out, n_in, in_off, lo, Lo, 6, -1, -1, -1) == -1
    assert Lb.rvc_batch_discard(ctx.handle) == 0


# ---------------------------------------------------------------- record checks
def test_batch_records_are_checked_when_added(ctx):
    from rvc_hip import _hip

    L = ctx._lib
    small, big = ctx.alloc(10), ctx.alloc(1000)
    assert L.rvc_batch_begin(ctx.handle) == 0
    assert L.rvc_batch_add(ctx.handle, 3, small, big, 0, 100, *([0] * 10)) == -1
    assert "holds 10 floats" in _hip.last_error()
    assert L.rvc_batch_add(ctx.handle, 20, big, big, big, *([1] * 11)) == -1
    assert "invalid batch op code 20" in _hip.last_error()
    assert L.rvc_batch_add(ctx.handle, 16, big, big, 0, 2, 4, 2, 4, *([0] * 7)) == -1  # no relative table
    assert L.rvc_batch_add(ctx.handle, 12, big, big, big, 2, 4, 3, 5, *([0] * 7)) == -1  # H*D > C
    assert L.rvc_batch_commit(ctx.handle) == 0  # nothing was recorded


# ---------------------------------------------------------------- transfers / stats
def test_batched_transfers(ctx):
    L = ctx._lib
    rng = np.random.default_rng(6)
    arrs = [_r(rng, n) for n in (1, 100, 4097)]
    ids = [ctx.alloc(a.size) for a in arrs]
    n = len(arrs)
    sizes = (ctypes.c_int64 * n)(*[a.size for a in arrs])
    datas = (F32P * n)(*[a.ctypes.data_as(F32P) for a in arrs])
    idv = (ctypes.c_int64 * n)(*ids)
    assert L.rvc_mem_upload_to_batch(ctx.handle, n, sizes, datas, idv) == 0
    outs = [np.zeros_like(a) for a in arrs]
    U8P = ctypes.POINTER(ctypes.c_uint8)
    dsts = (U8P * n)(*[o.ctypes.data_as(U8P) for o in outs])
    assert L.rvc_mem_download_batch(ctx.handle, idv, dsts, sizes, n) == 0
    for a, o in zip(arrs, outs):
        np.testing.assert_array_equal(a, o)
    bad = (ctypes.c_int64 * n)(1, 100, 5000)
    assert L.rvc_mem_upload_to_batch(ctx.handle, n, bad, datas, idv) == -1


def test_mem_stats_top_and_probe(ctx):
    L = ctx._lib
    a, b = ctx.alloc(1 << 20), ctx.alloc(123)
    outs = [ctypes.c_int64() for _ in range(11)]
    assert L.rvc_mem_stats(ctx.handle, *[ctypes.byref(o) for o in outs]) == 0
    v = [o.value for o in outs]
    assert v[4] >= 2 and v[5] >= 4 * ((1 << 20) + 123) and v[9] >= 4 << 20
    assert v[8] >= v[5] and v[0] == v[1] == v[2] == v[3] == v[10] == 0
    top = (ctypes.c_int64 * 6)()
    cnt = L.rvc_mem_top(ctx.handle, 2, top)
    assert cnt == 2 and top[0] >= top[3] and top[0] == v[9]
    buf = ctypes.create_string_buffer(256)
    assert L.rvc_probe_extensions(ctx.handle, buf, 256) == 0
    assert b"arch=gfx950" in buf.value and buf.value.startswith(b"shaderFloat16=1")
    assert L.rvc_probe_extensions(ctx.handle, buf, 8) == -1
    busy, subs = ctypes.c_int64(-1), ctypes.c_int64(-1)
    assert L.rvc_ts_stats(ctx.handle, ctypes.byref(busy), ctypes.byref(subs)) == 0
    if os.environ.get("RVC_TS") != "1":
        assert busy.value == 0 and subs.value == 0
    ctx.free(a)
    ctx.free(b)


def test_ts_stats_with_rvc_ts(monkeypatch):
    from rvc_hip import _hip

    monkeypatch.setenv("RVC_TS", "1")
    L = _hip.get_lib()
    h = L.rvc_engine_create()
    assert h > 0, _hip.last_error()
    try:
        x = np.ones(1 << 22, np.float32)
        xi = ctypes.c_int64()
        assert L.rvc_mem_upload(h, x.ctypes.data_as(F32P), x.size, ctypes.byref(xi)) == 0
        for _ in range(3):
            assert L.rvc_relu(h, xi.value, x.size) == 0
        busy, subs = ctypes.c_int64(), ctypes.c_int64()
        assert L.rvc_ts_stats(h, ctypes.byref(busy), ctypes.byref(subs)) == 0
        assert subs.value == 3 and busy.value > 0
        assert L.rvc_ts_reset(h) == 0
        assert L.rvc_ts_stats(h, ctypes.byref(busy), ctypes.byref(subs)) == 0
        assert subs.value == 0 and busy.value == 0
    finally:
        assert L.rvc_engine_destroy(h) == 0
