# -*- coding: utf-8 -*-
"""rvc_conv1d_noalloc (the conv1d entry point that allocates nothing: its
packed weights live in a fixed per-GPU device array) against rvc_conv1d on
the same buffers, through the C ABI.  Same kernels and packed weights, so
the two agree bit for bit; the numpy oracle is checked too (rel L2 <= 1e-4).
Two calls in a row, the second smaller, show that the array's leftover
contents from the first call never leak into the second; a weight set larger
than the array is rejected with a message."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import rel_l2
from oracle import nn_ref as nn

pytestmark = pytest.mark.gpu

_I64 = ctypes.c_int64


@pytest.fixture(scope="module")
def ctx():
    from rvc_hip import _hip
    from rvc_hip.hip_ops import HipContext

    assert _hip.has_so, _hip.so_load_error
    c = HipContext()
    yield c
    c.close()


def _run_both(ctx, B, C_in, C_out, L, K, stride, pad_l, pad_r, dil, seed):
    from rvc_hip import _hip

    lib = _hip.get_lib()
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, C_in, L)).astype(np.float32)
    w = (rng.standard_normal((C_out, C_in, K)) / np.sqrt(C_in * K)).astype(np.float32)
    b = rng.standard_normal(C_out).astype(np.float32)
    n_out = (L + pad_l + pad_r - dil * (K - 1) - 1) // stride + 1
    xi, wi, bi = ctx.upload(x), ctx.upload(w), ctx.upload(b)
    o1, o2 = ctx.alloc(B * C_out * n_out), ctx.alloc(B * C_out * n_out)
    try:
        args = [B, C_in, L, C_out, K, stride, pad_l, pad_r, dil]
        _hip._check(lib.rvc_conv1d(ctx.handle, xi, wi, bi, o1, *args), "rvc_conv1d")
        _hip._check(lib.rvc_conv1d_noalloc(ctx.handle, xi, wi, bi, o2, *args), "rvc_conv1d_noalloc")
        ref = ctx.download(o1, (B, C_out, n_out))
        got = ctx.download(o2, (B, C_out, n_out))
    finally:
        for buf in (xi, wi, bi, o1, o2):
            ctx.free(buf)
    return x, w, b, ref, got


def test_noalloc_matches_conv1d_twice_second_smaller(ctx):
    # first call: a decoder-stage ResBlock conv (114 688 packed weight floats)
    cases = [(2, 128, 128, 3000, 7, 1, 9, 9, 3, 1),
             # second call, smaller: C_out = 30 leaves pad columns in the packed rows
             (1, 32, 30, 517, 3, 1, 1, 1, 1, 2)]
    for B, C_in, C_out, L, K, s, pl, pr, d, seed in cases:
        x, w, b, ref, got = _run_both(ctx, B, C_in, C_out, L, K, s, pl, pr, d, seed)
        np.testing.assert_array_equal(got, ref)
        assert rel_l2(got, nn.conv1d(x, w, b, stride=s, padding=(pl, pr), dilation=d)) < 1e-4


def test_noalloc_strided_and_direct_paths(ctx):
    # stride 2 (MFMA path with packed weights) and stride 4 (direct kernel, no scratch)
    for B, C_in, C_out, L, K, s, pl, pr, d in [(1, 64, 96, 801, 3, 2, 1, 1, 1), (1, 1, 16, 400, 8, 4, 2, 2, 1)]:
        x, w, b, ref, got = _run_both(ctx, B, C_in, C_out, L, K, s, pl, pr, d, 7)
        np.testing.assert_array_equal(got, ref)
        assert rel_l2(got, nn.conv1d(x, w, b, stride=s, padding=(pl, pr), dilation=d)) < 1e-4


def test_noalloc_rejects_weights_beyond_the_array(ctx):
    from rvc_hip import _hip

    lib = _hip.get_lib()
    B, C, L, K = 1, 512, 64, 5  # 512 * 512 * 5 floats > 1 Mi
    xi, wi = ctx.upload(np.zeros((B, C, L), np.float32)), ctx.upload(np.zeros((C, C, K), np.float32))
    o = ctx.alloc(B * C * L)
    try:
        rc = lib.rvc_conv1d_noalloc(ctx.handle, xi, wi, 0, o, B, C, L, C, K, 1, 2, 2, 1)
        assert rc == -1
        assert "fixed scratch holds 1048576" in _hip.last_error()
        # the same call through the allocating entry point still works
        _hip._check(lib.rvc_conv1d(ctx.handle, xi, wi, 0, o, B, C, L, C, K, 1, 2, 2, 1), "rvc_conv1d")
    finally:
        for buf in (xi, wi, o):
            ctx.free(buf)
