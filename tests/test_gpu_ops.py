# -*- coding: utf-8 -*-
"""Op-level parity of the HIP backend against the numpy oracle (GPU).

Shapes follow the reference engine self-test (engine/test_ffi.py:506-586:
decoder conv1d / conv_t1d shapes) and BASELINE config 1; tolerance is the
self-test's relative L2 error < 1e-4 (engine/test_ffi.py:103-105)."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from oracle import loops
from oracle import nn_ref as nn

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ops():
    from rvc_hip import _hip, hip_ops

    assert _hip.has_so, _hip.so_load_error
    return hip_ops


def _r(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def test_mfma_gemm_layout(ops):
    # 1x1 conv = plain GEMM; a wrong accumulator/operand layout permutes rows/cols.
    rng = np.random.default_rng(0)
    x = _r(rng, 1, 2, 32)
    w = _r(rng, 32, 2, 1)
    got = ops.conv1d(x, w)
    want = loops.conv1d(x, w)
    assert rel_l2(got, want) < 1e-6


@pytest.mark.parametrize("B,C,O,T,K,pl,pr,d", [
    (1, 3, 4, 17, 3, 1, 1, 1),
    (2, 2, 3, 20, 5, 4, 4, 2),
    (1, 5, 70, 33, 7, 9, 9, 3),
    (1, 2, 2, 9, 3, 0, 1, 1),
    (3, 17, 33, 130, 11, 25, 25, 5),
])
def test_conv1d_small_vs_loops(ops, B, C, O, T, K, pl, pr, d):
    rng = np.random.default_rng(1)
    x, w, b = _r(rng, B, C, T), _r(rng, O, C, K), _r(rng, O)
    got = ops.conv1d(x, w, b, padding=(pl, pr), dilation=d)
    assert rel_l2(got, loops.conv1d(x, w, b, 1, pl, pr, d)) < TOL


@pytest.mark.parametrize("B,C,O,T", [
    (1, 192, 576, 1000),   # enc_p q/k/v at config 2
    (1, 192, 192, 1000),   # conv_o, flow res/skip
    (2, 96, 192, 37),      # flow pre, ragged length, batch 2
    (1, 192, 96, 1000),    # flow post (C_out not a multiple of 64)
    (1, 256, 48, 300),     # widest staged reduction, C_out not a multiple of 32
    (1, 24, 40, 4097),     # narrow reduction, one column past a tile edge
    (2, 256, 320, 4000),   # widest reduction on 64-column tiles (the largest LDS)
    (1, 40, 64, 2001),     # reduction rows and staging passes not whole batches
])
def test_conv1d_1x1_small_gemm(ops, B, C, O, T):
    """Plain 1x1 convs at a few thousand columns run the whole-reduction LDS
    kernel (C_in <= 256): against the oracle at rel L2 1e-4 and, on tiny
    slices, the float64 loops."""
    rng = np.random.default_rng(B * 1000 + C + O)
    x, w, b = _r(rng, B, C, T), _r(rng, O, C, 1, scale=C ** -0.5), _r(rng, O)
    got = ops.conv1d(x, w, b)
    assert got.shape == (B, O, T)
    assert rel_l2(got, nn.conv1d(x, w, b)) < TOL
    sl = loops.conv1d(x[:, :, :7], w, b)
    assert rel_l2(got[:, :, :7], sl) < TOL


@pytest.mark.parametrize("B,C,O,T,K,pad", [
    (1, 192, 768, 1000, 3, 1),   # enc_p FFN input conv at config 2
    (1, 768, 192, 1000, 3, 1),   # FFN output conv (128-channel chunks)
    (2, 192, 384, 1000, 5, 2),   # flow WaveNet in-layer shape, batch 2
    (1, 192, 384, 37, 5, 2),     # ragged length, one column tile
    (1, 64, 32, 300, 3, (2, 0)), # left padding only
    (1, 128, 100, 777, 5, 2),    # C_out not a multiple of 32
    (1, 512, 256, 130, 3, 1),    # 128-channel chunks at the smallest C_in
    (1, 192, 512, 1000, 7, 3),   # decoder conv_pre at config 2
    (2, 192, 512, 37, 7, 3),     # conv_pre, ragged short chunks, batch 2
    (1, 768, 192, 1000, 1, 0),   # enc_p phone embedding
    (2, 768, 2304, 499, 1, 0),   # HuBERT qkv at 10 s, batch 2
    (1, 3072, 768, 499, 1, 0),   # HuBERT FFN output
])
def test_conv1d_small_chunked(ops, B, C, O, T, K, pad):
    """K = 3 / 5 / 7 convs and wide 1x1 GEMMs on short sequences run the chunked
    whole-reduction kernel (no split-K): against the oracle at rel L2 1e-4,
    the first columns also against the float64 loops."""
    rng = np.random.default_rng(B * 7 + C + O + T)
    x, w, b = _r(rng, B, C, T), _r(rng, O, C, K, scale=(C * K) ** -0.5), _r(rng, O)
    got = ops.conv1d(x, w, b, padding=pad)
    pl, pr = (pad, pad) if isinstance(pad, int) else pad
    assert got.shape == (B, O, T + pl + pr - K + 1)
    assert rel_l2(got, nn.conv1d(x, w, b, 1, (pl, pr))) < TOL
    sl = loops.conv1d(x[:, :, :9], w, b, 1, pl, 0)
    assert rel_l2(got[:, :, :sl.shape[-1]], sl) < TOL


RESBLOCK = [(C, L, k, d) for C, L in ((256, 1024), (128, 2048), (64, 4096), (32, 8192))
            for k in (3, 7, 11) for d in (1, 3, 5)]


@pytest.mark.parametrize("C,L,k,d", RESBLOCK)
def test_conv1d_resblock_shapes(ops, C, L, k, d):
    rng = np.random.default_rng(C * 100 + k * 10 + d)
    x = _r(rng, 1, C, L)
    w = _r(rng, C, C, k, scale=1.0 / np.sqrt(C * k))
    b = _r(rng, C, scale=0.1)
    pad = (k * d - d) // 2
    got = ops.conv1d(x, w, b, padding=pad, dilation=d)
    assert rel_l2(got, nn.conv1d(x, w, b, padding=pad, dilation=d)) < TOL


@pytest.mark.parametrize("C,L,k,d", [(256, 30000, 3, 1), (128, 120000, 3, 3), (64, 240000, 3, 1),
                                     (32, 500000, 3, 5), (128, 240000, 3, 5)])
def test_conv1d_persistent_tiles(ops, C, L, k, d):
    """Grids large enough for the persistent MFMA kernel (32 x 256, 64 x 256,
    128 x 256 and 32 x 512 tiles, buffer-resource staging with out-of-range
    padding)."""
    print(f"persistent conv C={C} L={L} k={k} d={d}", flush=True)
    rng = np.random.default_rng(C + L)
    x = _r(rng, 1, C, L)
    w = _r(rng, C, C, k, scale=1.0 / np.sqrt(C * k))
    b = _r(rng, C, scale=0.1)
    pad = (k * d - d) // 2
    got = ops.conv1d(x, w, b, padding=pad, dilation=d)
    assert rel_l2(got, nn.conv1d(x, w, b, padding=pad, dilation=d)) < TOL


def test_conv1d_persistent_widest_halo(ops):
    """The persistent 64 x 256 tile at decoder stage 1's widest ResBlock conv
    (C = 128, k = 11, d = 5: a 306-sample staged row per channel), checked
    against torch's fp32 CPU conv1d (the numpy oracle needs about a minute
    for these 86 GFLOP)."""
    import torch

    C, L, k, d = 128, 240000, 11, 5
    print(f"persistent conv C={C} L={L} k={k} d={d}", flush=True)
    rng = np.random.default_rng(17)
    x = _r(rng, 1, C, L)
    w = _r(rng, C, C, k, scale=1.0 / np.sqrt(C * k))
    b = _r(rng, C, scale=0.1)
    pad = (k * d - d) // 2
    got = ops.conv1d(x, w, b, padding=pad, dilation=d)
    want = torch.nn.functional.conv1d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b), padding=pad,
                                      dilation=d).numpy()
    assert rel_l2(got, want) < TOL


@pytest.mark.parametrize("C_in,C_out,L,K", [(192, 512, 200, 7), (192, 768, 300, 3), (768, 192, 300, 3),
                                            (192, 384, 257, 5), (192, 576, 1000, 1)])
def test_conv1d_encoder_flow_shapes(ops, C_in, C_out, L, K):
    rng = np.random.default_rng(5)
    x, w, b = _r(rng, 1, C_in, L), _r(rng, C_out, C_in, K, scale=0.05), _r(rng, C_out)
    got = ops.conv1d(x, w, b, padding=(K - 1) // 2)
    assert rel_l2(got, nn.conv1d(x, w, b, padding=(K - 1) // 2)) < TOL


@pytest.mark.parametrize("C_out,k,s,B,L", [
    (256, 80, 40, 1, 64 * 40), (128, 8, 4, 1, 64 * 40), (64, 4, 2, 1, 64 * 40), (32, 1, 1, 1, 64 * 40),
    (256, 80, 40, 2, 1000 * 40 + 17),  # config-2 stage 0, batch 2, a ragged last tile
    (20, 7, 3, 1, 3001),               # channels and taps not multiples of the tile
    (256, 64, 32, 1, 777 * 32),        # 32 kHz stage 0
])
def test_conv1d_noise_conv_shapes(ops, C_out, k, s, B, L):
    """Single-input-channel strided convs (the NSF noise convs) against the
    oracle at rel L2 1e-4."""
    rng = np.random.default_rng(6)
    x, w, b = _r(rng, B, 1, L), _r(rng, C_out, 1, k), _r(rng, C_out)
    got = ops.conv1d(x, w, b, stride=s, padding=s // 2)
    assert rel_l2(got, nn.conv1d(x, w, b, stride=s, padding=s // 2)) < TOL


@pytest.mark.parametrize("B,C,O,T,K,pl,pr,d", [
    (1, 5, 70, 33, 3, 0, 0, 1),
    (2, 17, 64, 200, 2, 0, 0, 1),
    (1, 3, 40, 57, 5, 2, 1, 2),
])
def test_conv1d_stride2_small_vs_loops(ops, B, C, O, T, K, pl, pr, d):
    """Stride-2 convolutions run on the MFMA kernel's strided variant."""
    rng = np.random.default_rng(9)
    x, w, b = _r(rng, B, C, T), _r(rng, O, C, K), _r(rng, O)
    got = ops.conv1d(x, w, b, stride=2, padding=(pl, pr), dilation=d)
    assert rel_l2(got, loops.conv1d(x, w, b, 2, pl, pr, d)) < TOL


@pytest.mark.parametrize("T,K", [(2001, 3), (999, 2)])
def test_conv1d_hubert_feature_shapes(ops, T, K):
    """HuBERT feature-extractor layers: 512 -> 512, valid, stride 2."""
    rng = np.random.default_rng(10)
    x, w = _r(rng, 1, 512, T), _r(rng, 512, 512, K, scale=(2.0 / (512 * K)) ** 0.5)
    got = ops.conv1d(x, w, None, stride=2)
    assert rel_l2(got, nn.conv1d(x, w, None, stride=2)) < TOL


@pytest.mark.parametrize("C_in,C_out,L,K,s,p,op,d", [
    (512, 256, 50, 16, 10, 3, 0, 1),
    (256, 128, 200, 16, 10, 3, 0, 1),
    (128, 64, 500, 4, 2, 1, 0, 1),
    (64, 32, 1000, 4, 2, 1, 0, 1),
    (512, 256, 30, 24, 12, 6, 0, 1),
    (256, 128, 60, 20, 10, 5, 0, 1),
    (5, 7, 13, 3, 2, 0, 1, 1),
    (4, 6, 11, 3, 2, 1, 1, 2),
])
def test_conv_transpose1d_shapes(ops, C_in, C_out, L, K, s, p, op, d):
    rng = np.random.default_rng(7)
    x, w, b = _r(rng, 1, C_in, L), _r(rng, C_in, C_out, K, scale=0.05), _r(rng, C_out)
    got = ops.conv_transpose1d(x, w, b, stride=s, padding=p, output_padding=op, dilation=d)
    want = nn.conv_transpose1d(x, w, b, stride=s, padding=p, output_padding=op, dilation=d)
    assert got.shape == want.shape
    assert rel_l2(got, want) < TOL


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (3, 5, 7), (64, 768, 768), (1000, 768, 192), (1188, 64, 1188)])
def test_matmul(ops, M, K, N):
    rng = np.random.default_rng(8)
    a, b = _r(rng, M, K), _r(rng, K, N)
    assert rel_l2(ops.matmul(a, b), a.astype(np.float64) @ b) < TOL


def test_layer_norm_softmax(ops):
    rng = np.random.default_rng(9)
    x, g, b = _r(rng, 1000, 192), _r(rng, 192), _r(rng, 192)
    assert rel_l2(ops.layer_norm(x, g, b), nn.layer_norm(x, g, b)) < TOL
    s = _r(rng, 2, 300, 1000, scale=3.0)
    got = ops.softmax(s)
    assert rel_l2(got, nn.softmax(s)) < TOL
    np.testing.assert_allclose(got.sum(-1), 1.0, rtol=1e-5)


def test_elementwise_and_embedding(ops):
    rng = np.random.default_rng(10)
    a, b = _r(rng, 3, 1000), _r(rng, 3, 1000)
    a0 = a.copy()
    np.testing.assert_array_equal(ops.add(a, b), a + b)
    np.testing.assert_array_equal(ops.mul(a, b), a * b)
    np.testing.assert_array_equal(ops.add_inplace(a, b), a + b)
    np.testing.assert_array_equal(ops.mul_inplace(a, b), a * b)
    np.testing.assert_array_equal(ops.relu(a), np.maximum(a, 0))
    np.testing.assert_array_equal(ops.leaky_relu(a, 0.1), nn.leaky_relu(a, 0.1))
    np.testing.assert_array_equal(a, a0)  # inputs never mutated
    table = _r(rng, 256, 192)
    ids = rng.integers(-256, 256, size=(1, 1000))
    np.testing.assert_array_equal(ops.embedding(ids, table), nn.embedding(ids, table))


def test_error_paths(ops):
    rng = np.random.default_rng(11)
    with pytest.raises(ValueError):
        ops.conv1d(_r(rng, 1, 3, 10), _r(rng, 4, 2, 3))
    with pytest.raises(ValueError):
        ops.conv1d(_r(rng, 1, 3, 10), _r(rng, 4, 3, 3), stride=0)
    with pytest.raises(TypeError):
        ops.conv1d(np.ones((1, 3, 10), np.int32), _r(rng, 4, 3, 3))
    with pytest.raises(ValueError):
        ops.matmul(_r(rng, 3, 4), _r(rng, 5, 6))
    with pytest.raises(ValueError):
        ops.embedding(np.array([300]), _r(rng, 256, 4))
    assert ops.conv1d(_r(rng, 1, 3, 2), _r(rng, 4, 3, 5)).shape == (1, 4, 0)
    ctx = ops.get_context()
    with pytest.raises(RuntimeError, match="invalid buffer id"):
        ctx.download(987654321, (4,))


def test_persistent_weights_and_batch_api(ops):
    import ctypes

    from rvc_hip import _hip

    rng = np.random.default_rng(12)
    ctx = ops.get_context()
    x, w, b = _r(rng, 1, 64, 500), _r(rng, 32, 64, 3, scale=0.1), _r(rng, 32)
    pw, pb = ctx.persistent_upload(w), ctx.persistent_upload(b)
    got = ops.conv1d(x, w, b, padding=1, buf_w=pw, buf_b=pb)
    assert rel_l2(got, nn.conv1d(x, w, b, padding=1)) < TOL
    pw.free()
    pw.free()  # idempotent; a freed buffer falls back to uploading the array
    assert rel_l2(ops.conv1d(x, w, b, padding=1, buf_w=pw, buf_b=pb), got) == 0.0
    # record/commit: conv1d (op 2) then leaky (op 6) then copy (op 7), one commit
    L = _hip.get_lib()
    xi, wi, bi = ctx.upload(x), ctx.upload(w), ctx.upload(b)
    oi, ci = ctx.alloc(32 * 500), ctx.alloc(32 * 500)
    h = ctx.handle
    assert L.rvc_batch_begin(h) == 0
    assert L.rvc_batch_add(h, 2, xi, wi, bi, 1, 64, 500, 32, 3, 1, 1, 1, 1, oi, 0) == 0
    assert L.rvc_batch_add(h, 6, oi, 0, 0, 32 * 500, ops._f32_bits(0.1), 0, 0, 0, 0, 0, 0, 0, 0, 0) == 0
    assert L.rvc_batch_add(h, 7, ci, oi, 0, 32 * 500, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == 0
    assert L.rvc_batch_add(h, 99, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == -1
    assert "invalid batch op code" in _hip.last_error()
    assert L.rvc_batch_commit(h) == 0
    out = ctx.download(ci, (1, 32, 500))
    want = nn.leaky_relu(nn.conv1d(x, w, b, padding=1), 0.1)
    assert rel_l2(out, want) < TOL
    for i in (xi, wi, bi, oi, ci):
        ctx.free(i)
    with pytest.raises(RuntimeError, match="invalid buffer id"):
        ctx.free(xi)
    assert ctypes is not None
