# -*- coding: utf-8 -*-
"""Op-level HIP backend: the ``runtime/vulkan_ops.py`` op surface on MI355X.

Module-level functions carry the names and signatures the reference's
dispatcher calls (``runtime/backend.py:205-316``): ``matmul``, ``add``,
``mul``, ``relu``, ``conv1d``, ``conv_transpose1d``, ``embedding``,
``add_inplace``, ``mul_inplace``, ``layer_norm``, ``softmax``.  Register this
module as the ``hip`` backend with ``rvc_hip.backend_hip.register_op_backend``
and ``RVC_BACKEND=hip`` routes ``runtime.nn`` float32 ops here.

Semantics follow ``VulkanContext`` (``runtime/vulkan_ops.py:978-1994``):
float32 numpy arrays in, NEW float32 arrays out, inputs never mutated (also
for ``*_inplace`` / ``relu``); float64 is downcast and other dtypes raise
``TypeError``; bad shapes / parameters raise ``ValueError``; ``buf_*``
arguments take a resident ``PersistentBuffer`` and skip that upload.

One deliberate difference: there is no host shortcut for small tensors (the
reference computes < 1024-element inputs with numpy, ``runtime/vulkan_ops.py
:115``).  Every call here runs on the GPU, so results never silently come
from a CPU path.

Observability as in the reference: ``stats_reset()`` / ``stats_snapshot()``
count host->device uploads and device->host downloads with their bytes
(``runtime/vulkan_ops.py:139-150, 225-249``; every upload of an op argument,
``persistent_upload`` and ``PersistentBuffer.update`` counts, as does every
result download), and ``RVC_PROFILE=1`` times each module-level op into the
table of ``rvc_hip.profiler`` under ``"<op>/gpu"``.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np

from . import _hip
from . import profiler

__all__ = [
    "stats_reset",
    "stats_snapshot",
    "HipContext",
    "PersistentBuffer",
    "get_context",
    "matmul",
    "add",
    "mul",
    "relu",
    "conv1d",
    "conv_transpose1d",
    "embedding",
    "add_inplace",
    "mul_inplace",
    "layer_norm",
    "softmax",
    "rmsnorm",
    "leaky_relu",
]

_F32P = ctypes.POINTER(ctypes.c_float)

# ------------------------------------------------------------------ transfer counters
_stats_lock = threading.Lock()
_stats = {"uploads": 0, "downloads": 0, "upload_bytes": 0, "download_bytes": 0}


def stats_reset() -> None:
    """Zero the upload / download counters."""
    with _stats_lock:
        for k in _stats:
            _stats[k] = 0


def stats_snapshot() -> dict:
    """{"uploads", "downloads", "upload_bytes", "download_bytes"} since the
    last reset (process-wide, every context)."""
    with _stats_lock:
        return dict(_stats)


def _count(kind: str, nbytes: int) -> None:
    with _stats_lock:
        _stats[kind + "s"] += 1
        _stats[kind + "_bytes"] += int(nbytes)


def _traced(name: str):
    """Time the wrapped op under ``name`` when ``RVC_PROFILE`` is on (the
    reference's ``traced``, ``runtime/vulkan_ops.py:35-48``)."""

    def deco(fn):
        def wrap(*args, **kwargs):
            if not profiler.enabled():
                return fn(*args, **kwargs)
            with profiler.profile_op(name):
                return fn(*args, **kwargs)

        wrap.__name__ = fn.__name__
        wrap.__qualname__ = fn.__qualname__
        wrap.__doc__ = fn.__doc__
        wrap.__wrapped__ = fn
        return wrap

    return deco


def _f32_bits(v: float) -> int:
    """float32 bit pattern as a signed int64 (``runtime/vulkan_ops.py:255-261``)."""
    return int(np.float32(v).view(np.int32))


def _as_f32(a, name: str) -> np.ndarray:
    a = np.asarray(a)
    if not np.issubdtype(a.dtype, np.floating):
        raise TypeError(f"{name} must be a floating numpy array (float32; float64 is converted), "
                        f"got dtype={a.dtype}")
    if a.dtype != np.float32:
        a = a.astype(np.float32)
    return np.ascontiguousarray(a)


def _pads(padding):
    if isinstance(padding, (tuple, list)):
        return int(padding[0]), int(padding[1])
    return int(padding), int(padding)


class PersistentBuffer:
    """A device buffer owned by the caller (resident weights).

    ``free()`` is idempotent; a freed buffer passed as ``buf_*`` is ignored
    and the op uploads the array instead (``runtime/vulkan_ops.py:282-361,
    500-510``).
    """

    __slots__ = ("_ctx", "_buf", "shape", "nbytes")

    def __init__(self, ctx, buf, shape, nbytes):
        self._ctx = ctx
        self._buf = int(buf)
        self.shape = tuple(shape)
        self.nbytes = int(nbytes)

    @property
    def id(self):
        return self._buf

    @property
    def valid(self) -> bool:
        return self._buf is not None

    def free(self) -> None:
        if self._buf is not None:
            buf, self._buf = self._buf, None
            try:
                self._ctx.free(buf)
            except RuntimeError:
                pass

    def update(self, a) -> None:
        a = _as_f32(a, "PersistentBuffer.update")
        if self._buf is None:
            raise RuntimeError("PersistentBuffer already freed")
        if a.size * 4 > self.nbytes:
            raise ValueError(f"PersistentBuffer.update: {a.size * 4} bytes > {self.nbytes}")
        _count("upload", a.nbytes)
        _hip._check(self._ctx._lib.rvc_mem_upload_to(self._ctx.handle, a.ctypes.data_as(_F32P), a.size,
                                                     self._buf), "rvc_mem_upload_to")

    def __del__(self):
        try:
            import sys

            if not sys.is_finalizing():
                self.free()
        except Exception:  # noqa: BLE001
            pass

    def __repr__(self):
        return f"PersistentBuffer(shape={self.shape}, {'freed' if self._buf is None else f'buf={self._buf}'})"


def _resolve(pb):
    if pb is None:
        return None
    bid = getattr(pb, "id", None)
    return int(bid) if bid is not None else None


class HipContext:
    """One engine handle (device, stream, buffer registry) per process."""

    def __init__(self):
        self._lib = _hip.get_lib()
        self.handle = _hip.engine_create()
        self._lock = threading.RLock()

    # ---------------------------------------------------------------- memory
    def upload(self, a) -> int:
        a = np.ascontiguousarray(a)
        out = ctypes.c_int64(0)
        _count("upload", a.nbytes)
        with self._lock:
            _hip._check(self._lib.rvc_mem_upload_bytes(self.handle, a.ctypes.data_as(ctypes.c_void_p),
                                                       a.nbytes, ctypes.byref(out)), "rvc_mem_upload_bytes")
        return int(out.value)

    def alloc(self, n_floats: int) -> int:
        out = ctypes.c_int64(0)
        with self._lock:
            _hip._check(self._lib.rvc_mem_alloc(self.handle, max(int(n_floats), 1) * 4, ctypes.byref(out)),
                        "rvc_mem_alloc")
        return int(out.value)

    def persistent_upload(self, a) -> PersistentBuffer:
        a = _as_f32(a, "persistent_upload")
        return PersistentBuffer(self, self.upload(a), a.shape, a.nbytes)

    def download(self, buf: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _count("download", out.nbytes)
        with self._lock:
            _hip._check(self._lib.rvc_mem_download_bytes(self.handle, int(buf), out.ctypes.data_as(ctypes.c_void_p),
                                                         out.nbytes), "rvc_mem_download_bytes")
        return out

    def free(self, buf: int) -> None:
        with self._lock:
            _hip._check(self._lib.rvc_mem_free(self.handle, int(buf)), "rvc_mem_free")

    def close(self) -> None:
        if self.handle is not None:
            _hip.engine_destroy(self.handle)
            self.handle = None

    def _run(self, fn, temps):
        try:
            return fn()
        finally:
            for b in temps:
                try:
                    self.free(b)
                except RuntimeError:
                    pass

    def _in(self, arr, pb, temps):
        bid = _resolve(pb)
        if bid is None:
            bid = self.upload(arr)
            temps.append(bid)
        return bid

    def _out(self, n, temps):
        bid = self.alloc(n)
        temps.append(bid)
        return bid

    # ---------------------------------------------------------------- ops
    def matmul(self, a, b, buf_a=None, buf_b=None):
        a = _as_f32(a, "matmul a")
        b = _as_f32(b, "matmul b")
        if a.ndim != 2 or b.ndim != 2:
            raise ValueError(f"matmul needs 2-D inputs, got a.ndim={a.ndim} b.ndim={b.ndim}")
        M, K = a.shape
        K2, N = b.shape
        if K != K2:
            raise ValueError(f"matmul shape mismatch: a={a.shape} b={b.shape}")
        if M * N == 0:
            return np.zeros((M, N), dtype=np.float32)
        if K == 0:
            return np.zeros((M, N), dtype=np.float32)
        t = []

        def go():
            ai, bi = self._in(a, buf_a, t), self._in(b, buf_b, t)
            ci = self._out(M * N, t)
            with self._lock:
                _hip._check(self._lib.rvc_matmul(self.handle, ai, bi, ci, M, K, N), "rvc_matmul")
            return self.download(ci, (M, N))

        return self._run(go, t)

    def _binary(self, a, b, sym, name, buf_a=None, buf_b=None):
        a = _as_f32(a, f"{name} a")
        b = _as_f32(b, f"{name} b")
        if a.shape != b.shape:
            raise ValueError(f"{name} shape mismatch: a={a.shape} b={b.shape}")
        if a.size == 0:
            return np.empty(a.shape, dtype=np.float32)
        t = []

        def go():
            ai, bi = self._in(a, buf_a, t), self._in(b, buf_b, t)
            ci = self._out(a.size, t)
            with self._lock:
                _hip._check(getattr(self._lib, sym)(self.handle, ai, bi, ci, a.size), sym)
            return self.download(ci, a.shape)

        return self._run(go, t)

    def add(self, a, b, buf_a=None, buf_b=None):
        return self._binary(a, b, "rvc_add", "add", buf_a, buf_b)

    def mul(self, a, b, buf_a=None, buf_b=None):
        return self._binary(a, b, "rvc_mul", "mul", buf_a, buf_b)

    def add_inplace(self, a, b, buf_a=None, buf_b=None):
        """``a + b`` as a new array (the engine works on an uploaded copy)."""
        return self._binary(a, b, "rvc_add", "add_inplace", buf_a, buf_b)

    def mul_inplace(self, a, b, buf_a=None, buf_b=None):
        return self._binary(a, b, "rvc_mul", "mul_inplace", buf_a, buf_b)

    def _unary_inplace(self, a, name, call):
        a = _as_f32(a, name)
        if a.size == 0:
            return np.empty(a.shape, dtype=np.float32)
        t = []

        def go():
            ai = self.upload(a)
            t.append(ai)
            with self._lock:
                call(ai, a.size)
            return self.download(ai, a.shape)

        return self._run(go, t)

    def relu(self, a, buf_a=None):
        return self._unary_inplace(a, "relu", lambda i, n: _hip._check(self._lib.rvc_relu(self.handle, i, n),
                                                                        "rvc_relu"))

    relu_inplace = relu

    def leaky_relu(self, a, negative_slope=0.1):
        bits = _f32_bits(negative_slope)
        return self._unary_inplace(
            a, "leaky_relu", lambda i, n: _hip._check(self._lib.rvc_leaky_relu(self.handle, i, n, bits),
                                                      "rvc_leaky_relu"))

    def conv1d(self, x, w, b=None, stride=1, padding=0, dilation=1, buf_w=None, buf_b=None):
        x = _as_f32(x, "conv1d x")
        w = _as_f32(w, "conv1d w")
        if x.ndim != 3 or w.ndim != 3:
            raise ValueError(f"conv1d needs 3-D inputs, got x.ndim={x.ndim} w.ndim={w.ndim}")
        B, C_in, L = x.shape
        C_out, C_in2, K = w.shape
        if C_in != C_in2:
            raise ValueError(f"conv1d channel mismatch: x={x.shape} w={w.shape}")
        pad_l, pad_r = _pads(padding)
        stride, dilation = int(stride), int(dilation)
        if stride < 1 or dilation < 1 or pad_l < 0 or pad_r < 0 or K < 1:
            raise ValueError("conv1d: invalid parameters (stride/dilation >= 1, padding >= 0, K >= 1)")
        n_out = (L + pad_l + pad_r - dilation * (K - 1) - 1) // stride + 1
        if n_out <= 0:
            return np.zeros((B, C_out, 0), dtype=np.float32)
        if B == 0 or C_out == 0:
            return np.zeros((B, C_out, n_out), dtype=np.float32)
        bias = _as_f32(b, "conv1d b") if b is not None else None
        if bias is not None and bias.shape[0] != C_out:
            raise ValueError(f"conv1d bias length {bias.shape[0]} != C_out {C_out}")
        t = []

        def go():
            xi = self.upload(x)
            t.append(xi)
            wi = self._in(w, buf_w, t)
            bi = self._in(bias, buf_b, t) if bias is not None else 0
            oi = self._out(B * C_out * n_out, t)
            with self._lock:
                _hip._check(self._lib.rvc_conv1d(self.handle, xi, wi, bi, oi, B, C_in, L, C_out, K, stride,
                                                 pad_l, pad_r, dilation), "rvc_conv1d")
            return self.download(oi, (B, C_out, n_out))

        return self._run(go, t)

    def conv_transpose1d(self, x, w, b=None, stride=1, padding=0, output_padding=0, dilation=1,
                         buf_w=None, buf_b=None):
        x = _as_f32(x, "conv_transpose1d x")
        w = _as_f32(w, "conv_transpose1d w")
        if x.ndim != 3 or w.ndim != 3:
            raise ValueError(f"conv_transpose1d needs 3-D inputs, got x.ndim={x.ndim} w.ndim={w.ndim}")
        B, C_in, L = x.shape
        C_in2, C_out, K = w.shape
        if C_in != C_in2:
            raise ValueError(f"conv_transpose1d channel mismatch: x={x.shape} w={w.shape}")
        stride, padding = int(stride), int(padding)
        output_padding, dilation = int(output_padding), int(dilation)
        if stride < 1 or padding < 0 or output_padding < 0 or dilation < 1 or K < 1:
            raise ValueError("conv_transpose1d: invalid parameters "
                             "(stride/dilation >= 1, padding/output_padding >= 0)")
        n_out = (L - 1) * stride - 2 * padding + dilation * (K - 1) + output_padding + 1
        if n_out <= 0:
            return np.zeros((B, C_out, 0), dtype=np.float32)
        bias = _as_f32(b, "conv_transpose1d b") if b is not None else None
        if bias is not None and bias.shape[0] != C_out:
            raise ValueError(f"conv_transpose1d bias length {bias.shape[0]} != C_out {C_out}")
        if B == 0 or C_out == 0 or L == 0:
            out = np.zeros((B, C_out, n_out), dtype=np.float32)
            return out + bias.reshape(1, -1, 1) if bias is not None and L == 0 else out
        t = []

        def go():
            xi = self.upload(x)
            t.append(xi)
            wi = self._in(w, buf_w, t)
            bi = self._in(bias, buf_b, t) if bias is not None else 0
            oi = self._out(B * C_out * n_out, t)
            with self._lock:
                _hip._check(self._lib.rvc_conv_t1d(self.handle, xi, wi, bi, oi, B, C_in, L, C_out, K, stride,
                                                   padding, output_padding, dilation), "rvc_conv_t1d")
            return self.download(oi, (B, C_out, n_out))

        return self._run(go, t)

    def embedding(self, ids, table, buf_table=None):
        ids = np.asarray(ids)
        table = _as_f32(table, "embedding table")
        if table.ndim != 2:
            raise ValueError(f"embedding table must be 2-D, got ndim={table.ndim}")
        if not np.issubdtype(ids.dtype, np.integer):
            raise TypeError(f"embedding ids must be integers, got dtype={ids.dtype}")
        V, E = table.shape
        if ids.size == 0:
            return np.empty(ids.shape + (E,), dtype=np.float32)
        if int(ids.min()) < -V or int(ids.max()) >= V:
            raise ValueError(f"embedding ids out of range [-{V}, {V})")
        ids32 = np.ascontiguousarray(ids, dtype=np.int32)
        t = []

        def go():
            ii = self.upload(ids32)
            t.append(ii)
            ti = self._in(table, buf_table, t)
            oi = self._out(ids.size * E, t)
            with self._lock:
                _hip._check(self._lib.rvc_embed(self.handle, ii, ti, oi, ids.size, V, E), "rvc_embed")
            return self.download(oi, ids.shape + (E,))

        return self._run(go, t)

    def layer_norm(self, x, gamma, beta, eps=1e-5, buf_gamma=None, buf_beta=None):
        x = _as_f32(x, "layer_norm x")
        gamma = _as_f32(gamma, "layer_norm gamma")
        beta = _as_f32(beta, "layer_norm beta")
        if x.ndim < 1:
            raise ValueError("layer_norm needs at least 1-D input")
        cols = x.shape[-1]
        if gamma.size != cols or beta.size != cols:
            raise ValueError(f"layer_norm gamma/beta must have {cols} values")
        if x.size == 0:
            return np.empty(x.shape, dtype=np.float32)
        rows = x.size // cols
        t = []

        def go():
            xi = self.upload(x)
            t.append(xi)
            gi, bi = self._in(gamma, buf_gamma, t), self._in(beta, buf_beta, t)
            oi = self._out(x.size, t)
            with self._lock:
                _hip._check(self._lib.rvc_layernorm(self.handle, xi, gi, bi, oi, rows, cols, float(eps)),
                            "rvc_layernorm")
            return self.download(oi, x.shape)

        return self._run(go, t)

    def rmsnorm(self, x, gamma, eps=1e-5, buf_gamma=None):
        """out = x / sqrt(mean(x^2) + eps) * gamma over the last axis
        (runtime/backend.py:309-317, runtime/vulkan_ops.py:1994-2019)."""
        x = _as_f32(x, "rmsnorm x")
        gamma = _as_f32(gamma, "rmsnorm gamma")
        if gamma.ndim != 1:
            raise ValueError(f"rmsnorm gamma must be 1-D, got {gamma.ndim}-D")
        cols = gamma.shape[0]
        if x.ndim < 1 or x.shape[-1] != cols:
            raise ValueError(f"rmsnorm: x[-1]={x.shape[-1] if x.ndim else None} does not match gamma {gamma.shape}")
        if x.size == 0:
            return np.empty(x.shape, dtype=np.float32)
        rows = x.size // cols
        t = []

        def go():
            xi = self.upload(x)
            t.append(xi)
            gi = self._in(gamma, buf_gamma, t)
            oi = self._out(x.size, t)
            with self._lock:
                _hip._check(self._lib.rvc_rmsnorm(self.handle, xi, gi, oi, rows, cols, float(eps)), "rvc_rmsnorm")
            return self.download(oi, x.shape)

        return self._run(go, t)

    def softmax(self, x):
        x = _as_f32(x, "softmax x")
        if x.ndim < 1:
            raise ValueError("softmax needs at least 1-D input")
        cols = x.shape[-1]
        if x.size == 0:
            return np.empty(x.shape, dtype=np.float32)
        rows = x.size // cols
        t = []

        def go():
            xi = self.upload(x)
            t.append(xi)
            oi = self._out(x.size, t)
            with self._lock:
                _hip._check(self._lib.rvc_softmax(self.handle, xi, oi, rows, cols), "rvc_softmax")
            return self.download(oi, x.shape)

        return self._run(go, t)


_context = None
_context_lock = threading.Lock()


def get_context() -> HipContext:
    """Process-wide context, created lazily; a failure is not cached."""
    global _context
    if _context is not None:
        return _context
    with _context_lock:
        if _context is None:
            _context = HipContext()
        return _context


# ------------------------------------------------------------------ module-level ops
@_traced("matmul/gpu")
def matmul(a, b, buf_a=None, buf_b=None):
    return get_context().matmul(a, b, buf_a=buf_a, buf_b=buf_b)


@_traced("add/gpu")
def add(a, b, buf_a=None, buf_b=None):
    return get_context().add(a, b, buf_a=buf_a, buf_b=buf_b)


@_traced("mul/gpu")
def mul(a, b, buf_a=None, buf_b=None):
    return get_context().mul(a, b, buf_a=buf_a, buf_b=buf_b)


@_traced("relu/gpu")
def relu(a, buf_a=None):
    return get_context().relu(a, buf_a=buf_a)


@_traced("leaky_relu/gpu")
def leaky_relu(a, negative_slope=0.1):
    return get_context().leaky_relu(a, negative_slope)


@_traced("conv1d/gpu")
def conv1d(x, w, b=None, stride=1, padding=0, dilation=1, buf_w=None, buf_b=None):
    return get_context().conv1d(x, w, b, stride, padding, dilation, buf_w=buf_w, buf_b=buf_b)


@_traced("conv_transpose1d/gpu")
def conv_transpose1d(x, w, b=None, stride=1, padding=0, output_padding=0, dilation=1, buf_w=None,
                     buf_b=None):
    return get_context().conv_transpose1d(x, w, b, stride, padding, output_padding, dilation,
                                          buf_w=buf_w, buf_b=buf_b)


@_traced("embedding/gpu")
def embedding(ids, table, buf_table=None):
    return get_context().embedding(ids, table, buf_table=buf_table)


@_traced("add_inplace/gpu")
def add_inplace(a, b, buf_a=None, buf_b=None):
    return get_context().add_inplace(a, b, buf_a=buf_a, buf_b=buf_b)


@_traced("mul_inplace/gpu")
def mul_inplace(a, b, buf_a=None, buf_b=None):
    return get_context().mul_inplace(a, b, buf_a=buf_a, buf_b=buf_b)


@_traced("layer_norm/gpu")
def layer_norm(x, gamma, beta, eps=1e-5, buf_gamma=None, buf_beta=None):
    return get_context().layer_norm(x, gamma, beta, eps, buf_gamma=buf_gamma, buf_beta=buf_beta)


@_traced("rmsnorm/gpu")
def rmsnorm(x, gamma, eps=1e-5, buf_gamma=None):
    return get_context().rmsnorm(x, gamma, eps, buf_gamma=buf_gamma)


@_traced("softmax/gpu")
def softmax(x):
    return get_context().softmax(x)
