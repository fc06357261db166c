# -*- coding: utf-8 -*-
"""ctypes binding of ``librvc_hip.so`` (the HIP backend's C ABI).

Mirrors the reference loader ``runtime/_vulkan.py``: the library is looked up
without raising, ``has_so`` / ``available`` report the result as module-level
bools (``runtime/_vulkan.py:282-299``), ``so_load_error`` carries a readable
reason, every symbol gets ``restype`` / ``argtypes`` once at load
(``runtime/_vulkan.py:148-278``), and ``_check`` turns an rc of -1 into a
``RuntimeError`` carrying ``rvc_last_error`` (``runtime/_vulkan.py:320-324``).

Search order:
  1. ``RVC_HIP_SO`` (explicit path);
  2. ``librvc_hip.so`` next to this file (the in-tree build).

The module never falls back to anything: callers that need the GPU path get
a ``RuntimeError`` from ``get_lib()`` when the library is missing.
"""

from __future__ import annotations

import ctypes
import os

__all__ = [
    "has_so",
    "available",
    "so_path",
    "so_load_error",
    "is_available",
    "get_lib",
    "engine_create",
    "engine_destroy",
    "device_name",
    "last_error",
    "SYMBOLS",
]

I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32P = ctypes.POINTER(ctypes.c_float)
I64P = ctypes.POINTER(ctypes.c_int64)
CHARP = ctypes.c_char_p
VOIDP = ctypes.c_void_p
DBL = ctypes.c_double

# name -> (restype, argtypes); the full export list of include/rvc_hip.h
SYMBOLS = {
    "rvc_engine_create": (I64, []),
    "rvc_engine_destroy": (I32, [I64]),
    "rvc_mem_upload": (I32, [I64, F32P, I64, I64P]),
    "rvc_mem_upload_to": (I32, [I64, F32P, I64, I64]),
    "rvc_mem_upload_bytes": (I32, [I64, VOIDP, I64, I64P]),
    "rvc_mem_alloc": (I32, [I64, I64, I64P]),
    "rvc_mem_fill_zero": (I32, [I64, I64, I64]),
    "rvc_mem_download": (I32, [I64, I64, F32P, I64]),
    "rvc_mem_download_bytes": (I32, [I64, I64, VOIDP, I64]),
    "rvc_mem_free": (I32, [I64, I64]),
    "rvc_mem_upload_to_batch": (I32, [I64, I64, I64P, ctypes.POINTER(F32P), I64P]),
    "rvc_mem_download_batch": (I32, [I64, I64P, ctypes.POINTER(ctypes.POINTER(ctypes.c_uint8)), I64P, I64]),
    "rvc_matmul": (I32, [I64] * 7),
    "rvc_conv1d_noalloc": (I32, [I64] * 14),
    "rvc_add": (I32, [I64] * 5),
    "rvc_mul": (I32, [I64] * 5),
    "rvc_relu": (I32, [I64] * 3),
    "rvc_conv1d": (I32, [I64] * 14),
    "rvc_conv_t1d": (I32, [I64] * 14),
    "rvc_conv1d_bf16": (I32, [I64] * 14),
    "rvc_conv_t1d_bf16": (I32, [I64] * 14),
    "rvc_embed": (I32, [I64] * 7),
    "rvc_add_inplace": (I32, [I64] * 4),
    "rvc_mul_inplace": (I32, [I64] * 4),
    "rvc_leaky_relu": (I32, [I64] * 4),
    "rvc_copy": (I32, [I64] * 4),
    "rvc_layernorm": (I32, [I64] * 7 + [DBL]),
    "rvc_softmax": (I32, [I64] * 5),
    "rvc_rmsnorm": (I32, [I64] * 6 + [DBL]),
    "rvc_batch_begin": (I32, [I64]),
    "rvc_batch_add": (I32, [I64, I32] + [I64] * 14),
    "rvc_batch_add_copy_seg": (I32, [I64] * 6),
    "rvc_batch_add_add_seg": (I32, [I64] * 6),
    "rvc_batch_add_mul_seg": (I32, [I64] * 6),
    "rvc_batch_add_leaky_seg": (I32, [I64] * 5),
    "rvc_batch_add_gelu_seg": (I32, [I64] * 4),
    "rvc_batch_add_conv1d_seg": (I32, [I64] * 17),
    "rvc_batch_add_conv_t1d_seg": (I32, [I64] * 23),
    "rvc_batch_commit": (I32, [I64]),
    "rvc_batch_commit_async": (I32, [I64]),
    "rvc_batch_wait": (I32, [I64]),
    "rvc_batch_discard": (I32, [I64]),
    "rvc_device_name": (I32, [CHARP, I64]),
    "rvc_last_error": (I32, [CHARP, I64]),
    "rvc_ts_stats": (I32, [I64, I64P, I64P]),
    "rvc_ts_reset": (I32, [I64]),
    "rvc_mem_stats": (I32, [I64] + [I64P] * 11),
    "rvc_mem_top": (I64, [I64, I64, I64P]),
    "rvc_probe_extensions": (I32, [I64, CHARP, I64]),
    # exported for the reference loader; each returns -1 with a message
    "rvc_matmul_f16": (I32, [I64] * 7),
    "rvc_conv2d": (I32, [I64] * 16),
    "rvc_conv_t2d": (I32, [I64] * 19),
    "rvc_insert_zeros_2x": (I32, [I64] * 6),
    "rvc_batch_add_conv2d": (I32, [I64] * 16),
    "rvc_batch_add_conv_t2d": (I32, [I64] * 20),
    "rvc_batch_add_im2col_1d": (I32, [I64] * 11),
    "rvc_batch_add_im2col_2d": (I32, [I64] * 15),
    "rvc_batch_add_gru": (I32, [I64] * 7),
    "rvc_gru": (I32, [I64] * 7),
    "rvc_batch_add_gru_sync": (I32, [I64] * 4),
    "rvc_synth_create": (I64, [I64]),
    "rvc_synth_destroy": (I32, [I64]),
    "rvc_synth_set_weight": (I32, [I64, CHARP, F32P, I64P, I32]),
    "rvc_synth_finalize": (I32, [I64, I64, I64P, I64P, I32]),
    "rvc_synth_infer": (I32, [I64, F32P, I64P, F32P, I64P, F32P, F32P, I64, I64, F32P]),
    "rvc_synth_submit": (I64, [I64, F32P, I64, I64P, F32P, I64P, F32P, F32P, I64, I64]),
    "rvc_synth_collect": (I32, [I64, I64, F32P]),
    "rvc_synth_abort": (I32, [I64, I64]),
    "rvc_synth_infer_dev": (I32, [I64] * 10),
    "rvc_synth_decode": (I32, [I64, F32P, F32P, F32P, F32P, I64, I64, F32P]),
    "rvc_synth_decode_dev": (I32, [I64] * 8),
    "rvc_synth_prep": (I32, [I64, F32P, I64P, F32P, I64P, F32P, I64, I64, I64, F32P, F32P, F32P]),
    "rvc_synth_phase_offsets": (I32, [I64, F32P, I64, I64, F32P]),
    "rvc_synth_decode_chunks": (I32, [I64, I64, ctypes.POINTER(F32P), ctypes.POINTER(F32P), ctypes.POINTER(F32P),
                                      ctypes.POINTER(F32P), I64P, F32P, ctypes.POINTER(F32P)]),
    "rvc_synth_read": (I32, [I64, CHARP, F32P, I64]),
    "rvc_synth_set_precision": (I32, [I64, I32]),
    "rvc_synth_set_debug": (I32, [I64, I32]),
    "rvc_synth_set_timing": (I32, [I64, CHARP]),
    "rvc_synth_get_timing": (I32, [I64, ctypes.POINTER(DBL), I64P, ctypes.POINTER(DBL),
                                   ctypes.POINTER(DBL)]),
    "rvc_hubert_create": (I64, [I64]),
    "rvc_hubert_destroy": (I32, [I64]),
    "rvc_hubert_set_weight": (I32, [I64, CHARP, F32P, I64P, I32]),
    "rvc_hubert_finalize": (I32, [I64]),
    "rvc_hubert_frames": (I32, [I64, I64, I64P]),
    "rvc_hubert_encode": (I32, [I64, F32P, I64, I64, I32, F32P]),
    "rvc_hubert_encode_dev": (I32, [I64, I64, I64, I64, I32, I64]),
    "rvc_hubert_read": (I32, [I64, CHARP, F32P, I64]),
    "rvc_hubert_set_debug": (I32, [I64, I32]),
    "rvc_hubert_set_timing": (I32, [I64, CHARP]),
    "rvc_hubert_get_timing": (I32, [I64, ctypes.POINTER(DBL), I64P, ctypes.POINTER(DBL),
                                    ctypes.POINTER(DBL)]),
    "rvc_rmvpe_create": (I64, [I64]),
    "rvc_rmvpe_destroy": (I32, [I64]),
    "rvc_rmvpe_set_weight": (I32, [I64, CHARP, F32P, I64P, I32]),
    "rvc_rmvpe_finalize": (I32, [I64]),
    "rvc_rmvpe_frames": (I32, [I64, I64, I64P]),
    "rvc_rmvpe_infer": (I32, [I64, F32P, I64, DBL, F32P]),
    "rvc_rmvpe_infer_dev": (I32, [I64, I64, I64, DBL, I64]),
    "rvc_rmvpe_read": (I32, [I64, CHARP, F32P, I64]),
    "rvc_rmvpe_set_timing": (I32, [I64, CHARP]),
    "rvc_rmvpe_get_timing": (I32, [I64, ctypes.POINTER(DBL), I64P, ctypes.POINTER(DBL), ctypes.POINTER(DBL)]),
    "rvc_vc_create": (I64, [I64]),
    "rvc_vc_destroy": (I32, [I64]),
    "rvc_vc_set_index": (I32, [I64, F32P, I64, I64]),
    "rvc_vc_index_info": (I32, [I64, I64P, I64P]),
    "rvc_vc_search": (I32, [I64, F32P, I64, I64, F32P, I64P]),
    "rvc_vc_search_dev": (I32, [I64, I64, I64, I64, I64, I64]),
    "rvc_vc_prepare": (I32, [I64, F32P, I64, I64, DBL, F32P, DBL, F32P]),
    "rvc_vc_prepare_dev": (I32, [I64, I64, I64, I64, DBL, I64, DBL, I64]),
    "rvc_vc_change_rms": (I32, [I64, F32P, I64, I64, F32P, I64, I64, DBL, F32P]),
    "rvc_vc_change_rms_dev": (I32, [I64, I64, I64, I64, I64, I64, I64, DBL, I64]),
    "rvc_vc_to_int16": (I32, [I64, F32P, I64, ctypes.POINTER(ctypes.c_int16)]),
    "rvc_vc_to_int16_dev": (I32, [I64, I64, I64, I64]),
    "rvc_vc_set_timing": (I32, [I64, CHARP]),
    "rvc_vc_get_timing": (I32, [I64, ctypes.POINTER(DBL), I64P, ctypes.POINTER(DBL), ctypes.POINTER(DBL)]),
}


def _candidate_paths() -> list:
    here = os.path.dirname(os.path.abspath(__file__))
    paths = []
    env = os.environ.get("RVC_HIP_SO", "").strip()
    if env:
        paths.append(env)
    paths.append(os.path.join(here, "librvc_hip.so"))
    return paths


def _find() -> str | None:
    for p in _candidate_paths():
        if os.path.isfile(p):
            return os.path.abspath(p)
    return None


def _load():
    path = _find()
    if path is None:
        return None, None, (
            "librvc_hip.so not found; looked in:\n  - " + "\n  - ".join(_candidate_paths())
            + "\nbuild it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "or point RVC_HIP_SO at it")
    try:
        lib = ctypes.CDLL(path)
    except OSError as exc:
        return None, path, f"loading {path} failed: {exc}"
    missing = []
    for name, (res, args) in SYMBOLS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            missing.append(name)
            continue
        fn.restype = res
        fn.argtypes = args
    if missing:
        return None, path, f"{path} lacks exports: {', '.join(missing)}"
    return lib, path, ""


lib, so_path, so_load_error = _load()

has_so: bool = lib is not None
"""Whether the shared library loaded and exports every symbol."""

available: bool = has_so
"""Module-level bool (not a function), like ``runtime._vulkan.available``."""


def is_available() -> bool:
    return available


def get_lib() -> ctypes.CDLL:
    if lib is None:
        raise RuntimeError(f"librvc_hip.so unavailable ({so_load_error})")
    return lib


def last_error() -> str:
    buf = ctypes.create_string_buffer(4096)
    get_lib().rvc_last_error(buf, len(buf))
    return buf.value.decode("utf-8", "replace") or "unknown error"


def _check(rc: int, what: str) -> int:
    if rc == -1:
        raise RuntimeError(f"{what} failed: {last_error()}")
    return rc


def engine_create() -> int:
    h = get_lib().rvc_engine_create()
    if h < 0:
        raise RuntimeError(f"rvc_engine_create failed: {last_error()}")
    return int(h)


def engine_destroy(h: int) -> int:
    return int(get_lib().rvc_engine_destroy(int(h)))


def device_name() -> str:
    """Device name; creates (and destroys) a temporary engine when none is live."""
    L = get_lib()
    buf = ctypes.create_string_buffer(256)
    if L.rvc_device_name(buf, len(buf)) == 0:
        return buf.value.decode("utf-8", "replace")
    h = engine_create()
    try:
        _check(L.rvc_device_name(buf, len(buf)), "rvc_device_name")
    finally:
        engine_destroy(h)
    return buf.value.decode("utf-8", "replace")
