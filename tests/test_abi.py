# -*- coding: utf-8 -*-
"""CPU checks of the C-ABI boundary and the host logic (no GPU compute).

* librvc_hip.so loads and exports every symbol include/rvc_hip.h declares;
* the ctypes table covers the header exactly;
* error convention without a device: -1 + rvc_last_error text
  (engine/src/ffi.zig:36-45, :1110-1119);
* the host-side VitsConfig mirror against the reference-generated golden
  derivations."""

from __future__ import annotations

import ctypes
import json
import os
import re

import numpy as np
import pytest

from conftest import GOLDEN, ROOT

HEADER = os.path.join(ROOT, "include", "rvc_hip.h")


def _header_symbols():
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rvc_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def hip():
    from rvc_hip import _hip

    if not _hip.has_so:
        pytest.fail(f"librvc_hip.so must be built before the tests: {_hip.so_load_error}")
    return _hip


def test_header_symbols_exported(hip):
    syms = _header_symbols()
    assert len(syms) >= 40
    lib = ctypes.CDLL(hip.so_path)
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert sorted(hip.SYMBOLS) == syms


def test_error_convention_without_engine(hip):
    L = hip.get_lib()
    assert L.rvc_engine_destroy(424242) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_mem_free(424242, 1) == -1
    assert L.rvc_conv1d(424242, 1, 2, 0, 3, 1, 1, 1, 1, 1, 1, 0, 0, 1) == -1
    assert L.rvc_synth_destroy(777) == -1
    assert hip.last_error() == "invalid synth handle"
    buf = ctypes.create_string_buffer(5)
    assert L.rvc_last_error(buf, 5) == 0
    assert buf.value == b"inva"  # truncated, NUL-terminated
    assert L.rvc_last_error(buf, 0) == -1


def test_engine_create_reports_missing_device(hip):
    # On a machine without a GPU engine creation fails cleanly with a message;
    # on a GPU box it succeeds and is destroyed again.
    L = hip.get_lib()
    h = L.rvc_engine_create()
    if h == -1:
        assert hip.last_error()
        buf = ctypes.create_string_buffer(64)
        assert L.rvc_device_name(buf, 64) == -1
    else:
        assert h > 0 and L.rvc_engine_destroy(h) == 0


def test_vits_config_mirror_matches_reference_golden():
    from rvc_hip import synthetic as syn
    from rvc_hip.config import VitsConfig

    geoms = {"tiny": syn.GEOM_TINY, "40k": syn.GEOM_40K, "48k": syn.GEOM_48K}
    with open(os.path.join(GOLDEN, "vits_config.json")) as f:
        cases = json.load(f)
    for name, case in cases.items():
        w = syn.make_weights(geoms[name.split("_")[0]], seed=1)
        c = VitsConfig(w, case["config"], sr=case["sr_arg"])
        for k, v in case["derived"].items():
            assert getattr(c, k) == v, (name, k)


def test_synthetic_generator_is_seeded():
    from rvc_hip import synthetic as syn

    a = syn.make_weights(syn.GEOM_TINY, seed=3)
    b = syn.make_weights(syn.GEOM_TINY, seed=3)
    assert syn.weights_digest(a) == syn.weights_digest(b)
    assert syn.weights_digest(a) != syn.weights_digest(syn.make_weights(syn.GEOM_TINY, seed=4))
    f0 = syn.make_f0(200, np.random.default_rng(0))
    assert (f0 == 0).mean() >= 0.2 and f0.max() <= 400 and f0[f0 > 0].min() >= 80


def _ctypes_token(t):
    """Canonical token of a ctypes argument type (see make_loader_symbols.py)."""
    P = ctypes.POINTER
    table = {ctypes.c_int32: "I32", ctypes.c_int64: "I64", P(ctypes.c_float): "F32P", P(ctypes.c_int64): "I64P",
             P(P(ctypes.c_float)): "F32PP", P(P(ctypes.c_uint8)): "U8PP", ctypes.c_void_p: "VOIDP",
             ctypes.c_char_p: "CHARP", P(ctypes.c_char): "CHARP", ctypes.c_double: "DOUBLE",
             P(ctypes.c_double): "F64P", P(ctypes.c_int16): "I16P"}
    return table[t]


def _header_decls():
    """name -> argument type tokens of every prototype in include/rvc_hip.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    c_tok = {"int64_t": "I64", "int32_t": "I32", "float*": "F32P", "int64_t*": "I64P", "float**": "F32PP",
             "uint8_t**": "U8PP", "void*": "VOIDP", "char*": "CHARP", "double": "DOUBLE", "double*": "F64P",
             "int16_t*": "I16P"}
    out = {}
    for m in re.finditer(r"\b(?:int32_t|int64_t)\s+(rvc_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        toks = []
        for a in args:
            # "<base> <*...> <name>", const dropped: e.g. "const float* const* z" -> float**
            m2 = re.fullmatch(r"(\w+)\s*((?:\*\s*)*)(\w+)?", re.sub(r"\bconst\b", " ", a).strip())
            assert m2, (m.group(1), a)
            toks.append(c_tok[m2.group(1) + m2.group(2).replace(" ", "")])
        out[m.group(1)] = toks
    return out


def test_reference_loader_symbols_bind(hip):
    """Every symbol the reference's ctypes loader binds (runtime/_vulkan.py:
    148-278, no try/except) is exported with the same return width and, one
    by one, the same argument types -- in this package's ctypes table and in
    the C prototypes of include/rvc_hip.h the library is compiled against --
    so that loader can drive librvc_hip.so via RVC_CORE_DLL."""
    with open(os.path.join(GOLDEN, "reference_loader_symbols.json")) as f:
        ref = json.load(f)["symbols"]
    assert len(ref) == 56
    lib = ctypes.CDLL(hip.so_path)
    width = {"I32": ctypes.c_int32, "I64": ctypes.c_int64}
    decls = _header_decls()
    for name, spec in ref.items():
        assert hasattr(lib, name), name
        res, args = hip.SYMBOLS[name]
        assert len(args) == spec["nargs"] == len(spec["args"]), (name, len(args), spec["nargs"])
        assert [_ctypes_token(a) for a in args] == spec["args"], name
        assert decls[name] == spec["args"], (name, decls[name])
        assert res is width[spec["restype"]], name


def test_header_and_ctypes_table_agree(hip):
    """Every prototype of include/rvc_hip.h has the same argument types in
    rvc_hip._hip.SYMBOLS, and the two name the same exports."""
    decls = _header_decls()
    assert set(decls) == set(hip.SYMBOLS)
    for name, toks in decls.items():
        assert [_ctypes_token(a) for a in hip.SYMBOLS[name][1]] == toks, name


def test_not_provided_exports_fail_with_message(hip):
    L = hip.get_lib()
    assert L.rvc_batch_add_gru_sync(1, 1, 1, 1) == -1
    assert "rvc_batch_add_gru_sync: not provided" in hip.last_error()
    assert L.rvc_matmul_f16(1, 1, 1, 1, 1, 1, 1) == -1
    assert "rvc_matmul_f16: not provided" in hip.last_error()
    assert L.rvc_batch_add_im2col_2d(1, *([1] * 14)) == -1


def test_new_exports_reject_bad_handles(hip):
    L = hip.get_lib()
    a, b = ctypes.c_int64(), ctypes.c_int64()
    assert L.rvc_ts_stats(424242, ctypes.byref(a), ctypes.byref(b)) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_ts_reset(424242) == -1
    outs = [ctypes.c_int64() for _ in range(11)]
    assert L.rvc_mem_stats(424242, *[ctypes.byref(o) for o in outs]) == -1
    arr = (ctypes.c_int64 * 3)()
    assert L.rvc_mem_top(424242, 1, arr) == -1
    buf = ctypes.create_string_buffer(64)
    assert L.rvc_probe_extensions(424242, buf, 64) == -1
    assert L.rvc_rmsnorm(424242, 1, 2, 3, 1, 1, 1e-5) == -1
    assert L.rvc_batch_add_gelu_seg(424242, 1, 1, 0) == -1
    assert L.rvc_batch_add_conv_t1d_seg(424242, *([1] * 22)) == -1
    assert L.rvc_batch_add(424242, 12, 1, 2, 3, *([1] * 11)) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_conv2d(424242, *([1] * 15)) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_gru(424242, 1, 1, 1, 1, 1, 1) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_conv_t2d(424242, *([1] * 18)) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_insert_zeros_2x(424242, 1, 2, 1, 1, 1) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_batch_add_conv2d(424242, *([1] * 15)) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_batch_add_conv_t2d(424242, *([1] * 19)) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_batch_add_gru(424242, 1, 1, 1, 1, 1, 1) == -1
    assert hip.last_error() == "invalid engine handle"
    assert L.rvc_rmvpe_create(424242) == -1
    assert L.rvc_rmvpe_finalize(424242) == -1
    assert hip.last_error() == "invalid rmvpe handle"


def test_profile_summary_resblock_family():
    """The kernel-trace summary's ResBlock family: persistent instantiations
    with FAM = 1 (sixth template argument, with or without the staging flag
    after it) and three-group one-shot grids."""
    from rvc_hip.profsum import is_resblock

    assert is_resblock("conv1d_mfma_persist_kernel<64, 256, 32, 64, 8, 1, true>", (512, 1, 1))
    assert is_resblock("conv1d_mfma_persist_kernel<32, 512, 32, 64, 8, 1, false>", (512, 1, 1))
    assert is_resblock("conv1d_mfma_persist_kernel<32, 256, 32, 64, 8, 1>", (960, 1, 1))
    assert not is_resblock("conv1d_mfma_persist_kernel<64, 256, 32, 64, 8, 0, true>", (512, 1, 1))
    assert is_resblock("conv1d_mfma_kernel<64, 128, 32, 64, 8, 1, 1, 11, 1>", (79, 2, 3))
    assert not is_resblock("conv1d_mfma_kernel<64, 128, 32, 64, 8, 1, 1, 11, 1>", (79, 2, 1))
