# -*- coding: utf-8 -*-
"""CPU checks of the registration glue (rvc_hip.backend_hip) against
registries with the reference's signatures and behaviour:

* op level, ``runtime/backend.py:57-70`` (name normalisation, ValueError on a
  duplicate) and the probe-then-import selection of ``:111-151``;
* session level, ``runtime/backend_api.py:349-380`` (zero-argument factory,
  ValueError on a duplicate) with a ``VCBackendBase``-like base class;
* model level, ``bind_synthesizer`` reading ``weight_dict`` / ``cfg``.

The registries below restate only the reference behaviour these functions
rely on; the reference itself is not imported."""

from __future__ import annotations

import importlib
import types

import pytest


class OpRegistry:
    """The op-level registry contract of runtime/backend.py:57-70, 111-151."""

    def __init__(self):
        self.backends = {"numpy": {"module": None, "label": "numpy (CPU)"}}
        self.reason = None

    def register_backend(self, name, module_path, label="", probe=None):
        name = name.strip().lower()
        if not name or name in self.backends:
            raise ValueError(f"invalid or duplicate backend name {name!r}")
        self.backends[name] = {"module": module_path, "label": label or name, "probe": probe}

    def select(self, forced):
        info = self.backends.get(forced)
        if info is None:
            self.reason = "unknown"
            return "numpy"
        if info.get("probe") is not None and not info["probe"]():
            self.reason = f"backend {forced} probe failed"
            return "numpy"
        importlib.import_module(info["module"])
        return forced


class SessionApi:
    """The session registry contract of runtime/backend_api.py:349-380."""

    def __init__(self):
        self.BACKENDS = {}

    def register_backend(self, name, factory):
        name = name.strip().lower()
        if not name or name in self.BACKENDS or not callable(factory):
            raise ValueError(name)
        self.BACKENDS[name] = factory

    def get_backend_instance(self, name):
        return self.BACKENDS[name.strip().lower()]()


class VCBase:
    """Stand-in for VCBackendBase: subclasses override backend_id / policy."""

    backend_id = ""

    def __init__(self):
        self.rtf_last = None

    def policy(self, query=None):
        return "?"


def test_op_registration_and_duplicate():
    from rvc_hip import backend_hip

    reg = OpRegistry()
    assert backend_hip.register_op_backend(reg) is True
    info = reg.backends["hip"]
    assert info["module"] == "rvc_hip.hip_ops" and info["probe"] is backend_hip.probe
    assert info["label"].startswith("hip")
    # a second registration (module reload) is reported, not raised
    assert backend_hip.register_op_backend(reg) is False
    # the op module exposes the dispatcher's op names (runtime/backend.py:205-316)
    mod = importlib.import_module(info["module"])
    for op in ("matmul", "add", "mul", "relu", "conv1d", "conv_transpose1d", "embedding", "add_inplace",
               "mul_inplace", "layer_norm", "softmax", "rmsnorm"):
        assert callable(getattr(mod, op)), op


def test_probe_matches_library_state():
    from rvc_hip import _hip, backend_hip

    reg = OpRegistry()
    backend_hip.register_op_backend(reg)
    ok = backend_hip.probe()
    if not _hip.has_so:
        assert ok is False
    chosen = reg.select("hip")
    # without a GPU the probe fails and the reference dispatcher would pick numpy
    assert chosen == ("hip" if ok else "numpy")
    if not ok:
        assert "probe failed" in reg.reason


def test_ops_raise_without_device():
    """The op module never computes on the CPU: without an engine it raises."""
    from rvc_hip import backend_hip, hip_ops

    if backend_hip.probe():
        pytest.skip("a GPU is present")
    import numpy as np

    with pytest.raises(RuntimeError):
        hip_ops.conv1d(np.ones((1, 2, 8), np.float32), np.ones((3, 2, 3), np.float32))


def test_session_registration():
    from rvc_hip import backend_hip

    api = SessionApi()
    cls = backend_hip.register_session_backend(api, VCBase)
    assert api.BACKENDS["hip"] is cls
    inst = api.get_backend_instance("HIP")
    assert isinstance(inst, VCBase)
    assert inst.backend_id == "hip" and inst.policy() == "gpu" and inst.rtf_last is None
    with pytest.raises(ValueError):
        backend_hip.register_session_backend(api, VCBase)


def test_bind_synthesizer_uses_reference_geometry(monkeypatch):
    from rvc_hip import backend_hip, synth

    seen = {}

    class FakeSynth:
        def __init__(self, w, config=None, sr=None, ctx=None, geometry=None, precision=0):
            seen.update(w=w, geometry=geometry, ctx=ctx, precision=precision)

    monkeypatch.setattr(synth, "HipSynthesizer", FakeSynth)
    cfg = types.SimpleNamespace(upsample_rates=[12, 10, 2, 2], upsample_kernels=[24, 20, 4, 4], sr=48000)
    trn = types.SimpleNamespace(weight_dict={"k": 1}, cfg=cfg)
    backend_hip.bind_synthesizer(trn)
    assert seen["w"] == {"k": 1} and seen["geometry"] is cfg and seen["precision"] == 0
    backend_hip.bind_synthesizer(trn, precision=1)
    assert seen["precision"] == 1
