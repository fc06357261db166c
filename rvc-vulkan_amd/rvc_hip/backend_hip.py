# -*- coding: utf-8 -*-
"""Registration of the HIP backend with the reference's three extension points.

1. Op level -- ``runtime/backend.py:57-70``
   ``register_backend(name, module_path, label="", probe=None)``: the module
   named by ``module_path`` must expose the ``runtime.vulkan_ops`` op names
   (``rvc_hip.hip_ops`` does), ``probe()`` returns a bool, and
   ``RVC_BACKEND=hip`` selects it (``runtime/backend.py:111-151``).  A probe
   that fails makes the reference dispatcher fall back to numpy with a reason
   string; that fallback belongs to the reference's dispatcher, never to this
   package, whose ops raise when the library is missing.
2. Session level -- ``runtime/backend_api.py:349-366``
   ``register_backend(name, factory)`` with a ``Backend`` subclass; the
   reference's adapters only override ``backend_id`` and ``policy()`` on top of
   ``VCBackendBase`` (``runtime/backend_vulkan.py:44-51, 184-191``).
3. Model level -- the device-resident synthesis path that
   ``SynthesizerTrn.infer_controlled`` (``runtime/models/vits.py:2551-2595``)
   reaches through ``vulkan_ops.BatchRunner`` on the vulkan backend.
   ``bind_synthesizer`` builds a ``HipSynthesizer`` from a constructed
   reference ``SynthesizerTrn`` (its ``weight_dict`` and ``cfg``) so the caller
   can route ``infer_controlled`` / ``dec.forward`` to it; ``bind_hubert``
   does the same for a ``HubertEncoder`` (``runtime/models/hubert.py:355``),
   routing ``encode`` / ``encode_batch`` to a ``HipHubert``.

Every function takes the reference module or object as an argument, so this
package never imports the reference and the same code registers against any
registry with the reference's signatures.
"""

from __future__ import annotations

__all__ = [
    "BACKEND_NAME",
    "OP_MODULE",
    "LABEL",
    "probe",
    "register_op_backend",
    "make_session_backend",
    "register_session_backend",
    "bind_synthesizer",
    "bind_hubert",
]

BACKEND_NAME = "hip"
OP_MODULE = "rvc_hip.hip_ops"
LABEL = "hip (MI355X gfx950)"


def probe() -> bool:
    """True when the library loaded and an engine can be created and
    destroyed -- the same test as the reference's ``_probe_vulkan``
    (``runtime/backend.py:73-84``)."""
    try:
        from . import _hip

        if not _hip.has_so or not _hip.available:
            return False
        h = _hip.engine_create()
        _hip.engine_destroy(h)
        return True
    except Exception:  # noqa: BLE001  (a probe reports, it never raises)
        return False


def register_op_backend(registry, name: str = BACKEND_NAME) -> bool:
    """Register ``rvc_hip.hip_ops`` in an op-level registry with the
    signature of ``runtime.backend.register_backend``.

    Returns False when ``name`` is already registered (the reference raises
    ``ValueError`` for that, ``runtime/backend.py:66-67``; a module reload
    re-registering is not an error, as at ``runtime/backend.py:95-99``)."""
    try:
        registry.register_backend(name, OP_MODULE, label=LABEL, probe=probe)
    except ValueError:
        return False
    return True


def make_session_backend(base_cls):
    """A session adapter on top of ``base_cls`` (the reference's
    ``VCBackendBase``): ``backend_id = "hip"``, ``policy() == "gpu"``.

    The pipeline behind ``base_cls.process`` is the reference's; with
    ``RVC_BACKEND=hip`` its synthesis ops run on this backend."""

    class HipBackend(base_cls):
        backend_id = BACKEND_NAME

        def policy(self, query=None) -> str:
            return "gpu"

    HipBackend.__name__ = HipBackend.__qualname__ = "HipBackend"
    return HipBackend


def register_session_backend(api, base_cls):
    """``api.register_backend("hip", factory)`` with the adapter class as the
    zero-argument factory (``runtime/backend_api.py:349-366``); returns the
    class."""
    cls = make_session_backend(base_cls)
    api.register_backend(BACKEND_NAME, cls)
    return cls


def bind_synthesizer(trn, ctx=None, precision=0):
    """A ``HipSynthesizer`` holding the weights of a constructed reference
    ``SynthesizerTrn``: weights from ``trn.weight_dict``, upsample rates /
    kernels and sample rate from ``trn.cfg`` (``runtime/models/vits.py
    :2245-2266``), so both sides use the same geometry.  ``precision`` 1 / 2
    selects the bf16 modes (config 5; with the ResBlocks)."""
    from .synth import HipSynthesizer

    return HipSynthesizer(trn.weight_dict, geometry=trn.cfg, ctx=ctx, precision=precision)


def bind_hubert(encoder, ctx=None):
    """A ``HipHubert`` holding the weights of a constructed reference
    ``HubertEncoder``: its float32 state dict ``encoder._sd`` (prefix-stripped
    transformers keys, ``runtime/models/hubert.py:499-512``); the encoder's own
    derived entries (keys starting with ``_``) are skipped, the weight norm of
    the positional conv is applied again on the device side from
    ``weight_g``/``weight_v`` or ``parametrizations.weight.original0/1``."""
    from .hubert import HipHubert

    sd = {k: v for k, v in encoder._sd.items() if not k.startswith("_")}
    return HipHubert(sd, ctx=ctx)
