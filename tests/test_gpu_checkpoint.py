# -*- coding: utf-8 -*-
"""Sessions built from checkpoint files (``rvc_hip.checkpoint``): an RVC
inference ``.pth`` (fp16 weights + config list, as RVC writes them) gives the
synthesizer the oracle computes from the same fp16-rounded weights, within the
fp32 waveform bar (max-abs 1e-3); a ``pytorch_model.bin`` gives a HuBERT
session bit-identical to one built from the in-memory state dict."""

from __future__ import annotations

import collections

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def test_synthesizer_from_inference_pth(tmp_path):
    from oracle import vits_ref
    from rvc_hip import _hip, checkpoint, synthetic as syn

    if not _hip.has_so:
        pytest.fail(f"HIP backend missing: {_hip.so_load_error}")
    geom = syn.GEOM_TINY
    w = syn.make_weights(geom, seed=8)
    cfg = geom.config_array()
    weight = collections.OrderedDict((k, torch.from_numpy(np.ascontiguousarray(v)).half()) for k, v in w.items())
    path = tmp_path / "model.pth"
    torch.save({"weight": weight, "config": cfg, "info": "test", "sr": "40k", "f0": 1, "version": "v2"}, path)
    s = checkpoint.load_synthesizer(path, sr=geom.sr)
    w16 = {k: v.astype(np.float16).astype(np.float32) for k, v in w.items()}
    inp = syn.make_synth_inputs(geom, P=9, seed=31)
    wave = s.infer_controlled(inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    ref = vits_ref.Synthesizer(w16, config=cfg, sr=geom.sr).infer_controlled(
        inp["phone"], inp["pitch"], inp["nsff0"], inp["sid"], inp["nz"], inp["ns"])
    assert wave.shape == ref.shape
    assert float(np.abs(wave - ref).max()) <= 1e-3
    s.close()


def test_hubert_from_pytorch_model_bin(tmp_path):
    from rvc_hip import checkpoint, synthetic as syn
    from rvc_hip.hubert import HipHubert

    sd = syn.make_hubert_weights(syn.HUBERT_BASE, seed=1)
    torch.save({k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in sd.items()}, tmp_path / "pytorch_model.bin")
    a = checkpoint.load_hubert(tmp_path)
    b = HipHubert(sd)
    x = syn.make_hubert_input(8000, seed=2)
    np.testing.assert_array_equal(a.encode(x), b.encode(x))
    a.close()
    b.close()


def test_rmvpe_from_pt(tmp_path):
    from rvc_hip import checkpoint, synthetic as syn
    from rvc_hip.rmvpe import HipRMVPE

    w = syn.make_rmvpe_weights(seed=4)
    sd = collections.OrderedDict((k, torch.from_numpy(np.ascontiguousarray(v)).half()) for k, v in w.items())
    torch.save(sd, tmp_path / "rmvpe.pt")
    a = checkpoint.load_rmvpe(tmp_path / "rmvpe.pt")
    b = HipRMVPE({k: v.astype(np.float16).astype(np.float32) for k, v in w.items()})
    x = syn.make_rmvpe_audio(6000, seed=1)
    np.testing.assert_array_equal(a.infer_from_audio(x), b.infer_from_audio(x))
    a.close()
    b.close()
