# -*- coding: utf-8 -*-
"""The torch-free checkpoint reader (``rvc_hip.checkpoint``) against
``torch.save``, the format's own writer: every tensor must come back with the
values, shape and dtype torch saved (bfloat16 as float32), the RVC inference /
training / bare layouts must yield the state dict and config the reference's
``SynthesizerTrn`` would use, and a file naming any other global must be
refused without running it."""

from __future__ import annotations

import collections
import io
import os
import pickle
import zipfile

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rvc_hip import checkpoint as ck  # noqa: E402
from rvc_hip import synthetic as syn  # noqa: E402
from rvc_hip.config import VitsConfig  # noqa: E402


def _save(obj, path, **kw):
    torch.save(obj, path, **kw)
    return path


def test_tensors_round_trip(tmp_path):
    g = torch.Generator().manual_seed(0)
    base = torch.randn(6, 5, generator=g)
    obj = collections.OrderedDict(
        f32=torch.randn(3, 4, 5, generator=g),
        f16=torch.randn(7, generator=g).half(),
        bf16=torch.randn(2, 3, generator=g).bfloat16(),
        f64=torch.randn(4, generator=g).double(),
        i64=torch.arange(-5, 5),
        i32=torch.arange(6, dtype=torch.int32).reshape(2, 3),
        u8=torch.arange(250, 256, dtype=torch.uint8),
        b=torch.tensor([True, False, True]),
        scalar=torch.tensor(3.5),
        empty=torch.zeros(0, 4),
        transposed=base.t(),                 # non-contiguous view
        sliced=base[1:4, ::2],               # offset + stride into a shared storage
        param=torch.nn.Parameter(torch.ones(2, 2)),
    )
    out = ck.load_pth(_save(obj, tmp_path / "t.pth"))
    assert isinstance(out, collections.OrderedDict) and list(out) == list(obj)
    for k, t in obj.items():
        ref = t.detach().float().numpy() if t.dtype == torch.bfloat16 else t.detach().numpy()
        got = out[k]
        assert got.shape == ref.shape and got.dtype == ref.dtype, k
        np.testing.assert_array_equal(got, ref, err_msg=k)


def test_nested_containers_and_numbers(tmp_path):
    obj = {"a": [1, 2.5, "x", None, (3, torch.ones(2))], "b": {"c": np.float32(1.5), "d": np.arange(3)}, "e": True}
    out = ck.load_pth(_save(obj, tmp_path / "n.pth"))
    assert out["a"][:4] == [1, 2.5, "x", None] and out["e"] is True
    np.testing.assert_array_equal(out["a"][4][1], np.ones(2, np.float32))
    assert out["b"]["c"] == np.float32(1.5)
    np.testing.assert_array_equal(out["b"]["d"], np.arange(3))


def _rvc_inference_ckpt(w, cfg, half=True):
    """An RVC v2 inference checkpoint as RVC's savee writes it: fp16 weights
    under "weight", the config list, info, sr, f0, version."""
    weight = collections.OrderedDict(
        (k, torch.from_numpy(np.ascontiguousarray(v)).half() if half else torch.from_numpy(np.ascontiguousarray(v)))
        for k, v in w.items())
    return {"weight": weight, "config": cfg, "info": "10epoch", "sr": "40k", "f0": 1, "version": "v2"}


def test_rvc_layouts(tmp_path):
    geom = syn.GEOM_TINY
    w = syn.make_weights(geom, seed=4)
    cfg = geom.config_array()
    # inference layout, fp16 as RVC stores it
    wt, c = ck.synthesizer_weights(ck.load_pth(_save(_rvc_inference_ckpt(w, cfg), tmp_path / "inf.pth")))
    assert c == cfg and set(wt) == set(w)
    for k in w:
        np.testing.assert_array_equal(wt[k], w[k].astype(np.float16).astype(np.float32), err_msg=k)
        assert wt[k].dtype == np.float32
    # training layout: {"model": state_dict, ...}, float32, no config
    train = {"model": {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in w.items()}, "iteration": 7,
             "learning_rate": 1e-4, "optimizer": {"state": {}, "param_groups": [{"lr": 1e-4}]}}
    wt2, c2 = ck.synthesizer_weights(ck.load_pth(_save(train, tmp_path / "train.pth")))
    assert c2 is None
    for k in w:
        np.testing.assert_array_equal(wt2[k], w[k])
    # bare state dict
    wt3, c3 = ck.synthesizer_weights(ck.load_pth(_save({k: torch.from_numpy(np.ascontiguousarray(v))
                                                         for k, v in w.items()}, tmp_path / "bare.pth")))
    assert c3 is None and set(wt3) == set(w)
    # the geometry the reference's VitsConfig derives from the config list
    vc = VitsConfig(wt, c)
    assert vc.upsample_rates == list(geom.upsample_rates) and vc.sr == geom.sr and vc.upsample_kernels == list(geom.upsample_kernels)


def test_hubert_state_dict(tmp_path):
    sd = {"feature_projection.projection.weight": torch.randn(8, 4), "encoder.layer_norm.bias": torch.zeros(8)}
    out = ck.hubert_state_dict(ck.load_pth(_save(sd, tmp_path / "pytorch_model.bin")))
    np.testing.assert_array_equal(out["feature_projection.projection.weight"], sd["feature_projection.projection.weight"].numpy())


class _Marker:
    pass


def test_refuses_foreign_globals(tmp_path):
    """A data.pkl that names os.system (the classic malicious pickle) is
    refused before anything is called."""
    sentinel = tmp_path / "ran"

    class _Evil:
        def __reduce__(self):
            return (os.system, (f"touch {sentinel}",))

    path = tmp_path / "evil.pth"
    with zipfile.ZipFile(path, "w") as zf:
        zf.writestr("evil/data.pkl", pickle.dumps({"weight": _Evil()}, protocol=2))
        zf.writestr("evil/byteorder", "little")
    with pytest.raises(ck.CheckpointError, match="posix.system|os.system|nt.system"):
        ck.load_pth(path)
    assert not sentinel.exists()
    with zipfile.ZipFile(tmp_path / "cls.pth", "w") as zf:
        zf.writestr("a/data.pkl", pickle.dumps(_Marker(), protocol=2))
    with pytest.raises(ck.CheckpointError):
        ck.load_pth(tmp_path / "cls.pth")


def test_rejects_non_checkpoints(tmp_path):
    legacy = io.BytesIO()
    torch.save({"x": torch.ones(2)}, legacy, _use_new_zipfile_serialization=False)
    with pytest.raises(ck.CheckpointError, match="zip"):
        ck.load_pth(legacy.getvalue())
    with zipfile.ZipFile(tmp_path / "nodata.zip", "w") as zf:
        zf.writestr("x.txt", "hi")
    with pytest.raises(ck.CheckpointError, match="data.pkl"):
        ck.load_pth(tmp_path / "nodata.zip")
    with pytest.raises(ck.CheckpointError, match="no such file"):
        ck.load_pth(tmp_path / "missing.pth")
    # a storage member that is missing
    buf = io.BytesIO()
    torch.save({"x": torch.ones(3)}, buf)
    src = zipfile.ZipFile(io.BytesIO(buf.getvalue()))
    out = io.BytesIO()
    with zipfile.ZipFile(out, "w") as zf:
        for n in src.namelist():
            if "/data/" not in n:
                zf.writestr(n, src.read(n))
    with pytest.raises(ck.CheckpointError, match="missing"):
        ck.load_pth(out.getvalue())


def test_rmvpe_state_dict(tmp_path):
    """rmvpe.pt layout: fp16 tensors plus BatchNorm num_batches_tracked
    counters; the loader returns float32 arrays and drops the counters."""
    w = syn.make_rmvpe_weights(seed=2)
    keys = [k for k in w if k.startswith("unet.encoder.layers.0.") or k.startswith("fc.")]
    sd = collections.OrderedDict((k, torch.from_numpy(np.ascontiguousarray(w[k])).half()) for k in keys)
    sd["unet.encoder.bn.num_batches_tracked"] = torch.tensor(7)
    out = ck.rmvpe_state_dict(ck.load_pth(_save(sd, tmp_path / "rmvpe.pt")))
    assert set(out) == set(keys)
    for k in keys:
        assert out[k].dtype == np.float32
        np.testing.assert_array_equal(out[k], w[k].astype(np.float16).astype(np.float32))
