# -*- coding: utf-8 -*-
"""Torch-free reader for PyTorch checkpoints (``.pth`` / ``pytorch_model.bin``).

The reference reads checkpoints without torch through ``torch_compat.load_pth``
(``torch_compat.py:1005-1025``): a zip archive (PyTorch >= 1.6 format) whose
``data.pkl`` object graph refers to tensor storages stored as archive members
``data/<key>``.  This module reads the same format into numpy arrays, with one
difference in policy: the unpickler resolves only an allow-list of globals
(containers, the tensor / parameter rebuild functions, storage types, dtype
and size objects, numpy scalars and arrays) and raises ``CheckpointError`` for
anything else, so no code named by the file runs -- the reference falls back
to importing any other global (``torch_compat.py:889-896``).

Tensors come back as C-contiguous numpy arrays of their stored dtype
(bfloat16 widened to float32, as numpy has no bfloat16).  Legacy non-zip
checkpoints (``_use_new_zipfile_serialization=False``) are rejected, as in the
reference (``torch_compat.py:927-941``).

``synthesizer_weights`` applies ``SynthesizerTrn.__init__``'s layout rules
(``runtime/models/vits.py:2245-2262``): an inference checkpoint
``{"weight": state_dict, "config": [...], ...}``, a training checkpoint
``{"model": state_dict, ...}``, or a bare state dict.  ``load_synthesizer`` /
``load_hubert`` build the device-resident sessions from a checkpoint file.
"""

from __future__ import annotations

import codecs
import collections
import io
import os
import pickle
import zipfile

import numpy as np

__all__ = [
    "CheckpointError",
    "load_pth",
    "synthesizer_weights",
    "load_synthesizer",
    "hubert_state_dict",
    "load_hubert",
    "rmvpe_state_dict",
    "load_rmvpe",
]


class CheckpointError(Exception):
    """A file that is not a readable PyTorch zip checkpoint, or one whose
    object graph names a global outside the allow-list."""


# storage class name -> numpy dtype (torch/storage.py's typed storages)
_STORAGE_DTYPES = {
    "DoubleStorage": np.float64, "FloatStorage": np.float32, "HalfStorage": np.float16,
    "BFloat16Storage": "bfloat16", "LongStorage": np.int64, "IntStorage": np.int32,
    "ShortStorage": np.int16, "CharStorage": np.int8, "ByteStorage": np.uint8, "BoolStorage": np.bool_,
    "UntypedStorage": np.uint8,
}
# torch dtype attribute name -> numpy dtype (the v3 rebuild and dtype objects)
_DTYPE_NAMES = {
    "float64": np.float64, "double": np.float64, "float32": np.float32, "float": np.float32,
    "float16": np.float16, "half": np.float16, "bfloat16": "bfloat16", "int64": np.int64, "long": np.int64,
    "int32": np.int32, "int": np.int32, "int16": np.int16, "short": np.int16, "int8": np.int8, "uint8": np.uint8,
    "bool": np.bool_,
}


class _StorageType:
    def __init__(self, name, dtype):
        self.name = name
        self.dtype = dtype


class _Dtype:
    def __init__(self, name):
        self.name = name
        self.dtype = _DTYPE_NAMES[name]


def _np_dtype(d):
    return np.dtype(np.uint16) if d == "bfloat16" else np.dtype(d)


class _Storage:
    """One archive member ``data/<key>`` viewed as a flat array of its dtype."""

    def __init__(self, zf, prefix, key, dtype, byteorder):
        self.key = key
        self.dtype = dtype
        name = f"{prefix}data/{key}"
        try:
            raw = zf.read(name)
        except KeyError:
            raise CheckpointError(f"storage member {name!r} missing from the archive") from None
        dt = _np_dtype(dtype)
        if len(raw) % dt.itemsize:
            raise CheckpointError(f"storage {key}: {len(raw)} bytes is not a whole number of {dt} elements")
        arr = np.frombuffer(raw, dtype=dt.newbyteorder("<" if byteorder == "little" else ">"))
        self.flat = arr.astype(dt.newbyteorder("="), copy=False)


def _to_numpy(storage, offset, size, stride, dtype_override=None):
    if not isinstance(storage, _Storage):
        raise CheckpointError(f"tensor rebuild without a storage ({type(storage).__name__})")
    size = tuple(int(s) for s in size)
    stride = tuple(int(s) for s in stride)
    if len(size) != len(stride):
        raise CheckpointError("tensor rebuild: size and stride differ in length")
    n = int(np.prod(size)) if size else 1
    flat = storage.flat
    if n == 0:
        out = np.zeros(size, dtype=flat.dtype)
    else:
        last = int(offset) + sum((s - 1) * st for s, st in zip(size, stride))
        if offset < 0 or any(st < 0 for st in stride) or last >= flat.shape[0]:
            raise CheckpointError(f"tensor view outside its storage (offset {offset}, size {size}, stride {stride})")
        view = np.lib.stride_tricks.as_strided(flat[int(offset):], shape=size,
                                               strides=tuple(st * flat.itemsize for st in stride), writeable=False)
        out = np.array(view, order="C")  # a copy; keeps 0-d tensors 0-d
    kind = dtype_override if dtype_override is not None else storage.dtype
    if kind == "bfloat16":
        out = (out.astype(np.uint32) << 16).view(np.float32)
    return out


def _rebuild_tensor_v2(storage, storage_offset, size, stride, requires_grad=False, backward_hooks=None,
                       metadata=None):
    return _to_numpy(storage, storage_offset, size, stride)


def _rebuild_tensor(storage, storage_offset, size, stride):
    return _to_numpy(storage, storage_offset, size, stride)


def _rebuild_tensor_v3(storage, storage_offset, size, stride, requires_grad, backward_hooks, dtype, metadata=None):
    kind = dtype.dtype if isinstance(dtype, _Dtype) else None
    if isinstance(storage, _Storage) and kind is not None and storage.dtype != kind:
        # untyped storage reinterpreted as the tensor's dtype
        st = _Storage.__new__(_Storage)
        st.key, st.dtype = storage.key, kind
        st.flat = storage.flat.view(_np_dtype(kind))
        storage = st
    return _to_numpy(storage, storage_offset, size, stride, kind)


def _rebuild_parameter(data, requires_grad, backward_hooks, *state):
    return data


def _make_size(*args):
    return tuple(args[0]) if len(args) == 1 and isinstance(args[0], (tuple, list)) else tuple(args)


class _Unpickler(pickle.Unpickler):
    """Resolves an allow-list of globals only; tensors become numpy arrays."""

    _TORCH = {
        ("torch._utils", "_rebuild_tensor_v2"): _rebuild_tensor_v2,
        ("torch._utils", "_rebuild_tensor"): _rebuild_tensor,
        ("torch._utils", "_rebuild_tensor_v3"): _rebuild_tensor_v3,
        ("torch._utils", "_rebuild_parameter"): _rebuild_parameter,
        ("torch._utils", "_rebuild_parameter_v2"): _rebuild_parameter,
        ("torch._utils", "_rebuild_parameter_with_state"): _rebuild_parameter,
        ("torch", "Size"): _make_size,
    }
    _SAFE = {
        ("collections", "OrderedDict"): collections.OrderedDict,
        ("builtins", "set"): set,
        ("builtins", "frozenset"): frozenset,
        ("builtins", "complex"): complex,
        ("numpy", "dtype"): np.dtype,
        ("numpy", "ndarray"): np.ndarray,
        # protocol-2 pickles of bytes (numpy array payloads): str -> bytes
        ("_codecs", "encode"): codecs.encode,
    }

    def __init__(self, data, zf, prefix, byteorder):
        super().__init__(io.BytesIO(data), encoding="utf-8")
        self._zf = zf
        self._prefix = prefix
        self._byteorder = byteorder
        self._storages = {}

    def find_class(self, module, name):
        key = (module, name)
        if key in self._TORCH:
            return self._TORCH[key]
        if key in self._SAFE:
            return self._SAFE[key]
        if module == "torch" and name in _STORAGE_DTYPES:
            return _StorageType(name, _STORAGE_DTYPES[name])
        if module == "torch" and name in _DTYPE_NAMES:
            return _Dtype(name)
        if module in ("numpy.core.multiarray", "numpy._core.multiarray") and name in ("scalar", "_reconstruct"):
            return super().find_class(module, name)
        if module in ("numpy.core.numeric", "numpy._core.numeric") and name == "_frombuffer":
            return super().find_class(module, name)
        raise CheckpointError(f"checkpoint refers to {module}.{name}, which this reader does not load "
                              "(only tensors, containers and numbers are read)")

    def persistent_load(self, pid):
        # ('storage', storage_type, key, location, numel)
        if not (isinstance(pid, tuple) and len(pid) >= 3 and pid[0] == "storage"):
            raise CheckpointError(f"unsupported persistent id {pid!r}")
        st, key = pid[1], str(pid[2])
        dtype = st.dtype if isinstance(st, (_StorageType, _Dtype)) else np.uint8
        cached = self._storages.get(key)
        if cached is None or cached.dtype != dtype:
            cached = _Storage(self._zf, self._prefix, key, dtype, self._byteorder)
            self._storages[key] = cached
        return cached


def _find_data_pkl(zf):
    names = [n for n in zf.namelist() if n == "data.pkl" or n.endswith("/data.pkl")]
    if not names:
        return None, None
    name = min(names, key=len)
    return name, name[: -len("data.pkl")]


def load_pth(path_or_bytes):
    """The object graph of a PyTorch zip checkpoint with every tensor as a
    numpy array (the reference's ``torch_compat.load_pth``)."""
    src = io.BytesIO(path_or_bytes) if isinstance(path_or_bytes, (bytes, bytearray)) else os.fspath(path_or_bytes)
    try:
        zf = zipfile.ZipFile(src, "r")
    except FileNotFoundError:
        raise CheckpointError(f"no such file: {path_or_bytes}") from None
    except zipfile.BadZipFile:
        raise CheckpointError("not a PyTorch zip checkpoint (legacy torch.save files without "
                              "_use_new_zipfile_serialization are not read)") from None
    with zf:
        name, prefix = _find_data_pkl(zf)
        if name is None:
            raise CheckpointError("archive has no data.pkl: not a PyTorch >= 1.6 checkpoint")
        byteorder = "little"
        if f"{prefix}byteorder" in zf.namelist():
            byteorder = zf.read(f"{prefix}byteorder").decode("ascii", "replace").strip() or "little"
        try:
            return _Unpickler(zf.read(name), zf, prefix, byteorder).load()
        except CheckpointError:
            raise
        except Exception as e:  # noqa: BLE001
            raise CheckpointError(f"cannot read {name}: {type(e).__name__}: {e}") from e


def synthesizer_weights(obj):
    """``(weights, config)`` from a loaded synthesizer checkpoint, with the
    layout rules of ``runtime/models/vits.py:2247-2262``; weights are float32
    arrays keyed like the checkpoint, config the ``config`` list or None."""
    w, cfg = None, None
    if isinstance(obj, dict):
        if isinstance(obj.get("weight"), dict):
            w = obj["weight"]
            cfg = obj.get("config")
        elif isinstance(obj.get("model"), dict):
            w = obj["model"]
    if w is None:
        w = obj
    if not isinstance(w, dict):
        raise CheckpointError("checkpoint holds no state dict")
    out = {}
    for k, v in w.items():
        if isinstance(v, np.ndarray):
            out[str(k)] = np.asarray(v, dtype=np.float32, order="C")
    if cfg is not None:
        cfg = [c.tolist() if isinstance(c, np.ndarray) else c for c in cfg]
    return out, cfg


def load_synthesizer(path, sr=None, ctx=None, precision=0):
    """A device-resident ``HipSynthesizer`` from an RVC ``.pth`` file
    (``SynthesizerTrn(checkpoint_path)``, ``runtime/models/vits.py:2245``)."""
    from .synth import HipSynthesizer

    w, cfg = synthesizer_weights(load_pth(path))
    return HipSynthesizer(w, config=cfg, sr=sr, ctx=ctx, precision=precision)


def hubert_state_dict(obj):
    """Float32 state dict of a loaded ``pytorch_model.bin`` (transformers key
    names, as ``runtime/models/hubert.py:499-505`` reads them)."""
    sd = obj.get("state_dict", obj) if isinstance(obj, dict) else obj
    if not isinstance(sd, dict):
        raise CheckpointError("checkpoint holds no state dict")
    return {str(k): np.asarray(v, dtype=np.float32, order="C") for k, v in sd.items() if isinstance(v, np.ndarray)}


def load_hubert(path, ctx=None):
    """A device-resident ``HipHubert`` from ``pytorch_model.bin`` (a file, or
    a directory holding it, like ``HubertEncoder(model_dir)``)."""
    from .hubert import HipHubert

    p = os.fspath(path)
    if os.path.isdir(p):
        p = os.path.join(p, "pytorch_model.bin")
    return HipHubert(hubert_state_dict(load_pth(p)), ctx=ctx)


def rmvpe_state_dict(obj):
    """Float32 state dict of a loaded ``rmvpe.pt`` (fp16 storage cast to
    float32 as ``runtime/models/rmvpe.py:557-563`` does; the integer
    ``num_batches_tracked`` counters are dropped)."""
    sd = obj.get("state_dict", obj.get("model", obj)) if isinstance(obj, dict) else obj
    if not isinstance(sd, dict):
        raise CheckpointError("checkpoint holds no state dict")
    return {str(k): np.asarray(v, dtype=np.float32, order="C") for k, v in sd.items()
            if isinstance(v, np.ndarray) and not str(k).endswith("num_batches_tracked")}


def load_rmvpe(path, ctx=None):
    """A device-resident ``HipRMVPE`` from ``rmvpe.pt`` (``load_rmvpe``,
    ``runtime/models/rmvpe.py:955-966``, with the path given)."""
    from .rmvpe import HipRMVPE

    return HipRMVPE(rmvpe_state_dict(load_pth(os.fspath(path))), ctx=ctx)
