"""Device and dtype selection — the ``hip`` device of NimbleML's array backend.

Mirrors NimbleML/utils/np_backend.py (`device`, `using_gpu`, `dtype`, `set_device`,
`set_dtype`, `get_dtype`, `sync_device`, `as_label_indices`) for this path. The
only compute device here is ``hip`` (one MI355X per process); ``NIMBLEML_DEVICE``
values ``auto``, ``gpu``, ``cuda`` and ``hip`` all select it. ``cpu`` is refused:
this package has no CPU execution path. The compute dtype comes from
``NIMBLEML_DTYPE`` (``float32`` default, ``float16``), read at import like the
reference (np_backend.py:157-176), and is frozen into each model on construction.
"""
from __future__ import annotations

import os

import numpy as np

_DEVICE_PREFERENCE = os.environ.get("NIMBLEML_DEVICE", "auto").strip().lower()


def _resolve_device(name: str) -> str:
    name = name.strip().lower()
    if name in ("auto", "gpu", "cuda", "hip"):
        return "hip"
    if name == "cpu":
        raise ValueError(
            "nimbleml_amd runs on the HIP device only (NIMBLEML_DEVICE=hip); "
            "the CPU path is the reference NimbleML itself.")
    raise ValueError("device must be 'auto', 'gpu', 'cuda' or 'hip'")


device = _resolve_device(_DEVICE_PREFERENCE)
using_gpu = True


def _resolve_dtype(name):
    if isinstance(name, np.dtype) or isinstance(name, type):
        name = np.dtype(name).name
    name = str(name).strip().lower()
    if name in ("float16", "f16", "half"):
        return np.float16
    if name in ("float32", "f32", "single"):
        return np.float32
    if name in ("bfloat16", "bf16", "float64", "f64", "double"):
        raise ValueError(f"dtype {name!r} is not supported on the HIP path (float16 or float32)")
    raise ValueError("dtype must be 'float16' or 'float32'")


dtype = _resolve_dtype(os.environ.get("NIMBLEML_DTYPE", "float32"))


def get_dtype():
    return dtype


def set_dtype(name):
    """Set the global compute dtype for models constructed afterwards."""
    global dtype
    dtype = _resolve_dtype(name)
    os.environ["NIMBLEML_DTYPE"] = np.dtype(dtype).name
    return dtype


def set_device(name):
    global device
    device = _resolve_device(name)
    os.environ["NIMBLEML_DEVICE"] = device
    return device


def sync_device() -> None:
    """Block until queued device work finishes (np_backend.py:118-126)."""
    from nimbleml_amd import _native

    _native.synchronize()


def as_label_indices(label_indices, *, batch_size: int) -> np.ndarray:
    """int64 labels of length ``batch_size`` (np_backend.py:193-208)."""
    if not hasattr(label_indices, "dtype") and hasattr(label_indices, "data"):
        label_indices = label_indices.data
    labels = np.asarray(label_indices, dtype=np.int64).reshape(-1)
    if labels.size != batch_size:
        raise ValueError(f"label count ({labels.size}) must match batch size ({batch_size}).")
    return labels
