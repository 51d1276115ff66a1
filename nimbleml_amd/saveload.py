"""Weights-only checkpoints in the reference's .npz format (utils/saveload.py:16-41,
:265-300): the same parameter names, the same mismatch errors. Loading marks the
model's device copy stale; the next device call re-uploads it."""
from __future__ import annotations

import numpy as np

from nimbleml_amd.layers import Module, Sequential
from nimbleml_amd.tensor import Tensor


def named_parameters(module, prefix=""):
    """Yield (name, Tensor) for every learnable parameter (saveload.py:16-41)."""
    if isinstance(module, Sequential):
        for i, layer in enumerate(module.layers):
            child_prefix = f"{prefix}.layers.{i}" if prefix else f"layers.{i}"
            yield from named_parameters(layer, child_prefix)
        return
    if not isinstance(module, Module):
        return
    for name, value in vars(module).items():
        if name.startswith("_"):
            continue
        child_prefix = f"{prefix}.{name}" if prefix else name
        if isinstance(value, Tensor):
            if value.requires_grad:
                yield child_prefix, value
        elif isinstance(value, Module):
            yield from named_parameters(value, child_prefix)
        elif isinstance(value, (list, tuple)):
            for i, item in enumerate(value):
                if isinstance(item, Module):
                    yield from named_parameters(item, f"{child_prefix}.{i}")


def _mark_stale(model):
    if hasattr(model, "_invalidate_device"):
        model._invalidate_device()


def save(model, path):
    state = {name: np.asarray(p.data).reshape(p.shape) for name, p in named_parameters(model)}
    if not state:
        raise ValueError("Model has no parameters to save.")
    np.savez(path, **state)


def load_arrays(model, arrays):
    """Set every parameter from a ``{name: array}`` mapping (same checks as ``load``)."""
    expected = dict(named_parameters(model))
    if not expected:
        raise ValueError("Model has no parameters to load.")
    names, expected_names = set(arrays), set(expected)
    if names != expected_names:
        parts = []
        missing = sorted(expected_names - names)
        extra = sorted(names - expected_names)
        if missing:
            parts.append(f"missing {missing}")
        if extra:
            parts.append(f"unexpected {extra}")
        raise ValueError(f"Checkpoint mismatch: {', '.join(parts)}")
    for name, param in expected.items():
        loaded = np.asarray(arrays[name], dtype=param.data.dtype)
        if loaded.size != param.size:
            raise ValueError(f"Shape mismatch for {name}: expected {param.shape}, got {loaded.shape}")
        param.data[...] = loaded.ravel()
    _mark_stale(model)
    return model


def load(model, path):
    """Load parameters from .npz into an existing model (same architecture)."""
    with np.load(path) as data:
        if "_checkpoint_meta" in data.files:
            raise ValueError("File is a training checkpoint; use load_checkpoint() instead of load().")
        return load_arrays(model, {k: data[k] for k in data.files})
