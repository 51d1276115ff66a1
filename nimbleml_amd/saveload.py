"""Checkpoints in the reference's .npz formats (utils/saveload.py): weights-only
``save``/``load`` (:265-300) and training checkpoints ``save_checkpoint``/``load_checkpoint``
(:303-358) with the Adam/AdamW state, under the same names, keys and errors. Saving first
copies device-trained parameters back to the host (``GPT.sync_to_host``); loading marks
the model's device copy stale, and the next device call re-uploads it."""
from __future__ import annotations

import json

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


def _sync(model):
    if hasattr(model, "sync_to_host"):
        model.sync_to_host()


def save(model, path):
    """Save all learnable parameters to a .npz archive (saveload.py:265-270)."""
    _sync(model)
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
        param._bump_version()
    _mark_stale(model)
    return model


def load(model, path):
    """Load parameters from .npz into an existing model (same architecture)."""
    with np.load(path) as data:
        if "_checkpoint_meta" in data.files:
            raise ValueError("File is a training checkpoint; use load_checkpoint() instead of load().")
        return load_arrays(model, {k: data[k] for k in data.files})


_CHECKPOINT_VERSION = 1  # saveload.py:11-13
_META_KEY = "_checkpoint_meta"
_MODEL_PREFIX = "model/"


def _optimizer_state(optimizer):
    """(meta, arrays) of an Adam/AdamW (saveload.py:89-127): moments, and float32 masters of
    a float16 model, one flat array per parameter in ``optimizer.params`` order."""
    from nimbleml_amd.optim import Adam

    if not isinstance(optimizer, Adam):
        raise TypeError(f"Unsupported optimizer type for checkpoint: {type(optimizer).__name__}")
    groups = []
    for g in optimizer.param_groups:
        entry = {"lr": float(g["lr"])}
        if "weight_decay" in g:
            entry["weight_decay"] = float(g["weight_decay"])
        groups.append(entry)
    meta = {"class": type(optimizer).__name__, "param_groups": groups,
            "num_params": len(optimizer.params), "t": int(optimizer.t),
            "beta1": float(optimizer.beta1), "beta2": float(optimizer.beta2),
            "epsilon": float(optimizer.epsilon), "weight_decay": float(optimizer.weight_decay)}
    arrays = {}
    for i, (m, v) in enumerate(zip(optimizer.m, optimizer.v)):
        arrays[f"optimizer/m/{i}"] = m
        arrays[f"optimizer/v/{i}"] = v
    for i, master in enumerate(optimizer.masters):
        if master is not None:
            arrays[f"optimizer/master/{i}"] = master
    return meta, arrays


def _load_optimizer_state(optimizer, meta, data):
    """saveload.py:130-175 for Adam/AdamW."""
    cls = type(optimizer).__name__
    if meta["class"] != cls:
        raise ValueError(f"Optimizer class mismatch: checkpoint has {meta['class']!r}, model has {cls!r}")
    n = len(optimizer.params)
    if meta["num_params"] != n:
        raise ValueError(f"Optimizer parameter count mismatch: checkpoint has {meta['num_params']}, "
                         f"model has {n}")
    if len(optimizer.param_groups) != len(meta["param_groups"]):
        raise ValueError(f"Optimizer param group count mismatch: expected "
                         f"{len(optimizer.param_groups)}, got {len(meta['param_groups'])}")
    for group, saved in zip(optimizer.param_groups, meta["param_groups"]):
        group["lr"] = float(saved["lr"])
        if "weight_decay" in saved:
            group["weight_decay"] = float(saved["weight_decay"])
    optimizer.t = int(meta["t"])
    for key in ("beta1", "beta2", "epsilon", "weight_decay"):
        if float(getattr(optimizer, key)) != float(meta[key]):
            raise ValueError(f"Adam hyperparameter mismatch for {key}")
    sizes = [p.size for p in optimizer.params]

    def arr(kind, i):
        a = np.asarray(data[f"optimizer/{kind}/{i}"], dtype=np.float32).reshape(-1)
        if a.size != sizes[i]:
            raise ValueError(f"Array size mismatch: expected {sizes[i]}, got {a.size}")
        return a

    masters = [arr("master", i) if f"optimizer/master/{i}" in data.files else None
               for i in range(n)]
    optimizer._load_state([arr("m", i) for i in range(n)], [arr("v", i) for i in range(n)],
                          masters)


def save_checkpoint(path, model, optimizer=None, scheduler=None, *, step=None, extra=None):
    """Model weights plus optimizer state for resuming (saveload.py:303-326)."""
    if scheduler is not None:
        raise NotImplementedError("learning-rate schedulers are not part of this package")
    _sync(model)
    arrays = {f"{_MODEL_PREFIX}{name}": np.asarray(p.data).reshape(p.shape)
              for name, p in named_parameters(model)}
    if not arrays:
        raise ValueError("Model has no parameters to save.")
    meta = {"version": _CHECKPOINT_VERSION, "step": step, "extra": extra or {}}
    if optimizer is not None:
        opt_meta, opt_arrays = _optimizer_state(optimizer)
        meta["optimizer"] = opt_meta
        arrays.update(opt_arrays)
    arrays[_META_KEY] = np.array(json.dumps(meta))
    np.savez(path, **arrays)


def load_checkpoint(path, model, optimizer=None, scheduler=None):
    """Restore a checkpoint written by :func:`save_checkpoint` (saveload.py:329-358);
    returns ``{"step", "extra"}``."""
    if scheduler is not None:
        raise NotImplementedError("learning-rate schedulers are not part of this package")
    with np.load(path) as data:
        if _META_KEY not in data.files:
            raise ValueError("Not a training checkpoint (missing metadata); use load() for "
                             "weights-only files.")
        meta = json.loads(str(data[_META_KEY]))
        if meta.get("version") != _CHECKPOINT_VERSION:
            raise ValueError(f"Unsupported checkpoint version: {meta.get('version')}")
        expected = dict(named_parameters(model))
        prefixed = any(f"{_MODEL_PREFIX}{name}" in data.files for name in expected)
        arrays = {}
        for name in expected:  # saveload.py:248-262
            key = f"{_MODEL_PREFIX}{name}" if prefixed else name
            if key not in data.files:
                raise ValueError(f"Checkpoint missing parameter {name!r}")
            arrays[name] = data[key]
        if optimizer is not None and "optimizer" not in meta:
            raise ValueError("Checkpoint does not contain optimizer state.")
        load_arrays(model, arrays)
        if optimizer is not None:
            if hasattr(model, "_adam_stash"):
                model._adam_stash = None  # the checkpoint's state replaces the old one
            _load_optimizer_state(optimizer, meta["optimizer"], data)
        elif "optimizer" in meta:
            raise ValueError("Checkpoint contains optimizer state but no optimizer was provided.")
        if "scheduler" in meta:
            raise ValueError("Checkpoint contains scheduler state but no scheduler was provided.")
    return {"step": meta.get("step"), "extra": meta.get("extra") or {}}
