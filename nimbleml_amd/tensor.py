"""The ``Tensor`` surface the GPT path uses (NimbleML/utils/tensor.py:133-241).

A flat buffer plus a shape. Float data is coerced to the compute dtype
(tensor.py:147-153); ``from_int64`` keeps token ids as int64 (tensor.py:194-214).
``data`` is a host ``numpy.ndarray`` for parameters and inputs, or a
``DeviceArray`` for results left on the GPU (logits); ``np.asarray(t.data)``
works for both.

Autograd (tensor.py:271-352 for ``zero_grad``, ``backward`` and ``_accumulate_grad``):
each result that needs gradients holds a ``_backward`` closure and its input Tensors in
``_prev``; ``backward`` seeds this tensor's ``grad`` and runs the closures of the graph
below it in reverse topological order (tensor.py:286-332 with the post-order walk of
tensor.py:88-121). The closures are the GPT loss's (``GPT.compute_loss``) and the
modules' (``nimbleml_amd.layers``); each runs its backward on the device and adds the
gradients to its parameters' and inputs' ``grad``.
"""
from __future__ import annotations

from math import prod

import numpy as np

from nimbleml_amd import np_backend
from nimbleml_amd._native import DeviceArray


class Tensor:
    def __init__(self, data, shape, requires_grad=False, _children=(), _op=""):
        if isinstance(data, DeviceArray):
            self.data = data.reshape(-1)
        elif isinstance(data, (int, float)):
            self.data = np.array([float(data)], dtype=np_backend.dtype)
        else:
            self.data = np.asarray(data, dtype=np_backend.dtype).ravel()
        self.shape = tuple(shape)
        self.requires_grad = requires_grad
        self.grad = None
        self._op = _op
        self._prev = set(_children)
        self._backward = None
        self._version = 0  # bumped when the values change (device copies key on it)

    @classmethod
    def from_int64(cls, data, shape):
        obj = cls.__new__(cls)
        if isinstance(data, DeviceArray):
            obj.data = data.reshape(-1)
        else:
            obj.data = np.asarray(data, dtype=np.int64).reshape(-1)
        obj.shape = tuple(shape)
        obj.requires_grad = False
        obj.grad = None
        obj._op = ""
        obj._prev = set()
        obj._backward = None
        obj._version = 0
        return obj

    def _bump_version(self):
        """Mark the values changed: device copies made from the old values are rebuilt."""
        self._version += 1

    @property
    def ndim(self):
        return len(self.shape)

    @property
    def size(self):
        return prod(self.shape) if self.shape else 1

    @property
    def dtype(self):
        return self.data.dtype

    def _view(self, shape=None):
        if shape is None:
            shape = self.shape
        return self.data.reshape(shape) if shape else self.data.reshape(())

    def numpy(self) -> np.ndarray:
        return np.asarray(self.data).reshape(self.shape)

    def item(self) -> float:
        return float(np.asarray(self.data).reshape(-1)[0])

    # ------------------------------------------------------------------ autograd
    def zero_grad(self, set_to_none: bool = False):
        """tensor.py:271-279."""
        if set_to_none:
            self.grad = None
        else:
            gdt = getattr(self, "_grad_dtype", None) or np_backend.dtype
            self.grad = np.zeros(self.size, dtype=gdt)

    def _accumulate_grad(self, grad):
        """tensor.py:334-352: add ``grad`` (flattened) into ``self.grad``, in the compute dtype
        or the wider ``_grad_dtype`` an optimizer pins under fp16 (optimizers/optimizer.py:33-38)."""
        if not self.requires_grad:
            return
        gdt = getattr(self, "_grad_dtype", None) or np_backend.dtype
        grad = np.asarray(grad).reshape(-1).astype(gdt, copy=False)
        if self.grad is None:
            self.grad = grad.copy()
        else:
            self.grad = self.grad + grad

    def backward(self, grad=None, retain_graph=False):
        """tensor.py:286-332: add ``grad`` (default 1 for a scalar) to this tensor's ``grad``,
        then run every ``_backward`` closure of the graph below it, each after all the
        closures of the tensors computed from it. Unless ``retain_graph``, the closures and
        edges are released afterwards."""
        if grad is None:
            if self.size != 1:
                raise ValueError("grad must be specified for non-scalar tensors.")
            grad = np.array([1.0], dtype=np_backend.dtype)
        elif isinstance(grad, (int, float)):
            grad = np.array([float(grad)], dtype=np_backend.dtype)
        elif isinstance(grad, Tensor):
            grad = np.asarray(grad.data)
        else:
            grad = np.asarray(grad, dtype=np_backend.dtype)
        self._accumulate_grad(grad)
        topo = _backward_order(self)
        for node in reversed(topo):
            fn = node._backward
            if fn is not None:
                fn()
        if not retain_graph:
            for node in topo:
                node._backward = None
                node._prev = set()

    def __repr__(self):
        return f"Tensor(shape={self.shape}, data={self.data})"


def _backward_order(root):
    """The tensors reachable from ``root`` through ``_prev``, each after all of its inputs
    (an iterative post-order walk, tensor.py:88-121)."""
    order, visited, stack = [], set(), [(root, False)]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            order.append(node)
            continue
        if id(node) in visited:
            continue
        visited.add(id(node))
        stack.append((node, True))
        for child in node._prev:
            if id(child) not in visited:
                stack.append((child, False))
    return order
