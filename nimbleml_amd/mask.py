"""Additive attention masks (NimbleML/utils/mask.py:8-27).

``causal_mask_tensor(seq_len)`` is the (seq_len, seq_len) no-grad Tensor with −inf above the
diagonal and 0 elsewhere, in the compute dtype, cached per (seq_len, dtype);
``make_causal_mask`` returns its array. Passed to a module, this mask selects the causal
attention kernels (the modules compare a given mask with it), exactly as ``mask=None``
does for the fused block and trunk."""
from __future__ import annotations

from functools import lru_cache

import numpy as np

from nimbleml_amd import np_backend
from nimbleml_amd.tensor import Tensor


@lru_cache(maxsize=64)
def _causal_mask_cached(seq_len: int, dtype_name: str) -> Tensor:
    arr = np.triu(np.full((seq_len, seq_len), -np.inf, dtype=np.dtype(dtype_name)), k=1)
    return Tensor(arr, arr.shape, requires_grad=False)


def causal_mask_tensor(seq_len: int) -> Tensor:
    """The cached causal mask Tensor of the current compute dtype."""
    return _causal_mask_cached(int(seq_len), np.dtype(np_backend.dtype).name)


def make_causal_mask(seq_len: int) -> np.ndarray:
    """The causal mask as a (seq_len, seq_len) array."""
    t = causal_mask_tensor(seq_len)
    return np.asarray(t.data).reshape(t.shape)
