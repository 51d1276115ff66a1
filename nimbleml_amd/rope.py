"""Rotary position tables (GPT(use_rope=True)): the reference's float32 cos/sin cache
(utils/rope.py:12-19, GPT-NeoX half split) built with the same NumPy operations, so the
tables the device uses are the reference's bit for bit. The rotation itself runs on the
device (rope_kernel in csrc/ops_basic.hip)."""
from __future__ import annotations

import numpy as np


def build_rope_cache(seq_len: int, head_dim: int, base: float = 10000.0):
    """``(cos, sin)``, each ``(seq_len, head_dim)`` float32; both halves of a row hold
    the same ``position · θ_i`` with ``θ_i = base^(-i / (head_dim/2))``."""
    half = head_dim // 2
    theta = 1.0 / (base ** (np.arange(0, half, dtype=np.float32) / float(half)))
    angle = np.outer(np.arange(seq_len, dtype=np.float32), theta)
    angle = np.concatenate([angle, angle], axis=-1)
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32)
