"""Gradient mode: ``no_grad`` / ``enable_grad`` / ``is_grad_enabled``, the switches of
NimbleML/utils/grad_mode.py:1-35. ``GPT.compute_loss`` keeps the activations its backward
needs only while gradients are enabled and some parameter requires them."""
from __future__ import annotations

from contextlib import contextmanager

_state = {"enabled": True}


def is_grad_enabled() -> bool:
    return _state["enabled"]


@contextmanager
def _mode(enabled: bool):
    prev = _state["enabled"]
    _state["enabled"] = enabled
    try:
        yield
    finally:
        _state["enabled"] = prev


def no_grad():
    """Disable gradient tracking inside the ``with`` block."""
    return _mode(False)


def enable_grad():
    """Enable gradient tracking inside the ``with`` block."""
    return _mode(True)
