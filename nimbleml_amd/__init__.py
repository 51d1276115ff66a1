"""nimbleml_amd — NimbleML's GPT token loop, native to the MI355X (gfx950).

The same user-facing API as the reference for this path — ``GPT`` (forward,
``compute_loss``, ``forward_with_cache``, ``generate``), ``generate``, ``Tensor``,
``save``/``load`` — executed by hand-written HIP kernels through the C-ABI in
include/nimbleml_hip.h. Importing requires the built library
(``python nimbleml_amd/build.py``); there is no CPU fallback.
"""
from nimbleml_amd import np_backend
from nimbleml_amd._native import DeviceArray
from nimbleml_amd.generate import generate
from nimbleml_amd.grad_mode import enable_grad, is_grad_enabled, no_grad
from nimbleml_amd.gpt import GPT, KVCache
from nimbleml_amd.layers import (Dense, Embedding, FeedForward, FusedGPTTrunk,
                                 FusedTransformerBlock, Module, MultiHeadAttention, RMSNorm,
                                 Sequential, TransformerBlock)
from nimbleml_amd.mask import causal_mask_tensor, make_causal_mask
from nimbleml_amd.np_backend import device, set_device, set_dtype, using_gpu
from nimbleml_amd.optim import Adam, AdamW
from nimbleml_amd.saveload import (load, load_arrays, load_checkpoint, named_parameters, save,
                                   save_checkpoint)
from nimbleml_amd.tensor import Tensor

__all__ = [
    "GPT", "KVCache", "generate", "Tensor", "DeviceArray", "Dense", "Embedding", "RMSNorm",
    "MultiHeadAttention", "FeedForward", "FusedTransformerBlock", "FusedGPTTrunk",
    "TransformerBlock", "Module",
    "Sequential", "save", "load", "load_arrays", "named_parameters", "save_checkpoint",
    "load_checkpoint", "Adam", "AdamW", "device", "using_gpu",
    "set_device", "set_dtype", "np_backend", "no_grad", "enable_grad", "is_grad_enabled",
    "causal_mask_tensor", "make_causal_mask",
]
