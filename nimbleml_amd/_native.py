"""ctypes binding of ``libnimbleml_hip.so`` (C-ABI in include/nimbleml_hip.h).

Plays the part of the reference's ``_native_loader`` (NimbleML/_native_loader.py:20-28):
the library is required — there is no Python or CPU fallback for the hot path —
so a missing build raises ImportError, and a missing GPU raises RuntimeError at
first use. Every C call returns a status; failures become ``RuntimeError`` with
the library's message (the reference raises RuntimeError from CUDA errors,
native/src/sdpa_cuda.cu:10-14), except messages the reference raises as
``ValueError`` (sequence length / token-id range), which keep that type.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("NIMBLEML_HIP_LIB", os.path.join(_PKG, "_lib", "libnimbleml_hip.so"))

_INSTALL_HINT = (
    "nimbleml_amd requires its HIP library (libnimbleml_hip.so). Build it with\n"
    "  python nimbleml_amd/build.py\n"
    "(hipcc for gfx950, ROCm 7)."
)

vp = C.c_void_p
sz = C.c_size_t
i32 = C.c_int
f32 = C.c_float
i64 = C.c_int64
PI32 = C.POINTER(C.c_int32)

# name: (argtypes) — every function returns int status.
_SIGS = {
    "nml_with_hip": [],
    "nml_hip_available": [C.POINTER(C.c_int)],
    "nml_init": [i32],
    "nml_get_stream": [C.POINTER(vp)],
    "nml_set_stream": [vp],
    "nml_device_info": [C.c_char_p, sz, C.POINTER(C.c_int), C.POINTER(sz)],
    "nml_malloc": [sz, C.POINTER(vp)],
    "nml_free": [vp],
    "nml_memcpy_h2d": [vp, vp, sz],
    "nml_memcpy_d2h": [vp, vp, sz],
    "nml_memcpy_d2d": [vp, vp, sz],
    "nml_memset": [vp, i32, sz],
    "nml_synchronize": [],
    "nml_event_create": [C.POINTER(vp)],
    "nml_event_record": [vp],
    "nml_event_elapsed_ms": [vp, vp, C.POINTER(f32)],
    "nml_event_destroy": [vp],
    "nml_rmsnorm_forward_device": [vp, vp, vp, vp, vp, sz, sz, f32, i32],
    "nml_gelu_forward_device": [vp, vp, vp, sz, i32],
    "nml_embedding_gather_device": [vp, vp, vp, vp, sz, sz, sz, sz, sz, vp, vp, i32],
    "nml_linear_device": [vp, sz, vp, vp, vp, vp, sz, sz, sz, i32, i32],
    "nml_flash_sdpa_forward_device": [vp, vp, vp, vp, vp, vp, sz, sz, sz, f32],
    "nml_flash_sdpa_backward_device": [vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, f32],
    "nml_rmsnorm_backward_device": [vp, vp, vp, vp, vp, vp, vp, sz, sz, f32],
    "nml_linear_backward_device": [vp, vp, vp, vp, vp, vp, sz, sz, sz, vp, i32],
    "nml_rmsnorm_backward_typed_device": [vp, vp, vp, vp, vp, sz, sz, f32, i32],
    "nml_embedding_backward_device": [vp, vp, vp, sz, sz, sz, i32],
    "nml_causal_attention_device": [vp, vp, vp, vp, sz, sz, sz, f32, i32],
    "nml_decode_attention_device": [vp, vp, vp, vp, vp, sz, sz, sz, sz, f32, vp, i32],
    "nml_sdpa_forward_device": [vp, vp, vp, vp, vp, sz, sz, sz, f32, i32, i32],
    "nml_tied_ce_forward_device": [vp, vp, vp, sz, sz, sz, i64, i32, C.POINTER(C.c_double), i32],
    "nml_tied_ce_forward_device_noalloc": [vp, vp, vp, sz, sz, sz, i64, i32,
                                           C.POINTER(C.c_double), i32],
    "nml_sample_device": [vp, sz, sz, f32, i32, f32, f32, vp, vp, sz, vp, vp, i32],
    "nml_adamw_step_device": [vp, vp, vp, vp, sz, f32, f32, f32, f32, f32, f32, f32],
    "nml_clip_grad_norm_device": [C.POINTER(vp), C.POINTER(sz), sz, f32, C.POINTER(f32)],
    "nml_model_create": [i32, i32, i32, i32, i32, i32, i32, C.POINTER(vp)],
    "nml_model_destroy": [vp],
    "nml_model_set_param": [vp, i32, i32, vp, sz],
    "nml_model_param_ptr": [vp, i32, i32, C.POINTER(vp)],
    "nml_model_forward": [vp, vp, sz, sz, vp, i32],
    "nml_model_blocks_forward": [vp, vp, vp, sz, sz, i32, i32, vp],
    "nml_model_mha_forward": [vp, i32, vp, vp, sz, sz, i32, vp],
    "nml_model_blocks_forward_train": [vp, vp, vp, sz, sz, i32, i32, vp],
    "nml_model_blocks_backward": [vp, vp, vp],
    "nml_model_mha_forward_train": [vp, i32, vp, vp, sz, sz, i32, vp],
    "nml_model_mha_backward": [vp, vp, vp],
    "nml_model_loss": [vp, vp, vp, sz, sz, i64, i32, C.POINTER(C.c_double)],
    "nml_model_zero_grad": [vp],
    "nml_model_grad_ptr": [vp, i32, i32, C.POINTER(C.c_void_p)],
    "nml_model_loss_train": [vp, vp, vp, sz, sz, i64, i32, C.POINTER(C.c_double)],
    "nml_model_backward": [vp, C.c_double],
    "nml_model_logits_backward": [vp, vp, sz, sz, vp],
    "nml_model_saved_generation": [vp, C.POINTER(C.c_ulonglong)],
    "nml_model_adamw_step": [vp, f32, f32, f32, f32, f32, f32, f32],
    "nml_model_adam_moments": [vp, i32, i32, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)],
    "nml_model_adam_state_init": [vp],
    "nml_model_adam_master": [vp, i32, i32, C.POINTER(C.c_void_p)],
    "nml_model_adamw_update": [vp, i32, i32, sz, sz, f32, f32, f32, f32, f32, f32, f32],
    "nml_cache_create": [vp, sz, C.POINTER(vp)],
    "nml_cache_destroy": [vp],
    "nml_cache_length": [vp, C.POINTER(sz)],
    "nml_model_forward_cached": [vp, vp, vp, sz, sz, vp, i32],
    "nml_model_prefill_ragged": [vp, vp, vp, sz, PI32, sz, vp],
    "nml_model_generate": [vp, vp, sz, PI32, sz, sz, f32, i32, f32, f32, vp, vp, sz, i32],
    "nml_model_last_decode_ms": [vp, C.POINTER(f32)],
    "nml_model_last_decode_path": [vp, C.POINTER(C.c_int)],
}

# Parameter kinds (enum nml_param_kind).
P_TOKEN_EMB, P_POS_EMB, P_LN_F = 0, 1, 2
P_ROPE_COS, P_ROPE_SIN = 3, 4
P_LN1, P_WQKV, P_BQKV, P_WO, P_BO, P_LN2, P_W1, P_B1, P_W2, P_B2 = range(10, 20)

F32, F16 = 0, 1

_lib = None
_lock = threading.Lock()
_initialised = False


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(_INSTALL_HINT)
    lib = C.CDLL(LIB_PATH)
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    lib.nml_last_error.argtypes = []
    lib.nml_last_error.restype = C.c_char_p
    _lib = lib
    return lib


lib = _load()


def exported_symbols():
    """Names of the C-ABI functions this binding expects the library to export."""
    return sorted(list(_SIGS) + ["nml_last_error"])


_VALUE_ERRORS = ("exceeds maximum sequence length", "out of range [0,", "must match batch size",
                 "must be divisible by")


def check(rc: int) -> None:
    if rc != 0:
        msg = (lib.nml_last_error() or b"unknown error").decode("utf-8", "replace")
        if any(s in msg for s in _VALUE_ERRORS):
            raise ValueError(msg)
        raise RuntimeError(msg)


def device_count() -> int:
    n = C.c_int(0)
    check(lib.nml_hip_available(C.byref(n)))
    return int(n.value)


def ensure_init(device: int = 0) -> None:
    """Select the GPU and create the library stream (once)."""
    global _initialised
    if _initialised:
        return
    with _lock:
        if _initialised:
            return
        if device_count() == 0:
            raise RuntimeError(
                "NIMBLEML_DEVICE=hip but no HIP device is visible; nimbleml_amd has no CPU path "
                "(use the reference NimbleML for CPU runs).")
        check(lib.nml_init(int(device)))
        _initialised = True


def synchronize() -> None:
    ensure_init()
    check(lib.nml_synchronize())


def device_info() -> dict:
    ensure_init()
    name = C.create_string_buffer(256)
    cus = C.c_int(0)
    mem = C.c_size_t(0)
    check(lib.nml_device_info(name, 256, C.byref(cus), C.byref(mem)))
    return {"name": name.value.decode(), "compute_units": cus.value, "total_mem": mem.value}


def np_dtype_code(dt) -> int:
    dt = np.dtype(dt)
    if dt == np.float32:
        return F32
    if dt == np.float16:
        return F16
    raise ValueError(f"unsupported dtype {dt} (float32 or float16)")


# Host-to-device copies made by this binding (calls, bytes): DeviceArray.from_host and the
# parameter uploads of device models. Tests read it to check what a call re-uploads.
h2d_stats = {"calls": 0, "bytes": 0}


def count_h2d(nbytes: int) -> None:
    h2d_stats["calls"] += 1
    h2d_stats["bytes"] += int(nbytes)


class DeviceArray:
    """A contiguous device buffer with a NumPy dtype and shape.

    ``np.asarray(dev)`` copies it to the host, so code written for the reference's
    ``np.asarray(tensor.data)`` keeps working on device results.
    """

    __slots__ = ("ptr", "shape", "dtype", "nbytes", "_owner", "__weakref__")

    def __init__(self, shape, dtype, ptr=None, owner=None):
        ensure_init()
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        if ptr is None:
            p = vp()
            check(lib.nml_malloc(max(self.nbytes, 1), C.byref(p)))
            self.ptr = p.value
            self._owner = None
        else:
            self.ptr = ptr
            self._owner = owner if owner is not None else self

    @classmethod
    def from_host(cls, arr, dtype=None):
        a = np.ascontiguousarray(arr if dtype is None else np.asarray(arr, dtype=dtype))
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(lib.nml_memcpy_h2d(d.ptr, a.ctypes.data, a.nbytes))
            count_h2d(a.nbytes)
        return d

    @property
    def ndim(self):
        return len(self.shape)

    @property
    def size(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            check(lib.nml_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    get = numpy  # CuPy-style host copy, as the reference's `.get()` probes expect

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a if dtype is None else a.astype(dtype, copy=False)

    def reshape(self, *shape):
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if -1 in shape:
            known = int(np.prod([s for s in shape if s != -1], dtype=np.int64))
            shape[shape.index(-1)] = self.size // max(known, 1)
        if int(np.prod(shape, dtype=np.int64)) != self.size:
            raise ValueError(f"cannot reshape {self.shape} to {tuple(shape)}")
        return DeviceArray(shape, self.dtype, ptr=self.ptr, owner=self._owner or self)

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype})"

    def __del__(self):
        if getattr(self, "_owner", 1) is None and getattr(self, "ptr", None) and lib is not None:
            try:
                lib.nml_free(self.ptr)
            except Exception:
                pass
            self.ptr = None


def ptr(x) -> int | None:
    """Device pointer of a DeviceArray (None passes through)."""
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    raise TypeError(f"expected a DeviceArray, got {type(x).__name__}")


class Timer:
    """HIP events on the library stream."""

    def __init__(self):
        ensure_init()
        self._a, self._b = vp(), vp()
        check(lib.nml_event_create(C.byref(self._a)))
        check(lib.nml_event_create(C.byref(self._b)))

    def start(self):
        check(lib.nml_event_record(self._a))

    def stop(self) -> float:
        check(lib.nml_event_record(self._b))
        ms = f32(0)
        check(lib.nml_event_elapsed_ms(self._a, self._b, C.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            lib.nml_event_destroy(self._a)
            lib.nml_event_destroy(self._b)
        except Exception:
            pass
