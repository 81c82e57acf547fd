"""ctypes binding of libcobra_amd.so (the C ABI declared in include/cobra_amd.h).

The library is loaded once, after ``torch`` (so both share the HIP runtime
that torch loaded), from this package directory only.  There is no fallback:
if the library is missing or cannot be loaded, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcobra_amd.so")
ABI_VERSION = 11

F16 = 0
F32 = 1
BF16 = 2
PLAN_FUSED = 0
PLAN_STAGED = 1
PLAN_PADDED = 2
# Epilogue / row-mask flags (COBRA_EPI_* in include/cobra_amd.h).
EPI_GELU = 1
EPI_MASK_BRANCH = 2
EPI_MASK_RESID = 4
EPI_MASK_OUT = 8

_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/cobra_amd.h one to one.
SIGNATURES = {
    "cobra_version": (_c_int, []),
    "cobra_error_string": (ctypes.c_char_p, [_c_int]),
    "cobra_ln_fwd": (
        _c_int, [_vp, _c_int, _vp, _c_int, _vp, _vp, _vp, _c_int, _vp, _vp, _c_int, _c_i64, _c_i64, _c_f32, _vp],
    ),
    "cobra_ln_fwd_strided": (
        _c_int,
        [_vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _vp, _c_int, _vp, _c_i64, _vp, _c_int, _c_i64, _c_i64,
         _c_i64, _c_f32, _vp],
    ),
    "cobra_linear_fwd": (
        _c_int, [_vp, _vp, _c_int, _vp, _vp, _c_int, _vp, _c_int, _vp, _c_int, _c_i64, _c_i64, _c_i64, _vp],
    ),
    "cobra_linear_ln_fwd": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _vp, _vp, _vp, _vp, _c_int, _c_i64, _c_i64, _c_i64, _c_f32,
         _vp],
    ),
    "cobra_ln_linear_fwd": (
        _c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_f32, _vp],
    ),
    "cobra_mask_bits": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "cobra_attn_fwd": (_c_int, [_vp, _vp, _c_int, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _c_int, _vp]),
    "cobra_qkv_attn_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "cobra_qkv_attn_fwd": (
        _c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _c_int, _vp],
    ),
    "cobra_layer_plan": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "cobra_layer_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "cobra_layer_fwd": (
        _c_int,
        [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_f32, _vp],
    ),
    "cobra_layer_bind": (
        _vp,
        [_c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_f32],
    ),
    "cobra_layer_run": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "cobra_layer_unbind": (None, [_vp]),
    "cobra_block_plan": (_c_int, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "cobra_block_fwd": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_f32, _vp],
    ),
    "cobra_layer_fwd_noalloc": (
        _c_int,
        [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_f32, _vp],
    ),
}

# COBRA_NOALLOC_MAX_BYTES: the device scratch of cobra_layer_fwd_noalloc.
NOALLOC_MAX_BYTES = 128 << 20

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


class CobraError(RuntimeError):
    """A C-ABI call returned a non-zero hipError_t code."""

    def __init__(self, fn: str, code: int, msg: str) -> None:
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.fn = fn
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it first (__graft_entry__.build() or "
                    "python -m cobra_amd.build); there is no non-HIP fallback"
                )
            handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            ver = handle.cobra_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


_host = None


def host():
    """The host-side companion module (``cobra_host.so``: the sublayer's native
    steady-state call), loaded after the C-ABI library it links; raises if missing."""
    global _host
    if _host is None:
        lib()
        path = os.path.join(os.path.dirname(LIB_PATH), "cobra_host.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it first (__graft_entry__.build() or "
                               "python -m cobra_amd.build)")
        import importlib.util

        spec = importlib.util.spec_from_file_location("cobra_amd.cobra_host", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _host = mod
    return _host


def check(fn: str, code: int) -> None:
    if code != 0:
        msg = lib().cobra_error_string(code)
        raise CobraError(fn, code, msg.decode() if msg else "?")


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))
