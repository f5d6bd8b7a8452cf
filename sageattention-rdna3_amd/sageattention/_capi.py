"""ctypes binding of the C ABI declared in include/sageattn_mi355x.h.

The library ``libsage_mi355x.so`` is built in-tree next to this file by
``sageattention-rdna3_amd/build.py`` (or the path in ``SAGEATTN_MI355X_LIB``).
Loading happens after ``import torch`` so the library binds to the HIP runtime
torch already loaded (both carry the soname libamdhip64.so.7).  There is no
fallback: when the library is missing every native call raises RuntimeError,
like the reference's ``_get_native_ops`` (sageattention/core.py:22-37).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime first)

LIB_NAME = "libsage_mi355x.so"
ABI_VERSION = 2
MAX_KV_SPLITS = 16

DTYPE_F16 = 0
DTYPE_BF16 = 1

OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_ALIGNMENT = -3
ERR_HIP = -4

_STATUS_NAMES = {
    ERR_INVALID_ARG: "SAGE_ERR_INVALID_ARG",
    ERR_UNSUPPORTED: "SAGE_ERR_UNSUPPORTED",
    ERR_ALIGNMENT: "SAGE_ERR_ALIGNMENT",
    ERR_HIP: "SAGE_ERR_HIP",
}

# Every exported symbol with its ctypes signature (restype, argtypes).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
SIGNATURES = {
    "sage_abi_version": (ctypes.c_int, []),
    "sage_last_error": (ctypes.c_char_p, []),
    "sage_k_mean_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "sage_k_mean": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "sage_quant_qk_i8": (_I, [_P, _P, _P, _P, _P, _P, _P, _I,
                              _I64, _I64, _I64, _I64, _I64, _I64,
                              _I64, _I64, _I64, _I64, _I64, _I64,
                              ctypes.c_double, _P]),
    "sage_prep_kv_i8": (_I, [_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64,
                             _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "sage_prep_kv_i8_smooth": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64,
                                    _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "sage_v_layout_padded_len": (_I64, [_I64]),
    "sage_v_layout": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "sage_attn_i8_fwd": (_I, [_P, _P, _P, _P, _P, _P, _I,
                              _I64, _I64, _I64, _I64, _I64, _I64,
                              _I64, _I64, _I64, _I, _P]),
    "sage_attn_i8_fwd_lse": (_I, [_P, _P, _P, _P, _P, _P, _P, _I,
                                  _I64, _I64, _I64, _I64, _I64, _I64,
                                  _I64, _I64, _I64, _I, _P]),
    "sage_attn_i8_fwd_qfused": (_I, [_P, _P, _P, _P, _P, _P, _I,
                                     _I64, _I64, _I64, _I64, _I64, _I64,
                                     _I64, _I64, _I64, _I64, _I64, _I64,
                                     _I, ctypes.c_double, _I, _P, _I64, _P]),
    "sage_attn_i8_fwd_qfused_vrows": (_I, [_P, _P, _P, _P, _P, _P, _I,
                                           _I64, _I64, _I64, _I64, _I64, _I64,
                                           _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                           _I, ctypes.c_double, _I, _P, _I64, _P]),
    "sage_attn_i8_fwd_qfused_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I,
                                             _I64, _I64, _I64, _I64, _I64, _I64,
                                             _I64, _I64, _I64, _I64, _I64, _I64,
                                             _I, ctypes.c_double, _I, _P]),
    "sage_attn_direct_fwd": (_I, [_P, _P, _P, _P, _P, _I,
                                  _I64, _I64, _I64, _I64, _I64, _I64,
                                  _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                  _I, ctypes.c_double, _I, _P, _I64, _P]),
    "sage_attn_direct_fwd_vrows": (_I, [_P, _P, _P, _P, _P, _I,
                                        _I64, _I64, _I64, _I64, _I64, _I64,
                                        _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                        _I, ctypes.c_double, _I, _P, _I64, _P]),
    "sage_attn_workspace_bytes": (_I64, [_I, _I64, _I64, _I64, _I64, _I64, _I, _I]),
    "sage_attn_split_plan": (_I, [_I, _I64, _I64, _I64, _I64, _I64, _I, _I, _P, _P]),
}


class SageError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, func: str, code: int, message: str):
        self.func = func
        self.code = code
        super().__init__(f"{func} failed with {_STATUS_NAMES.get(code, code)}: {message}")


_lib = None
_lib_error = None
_lock = threading.Lock()


def library_path() -> str:
    env = os.environ.get("SAGEATTN_MI355X_LIB")
    if env:
        return env
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def load():
    """Load (once) and return the ctypes library; raise RuntimeError if unavailable."""
    global _lib, _lib_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        try:
            lib = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            ver = lib.sage_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"ABI version {ver} != expected {ABI_VERSION}")
        except Exception as e:  # noqa: BLE001 - re-raised with context below
            _lib_error = e
            raise RuntimeError(
                "sageattention native library (libsage_mi355x.so) is not available. "
                "Build it with:\n  python sageattention-rdna3_amd/build.py\n"
                f"on a system with ROCm/hipcc (target gfx950). Path tried: {path}\n"
                f"Original error: {e}"
            ) from e
        _lib = lib
        return lib


def check(func: str, rc: int) -> None:
    if rc != OK:
        msg = _lib.sage_last_error() if _lib is not None else b""
        raise SageError(func, rc, (msg or b"").decode(errors="replace"))


def call(func: str, *args) -> None:
    lib = load()
    check(func, getattr(lib, func)(*args))


def split_plan(quantized: bool, batch: int, q_heads: int, q_len: int, kv_len: int, head_dim: int,
               is_causal: bool, num_splits: int = 0):
    """(whole q-blocks, splits of the others) that such a launch runs on the current device."""
    whole, splits = ctypes.c_int64(0), ctypes.c_int(0)
    call("sage_attn_split_plan", int(quantized), batch, q_heads, q_len, kv_len, head_dim, int(bool(is_causal)),
         int(num_splits), ctypes.byref(whole), ctypes.byref(splits))
    return whole.value, splits.value


def query(func: str, *args) -> int:
    """Call a size query (non-negative result, or a negative status raised as SageError)."""
    lib = load()
    v = getattr(lib, func)(*args)
    if v < 0:
        check(func, int(v))
    return int(v)
