"""ctypes binding of liblr_attn.so, the C ABI declared in include/lr_attn.h.

Loading fails loudly when the library has not been built: there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "liblr_attn.so"
HEADER = PKG.parent / "include" / "lr_attn.h"

HIP_ERRORS = {0: "hipSuccess", 1: "hipErrorInvalidValue", 2: "hipErrorOutOfMemory", 98: "hipErrorInvalidDeviceFunction",
              100: "hipErrorNoDevice", 101: "hipErrorInvalidDevice", 209: "hipErrorNoBinaryForGpu",
              400: "hipErrorInvalidHandle", 700: "hipErrorIllegalAddress", 719: "hipErrorLaunchFailure"}


class LrError(RuntimeError):
    """A non-zero hipError_t returned by an lr_* entry point."""

    def __init__(self, fn: str, code: int):
        self.fn, self.code = fn, code
        super().__init__(f"{fn} returned {code} ({HIP_ERRORS.get(code, 'hipError')})")


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); the order mirrors include/lr_attn.h
SIGNATURES = {
    "lr_attn_abi_version": (_I, []),
    "lr_attn_init": (_I, []),
    "lr_attention_bf16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I64, _I64, _I64, _P]),
    "lr_attention_bf16_ex": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I,
                                  _P]),
    "lr_rms_rope_bf16": (_I, [_P, _I64, _I64, _P, _I64, _I64, _I, _I64, _I64, _I, _P, _I, _I, _P, _P, _I64, _I, _I, _F,
                              _I, _P]),
    "lr_rms_rope_qk_bf16": (_I, [_P, _P, _I64, _I, _I64, _I64, _P, _P, _P, _I64, _I, _F, _P]),
    "lr_joint_attention_workspace_bytes": (_SZ, [_I, _I]),
    "lr_joint_attention_fused": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I64, _I, _I, _F, _I, _I, _I, _I, _I,
                                      _I, _F, _I64, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "lr_joint_kv_prepare": (_I, [_P, _I64, _P, _I64, _P, _I, _P, _P, _I64, _I, _I, _F, _I, _I, _I, _P, _SZ, _P]),
    "lr_joint_attention_prepared": (_I, [_P, _P, _SZ, _P, _P, _I, _P, _P, _I64, _I, _I, _F, _I, _I, _I, _I, _I, _I,
                                         _F, _I64, _I64, _I, _P]),
    "lr_joint_q_prepare": (_I, [_P, _I64, _P, _I64, _P, _I, _P, _P, _I64, _I, _I, _F, _I, _I, _P]),
    "lr_joint_attention_images": (_I, [_P, _I64, _P, _SZ, _P, _I64, _I, _I, _I, _I, _I, _I, _F, _P]),
    "lr_joint_prepare": (_I, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I, _P, _P, _P, _P, _I64, _I, _I, _F, _I,
                              _I, _I, _I, _I, _P, _SZ, _P]),
    "lr_joint_attention_fused_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I64, _I, _I, _F, _I, _I,
                                              _I, _I, _I, _I, _F, _I64, _I64, _I64, _I64, _I, _P]),
    "lr_int8_attention_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "lr_int8_attention": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I] + [_I64] * 9 + [_F, _P]),
    "lr_int8_attention_rows": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I] + [_I64] * 9 + [_F, _P]),
    "lr_int8_attention_prep": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I] + [_I64] * 9 + [_P]),
    "lr_int8_attention_kernel": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _F, _I, _P]),
    "lr_int8_attention_prep_rope": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I] + [_I64] * 9 +
                                    [_P, _P, _P, _I64, _I, _F, _P]),
    "lr_attention_ws_bytes": (_SZ, [_I, _I, _I, _I]),
    "lr_attention_bf16_ws": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _I64, _I64, _I64, _P, _SZ, _P]),
    "lr_attention_kmask_workspace_bytes": (_SZ, [_I, _I]),
    "lr_attention_kmask_bf16": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I64, _I64, _I64, _P, _SZ, _P]),
    "lr_joint_attention_fused_ex": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _I64, _I, _I, _F, _I, _I, _I, _I,
                                         _I, _I, _F, _I64, _I64, _I64, _I64, _I, _P, _SZ, _I, _P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library (RuntimeError if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m localrouter_amd.build` "
                               "(there is no fallback path)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an lr_* entry point that returns a hipError_t; raise LrError when it is not 0."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise LrError(name, rc)
