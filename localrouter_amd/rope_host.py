"""ctypes mirror of include/lr_rope.h: the host RoPE position and table builders of liblr_attn.so (CPU only).

Same tables as localrouter_amd.rope (numpy), computed by the library's C++ code, which engines link instead of
re-implementing rope.zig / layout.zig. Each builder returns numpy arrays; a rejected argument raises LrError.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "lr_rope.h"

_P, _I, _I64, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double

# name -> (restype, argtypes); the order mirrors include/lr_rope.h
SIGNATURES = {
    "lr_rope_sincos": (_I, [_P, _I64, _P, _P]),
    "lr_rope_qwen_omegas": (None, [_P]),
    "lr_rope_qwen_text_ids": (_I, [_P, _I, _I]),
    "lr_rope_qwen_image_ids": (_I, [_P, _I, _I, _I, _I, _I]),
    "lr_rope_qwen_table": (_I, [_P, _I, _P, _P, _P]),
    "lr_rope_grid2d_table": (_I, [_I, _I, _I, _D, _P, _P]),
    "lr_rope_edit_table": (_I, [_I, _I, _I, _I, _P, _P]),
    "lr_rope_video3d_table": (_I, [_I, _I, _I, _I, _D, _P, _P]),
    "lr_rope_h3_rows": (_I64, [_I, _I, _I, _I, _I, _I]),
    "lr_rope_h3_positions": (_I, [_I, _I, _I, _I, _I, _I, _P]),
    "lr_rope_h3_table": (_I, [_P, _I64, _P, _P]),
}

_bound = None


def lib() -> ctypes.CDLL:
    global _bound
    if _bound is None:
        L = _lib.load()
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _bound = L
    return _bound


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _check(name: str, rc: int) -> None:
    if rc != 0:
        raise _lib.LrError(name, rc)


def sincos(x: np.ndarray):
    """The library's engine sincos of f64 angles: (sin, cos)."""
    x = np.ascontiguousarray(x, np.float64)
    s, c = np.empty_like(x), np.empty_like(x)
    _check("lr_rope_sincos", lib().lr_rope_sincos(_ptr(x), x.size, _ptr(s), _ptr(c)))
    return s, c


def qwen_omegas() -> np.ndarray:
    out = np.empty(64, np.float64)
    lib().lr_rope_qwen_omegas(_ptr(out))
    return out


def qwen_text_ids(n: int, first: int = 0) -> np.ndarray:
    ids = np.empty((max(n, 0), 3), np.float32)
    _check("lr_rope_qwen_text_ids", lib().lr_rope_qwen_text_ids(_ptr(ids), n, first))
    return ids


def qwen_image_ids(h: int, w: int, pos: int, target_h: int | None = None, target_w: int | None = None) -> np.ndarray:
    target_h = h if target_h is None else target_h
    target_w = w if target_w is None else target_w
    ids = np.empty((max(h * w, 0), 3), np.float32)
    _check("lr_rope_qwen_image_ids", lib().lr_rope_qwen_image_ids(_ptr(ids), h, w, pos, target_h, target_w))
    return ids


def qwen_table(ids: np.ndarray, om: np.ndarray | None = None):
    ids = np.ascontiguousarray(ids, np.float32)
    n = ids.shape[0]
    c, s = np.empty((n, 64), np.float32), np.empty((n, 64), np.float32)
    omp = None if om is None else _ptr(np.ascontiguousarray(om, np.float64))
    _check("lr_rope_qwen_table", lib().lr_rope_qwen_table(_ptr(ids), n, omp, _ptr(c), _ptr(s)))
    return c, s


def _table(name: str, rows: int, *args):
    c, s = np.empty((rows, 64), np.float32), np.empty((rows, 64), np.float32)
    _check(name, getattr(lib(), name)(*args, _ptr(c), _ptr(s)))
    return c, s


def grid2d_table(n_text: int, gh: int, gw: int, theta: float = 10000.0):
    return _table("lr_rope_grid2d_table", n_text + gh * gw, n_text, gh, gw, theta)


def edit_table(n_text: int, frames: int, gh: int, gw: int):
    return _table("lr_rope_edit_table", n_text + frames * gh * gw, n_text, frames, gh, gw)


def video3d_table(n_text: int, t: int, gh: int, gw: int, theta: float = 10000.0):
    return _table("lr_rope_video3d_table", n_text + t * gh * gw, n_text, t, gh, gw, theta)


def h3_rows(l: int, t: int, h: int, w: int, a: int, first_frame: bool = False) -> int:
    return int(lib().lr_rope_h3_rows(l, t, h, w, a, int(first_frame)))


def h3_positions(l: int, t: int, h: int, w: int, a: int, first_frame: bool = False) -> np.ndarray:
    rows = h3_rows(l, t, h, w, a, first_frame)
    if rows < 0:
        raise _lib.LrError("lr_rope_h3_rows", 1)
    pos = np.empty((rows, 3), np.float64)
    _check("lr_rope_h3_positions", lib().lr_rope_h3_positions(l, t, h, w, a, int(first_frame), _ptr(pos)))
    return pos


def h3_rope_table(pos: np.ndarray, inv_freq: np.ndarray) -> np.ndarray:
    pos = np.ascontiguousarray(pos, np.float64)
    inv = np.ascontiguousarray(inv_freq, np.float32)
    assert inv.shape == (16,)
    out = np.empty((pos.shape[0], 48, 2, 2), np.uint16)
    _check("lr_rope_h3_table", lib().lr_rope_h3_table(_ptr(pos), pos.shape[0], _ptr(inv), _ptr(out)))
    return out
