"""CPU oracle for the DiT joint-attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the
checker (or as the reported CPU baseline). The product (localrouter_amd) never imports it.

Two layers:
  * liblro.so (lro.c): the C restatement -- seeded bf16 inputs, RMSNorm + RoPE, fp64 brute-force attention (the pin),
    fp32 flash-style attention (the CPU baseline), the fused op. Wrapped here with numpy arrays.
  * brute_* below: an independent pure-numpy fp64 restatement for tiny shapes, used to cross-check liblro.so.

  * lro_int8.c: MiniMax H3's INT8 attention chain (K anchor, Hadamard rotation, int8 quantisers, attention over the
    quantised operands); wrapped by the i8_* functions and int8_attention below.

Reference semantics (jayleaton/localrouter): kernels/cuda/qwen_image/attention.cu:253-444 (attention, mask, GQA),
kernels/cuda/minimax/kitchen/rms_rope.cu:37-230 + rope_device.cuh:65-98 (RMSNorm + RoPE),
src/engines/qwen_image/triton_k.zig:44-53 (Qwen's fp32 cos/sin form).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liblro.so"
D = 128

TABLE_NONE, TABLE_COSSIN_F32, TABLE_MAT2_BF16, TABLE_MAT2_F32 = 0, 1, 2, 3
PAIR_INTERLEAVED, PAIR_SPLIT_HALF = 0, 1

MUTANTS = {
    "rope_sign": 1,
    "no_eps": 2,
    "pairing": 3,
    "no_scale": 4,
    "causal_off_by_one": 5,
    "gqa_mod": 6,
    "no_weight": 7,
    "table_transposed": 8,
    "no_round_norm": 9,
    "no_round_prepared": 10,
}


def build_oracle(force: bool = True) -> Path:
    """Compile liblro.so with the committed Makefile (gcc, OpenMP)."""
    cmd = ["make", "-C", str(HERE)] + (["-B"] if force else []) + ["liblro.so"]
    subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return LIB_PATH


_lib = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build_oracle()
        L = ctypes.CDLL(str(LIB_PATH))
        L.lro_set_mutant.argtypes = [ctypes.c_int]
        L.lro_num_threads.restype = ctypes.c_int
        L.lro_set_threads.argtypes = [ctypes.c_int]
        L.lro_synth_normal_bf16.argtypes = [ctypes.c_uint64, ctypes.c_uint64, _I64, _P]
        L.lro_f32_to_bf16_array.argtypes = [_P, _P, _I64]
        L.lro_bf16_to_f32_array.argtypes = [_P, _P, _I64]
        L.lro_rms_rope.argtypes = [_P, _I64, ctypes.c_int, _I64, _P, _P, ctypes.c_int, _P, _P, _I64, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_float, _P]
        L.lro_rms_rope_ex.argtypes = [_P, _I64, ctypes.c_int, _I64, _P, _P, ctypes.c_int, _P, _P, _I64, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_float, ctypes.c_int, _P]
        L.lro_attention_f64.argtypes = [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.lro_attention_f32.argtypes = [_P, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_float, _P, _I64]
        L.lro_joint_attention.argtypes = [_P, _P, _P, _I64, _I64, _I64, _P, _P, ctypes.c_int, _P, _P, _P, _P, _I64,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                          ctypes.c_int, ctypes.c_int, _P]
        L.lro_joint_attention_ex.argtypes = list(L.lro_joint_attention.argtypes[:-1]) + [ctypes.c_int, _P]
        L.lro_i8_rotate.argtypes = [_P, ctypes.c_int, ctypes.c_int]
        L.lro_i8_anchor.argtypes = [_P, _I64, ctypes.c_int, ctypes.c_int]
        L.lro_i8_anchor.restype = ctypes.c_int
        L.lro_i8_quant_rows.argtypes = [_P, _I64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        _P, _P]
        L.lro_i8_quant_v.argtypes = [_P, _I64, ctypes.c_int, ctypes.c_int, _P, _P]
        L.lro_i8_attention.argtypes = [_P, _P, _P, _P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_float, _P]
        L.lro_i8_attention_p8.argtypes = [_P, _P, _P, _P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_float, ctypes.c_int, _P]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


class mutant:
    """Context manager planting a mistake in the C oracle (tests of the pins only)."""

    def __init__(self, name: str):
        self.code = MUTANTS[name]

    def __enter__(self):
        lib().lro_set_mutant(self.code)
        return self

    def __exit__(self, *exc):
        lib().lro_set_mutant(0)


def set_threads(n: int) -> None:
    lib().lro_set_threads(int(n))


def num_threads() -> int:
    return int(lib().lro_num_threads())


# ------------------------------------------------------------------------------------------ bf16 helpers and inputs
def synth_bf16(seed: int, stream: int, shape) -> np.ndarray:
    """Seeded N(0,1) values rounded to bf16, as uint16 bits (splitmix64 counter -> Box-Muller; lro.c documents it)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    lib().lro_synth_normal_bf16(ctypes.c_uint64(seed), ctypes.c_uint64(stream), n, _ptr(out))
    return out.reshape(shape)


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    return (x.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().lro_f32_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


# ------------------------------------------------------------------------------------------ liblro.so wrappers
def rms_rope(x: np.ndarray, w=None, *, table_kind=TABLE_NONE, ta=None, tb=None, pairing=PAIR_INTERLEAVED,
             rot=128, eps=1e-6, w_bf16=None, round_norm=False) -> np.ndarray:
    """x: uint16 (bf16 bits) [rows, heads, 128] -> fp32 [rows, heads, 128]. Row r uses table row r.
    Tables: COSSIN: ta = cos, tb = sin fp32 [rows, >= rot/2]; MAT2_BF16: ta uint16 [rows, >= 2*rot];
    MAT2_F32: ta fp32 [rows, >= 2*rot]. round_norm: the normalised value rounded to bf16 before the rotation
    (rms_rope.cu:143-150)."""
    x = np.ascontiguousarray(x)
    rows, heads, d = x.shape
    assert d == D
    y = np.empty((rows, heads, D), dtype=np.float32)
    stride = 0
    if table_kind != TABLE_NONE:
        ta = np.ascontiguousarray(ta)
        stride = ta.shape[1]
        if tb is not None:
            tb = np.ascontiguousarray(tb)
            assert tb.shape == ta.shape
    wp = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    wb = None if w_bf16 is None else np.ascontiguousarray(w_bf16, dtype=np.uint16)
    lib().lro_rms_rope_ex(_ptr(x), rows, heads, heads * D, _ptr(wp), _ptr(wb), table_kind, _ptr(ta), _ptr(tb),
                          stride, pairing, rot, ctypes.c_float(eps), int(bool(round_norm)), _ptr(y))
    return y


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, *, p0=0, nkeys=None, causal=False, scale=None,
              precise=True, rows=None) -> np.ndarray:
    """q fp32 [W, H, 128], k, v fp32 [nkeys, HK, 128] -> fp32 [W, H, 128] (or [len(rows), H, 128]).
    precise: fp64 brute force; else the fp32 flash-style CPU path (the baseline), optionally on a subset of rows."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    W, H, _ = q.shape
    nk, HK, _ = k.shape
    nkeys = nk if nkeys is None else nkeys
    scale = np.float32(1.0 / np.sqrt(np.float32(D))) if scale is None else np.float32(scale)
    if precise:
        assert rows is None
        out = np.empty((W, H, D), dtype=np.float32)
        lib().lro_attention_f64(_ptr(q), _ptr(k), _ptr(v), _ptr(out), p0, W, H, HK, nkeys, int(causal),
                                ctypes.c_float(scale))
        return out
    if rows is not None:
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        out = np.empty((len(rows), H, D), dtype=np.float32)
        lib().lro_attention_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(out), p0, W, H, HK, nkeys, int(causal),
                                ctypes.c_float(scale), _ptr(rows), len(rows))
        return out
    out = np.empty((W, H, D), dtype=np.float32)
    lib().lro_attention_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(out), p0, W, H, HK, nkeys, int(causal),
                            ctypes.c_float(scale), None, 0)
    return out


def joint_attention(q_raw, k_raw, v, *, wq=None, wk=None, table_kind=TABLE_NONE, qa=None, qb=None, ka=None,
                    kb=None, pairing=PAIR_INTERLEAVED, rot=128, eps=1e-6, p0=0, causal=False, scale=None, n_pre=0,
                    precise=True, round_prepared=False) -> np.ndarray:
    """The fused op on bf16-bit inputs q_raw [Sq, H, 128], k_raw, v [Sk, HK, 128] -> fp32 [Sq, H, 128].
    Query i uses q-table row i, key j >= n_pre uses k-table row j - n_pre, keys j < n_pre are used as given.
    round_prepared: the normalised, rotated q and k rounded to bf16 before the attention, as the reference's chain
    stores them (dit.zig:252-263)."""
    q_raw, k_raw, v = (np.ascontiguousarray(a) for a in (q_raw, k_raw, v))
    Sq, H, _ = q_raw.shape
    Sk, HK, _ = k_raw.shape
    scale = np.float32(1.0 / np.sqrt(np.float32(D))) if scale is None else np.float32(scale)
    stride = 0
    if table_kind != TABLE_NONE:
        qa = np.ascontiguousarray(qa)
        ka = qa if ka is None else np.ascontiguousarray(ka)
        stride = qa.shape[1]
        assert ka.shape[1] == stride
        if table_kind == TABLE_COSSIN_F32:
            qb = np.ascontiguousarray(qb)
            kb = qb if kb is None else np.ascontiguousarray(kb)
    wq = None if wq is None else np.ascontiguousarray(wq, dtype=np.float32)
    wk = None if wk is None else np.ascontiguousarray(wk, dtype=np.float32)
    out = np.empty((Sq, H, D), dtype=np.float32)
    lib().lro_joint_attention_ex(_ptr(q_raw), _ptr(k_raw), _ptr(v), H * D, HK * D, HK * D, _ptr(wq), _ptr(wk),
                                 table_kind, _ptr(qa), _ptr(qb), _ptr(ka), _ptr(kb), stride, pairing, rot,
                                 ctypes.c_float(eps), Sq, Sk, H, HK, p0, int(causal), ctypes.c_float(scale), n_pre,
                                 int(precise), int(bool(round_prepared)), _ptr(out))
    return out


# ------------------------------------------------------------------------------------------ pure numpy fp64 brute force
def brute_rms_rope(x_f32: np.ndarray, w=None, *, cos=None, sin=None, mat=None, pairing=PAIR_INTERLEAVED, rot=128,
                   eps=1e-6, round_norm=False) -> np.ndarray:
    """fp64 restatement on float inputs [rows, heads, 128]; cos/sin [rows, rot/2] or mat [rows, rot/2, 2, 2].
    round_norm: the normalised value rounded to fp32, then to bf16 (numpy's own rounding, ties to even) before the
    rotation."""
    x = x_f32.astype(np.float64)
    rr = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * rr * (1.0 if w is None else np.asarray(w, np.float64))
    if round_norm:
        f = y.astype(np.float32)
        b = f.view(np.uint32).astype(np.uint64)
        b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16       # RNE to the upper 16 bits (finite inputs)
        y = b.astype(np.uint32).view(np.float32).astype(np.float64)
    if cos is None and mat is None:
        return y
    P = rot // 2
    if pairing == PAIR_INTERLEAVED:
        a_idx, b_idx = np.arange(P) * 2, np.arange(P) * 2 + 1
    else:
        a_idx, b_idx = np.arange(P), np.arange(P) + P
    if mat is None:
        c = np.asarray(cos, np.float64)[:, None, :P]
        s = np.asarray(sin, np.float64)[:, None, :P]
        f00, f01, f10, f11 = c, -s, s, c
    else:
        m = np.asarray(mat, np.float64)[:, None, :P]
        f00, f01, f10, f11 = m[..., 0, 0], m[..., 0, 1], m[..., 1, 0], m[..., 1, 1]
    xa, xb = y[..., a_idx].copy(), y[..., b_idx].copy()
    y[..., a_idx] = f00 * xa + f01 * xb
    y[..., b_idx] = f10 * xa + f11 * xb
    return y


def brute_attention(q, k, v, *, p0=0, nkeys=None, causal=False, scale=None) -> np.ndarray:
    """fp64 dense softmax attention: q [W, H, d], k, v [nk, HK, d] (scale d^-0.5 in fp32 by default)."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    W, H, d = q.shape
    nk, HK, _ = k.shape
    nkeys = nk if nkeys is None else nkeys
    scale = float(np.float32(1.0 / np.sqrt(np.float32(d)))) if scale is None else float(scale)
    G = H // HK
    out = np.zeros((W, H, v.shape[-1]))
    j = np.arange(nk)
    for h in range(H):
        s = q[:, h, :] @ k[:, h // G, :].T * scale
        vis = (j[None, :] < nkeys)
        if causal:
            vis = vis & (j[None, :] <= p0 + np.arange(W)[:, None])
        s = np.where(vis, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ v[:, h // G, :]
    return out


# ------------------------------------------------------------------------------------------ INT8 chain (lro_int8.c)
I8_KGROUP = 16   # keys per K scale


def i8_rotation_for(seq: int, d: int = D) -> int:
    """H4 for sequences up to 256 tokens, else the signed H128 (head dim 128) or the plain H64 (head dim 64)
    (src/engines/minimax_h3/launch.zig:387-391, kernels/cuda/minimax/kitchen_launch.cu:236-241)."""
    return 4 if seq <= 256 else d


def i8_scale(d: int = D) -> float:
    """The softmax scale a caller passes for head dim d: d^-0.5 rounded to fp32 (0x3db504f3 for 128)."""
    return float(np.float32(1.0 / np.sqrt(d)))


def i8_rotate(x: np.ndarray, kind: int) -> np.ndarray:
    """Rotate every row of x (fp32 [..., d], d 64 or 128) in the operation order of the reference's convrot helpers;
    returns a copy."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    d = y.shape[-1]
    for row in y.reshape(-1, d):
        lib().lro_i8_rotate(_ptr(row), d, kind)
    return y


def i8_anchor(k_head_bits: np.ndarray) -> int:
    """Anchor row of one kv head's keys (uint16 bf16 bits [Lk, d])."""
    k = np.ascontiguousarray(k_head_bits, dtype=np.uint16)
    d = k.shape[-1]
    return int(lib().lro_i8_anchor(_ptr(k), d, k.shape[0], d))


def i8_quant_rows(x_bits: np.ndarray, rot: int, anchor: int = -1, group: int = 1):
    """int8 [rows, d] and the per-group scales of one head's rows (bf16 bits [rows, d])."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, d = x.shape
    out = np.zeros((rows, d), np.int8)
    sc = np.zeros(((rows + group - 1) // group,), np.float32)
    lib().lro_i8_quant_rows(_ptr(x), d, rows, d, rot, anchor, group, _ptr(out), _ptr(sc))
    return out, sc


def i8_quant_v(v_bits: np.ndarray):
    v = np.ascontiguousarray(v_bits, dtype=np.uint16)
    rows, d = v.shape
    out = np.zeros((rows, d), np.int8)
    sc = np.zeros((d,), np.float32)
    lib().lro_i8_quant_v(_ptr(v), d, rows, d, _ptr(out), _ptr(sc))
    return out, sc


def i8_attention(q8, qs, k8, ks, v8, vs, kgroup: int = I8_KGROUP, scale: float | None = None) -> np.ndarray:
    q8, k8, v8 = (np.ascontiguousarray(a, dtype=np.int8) for a in (q8, k8, v8))
    qs, ks, vs = (np.ascontiguousarray(a, dtype=np.float32) for a in (qs, ks, vs))
    d = q8.shape[1]
    scale = i8_scale(d) if scale is None else scale
    out = np.zeros((q8.shape[0], d), np.float32)
    lib().lro_i8_attention(_ptr(q8), _ptr(qs), _ptr(k8), _ptr(ks), kgroup, _ptr(v8), _ptr(vs), q8.shape[0],
                           k8.shape[0], d, scale, _ptr(out))
    return out


def i8_attention_p8(q8, qs, k8, ks, v8, vs, cta: int, kgroup: int = I8_KGROUP, scale: float | None = None) -> np.ndarray:
    """i8_attention with P rounded to u8 against each cta-key tile's row max, as the reference's kernel rounds it."""
    q8, k8, v8 = (np.ascontiguousarray(a, dtype=np.int8) for a in (q8, k8, v8))
    qs, ks, vs = (np.ascontiguousarray(a, dtype=np.float32) for a in (qs, ks, vs))
    d = q8.shape[1]
    scale = i8_scale(d) if scale is None else scale
    out = np.zeros((q8.shape[0], d), np.float32)
    lib().lro_i8_attention_p8(_ptr(q8), _ptr(qs), _ptr(k8), _ptr(ks), kgroup, _ptr(v8), _ptr(vs), q8.shape[0],
                              k8.shape[0], d, scale, cta, _ptr(out))
    return out


def i8_cta_for(sk: int, d: int = D) -> int:
    """Key tile of the P rounding: 128 keys past 1024 keys at head dim 128, else 64 (src/engines/minimax_h3/
    launch.zig:333, kernels/cuda/minimax/kitchen_launch.cu:107)."""
    return 128 if sk > 1024 and d >= 128 else 64


def int8_attention(qkv_bits: np.ndarray, heads: int, rows=None) -> tuple[np.ndarray, dict]:
    """The whole chain for packed qkv (bf16 bits [S, 3, heads, d], d 64 or 128): per head the K anchor, Q (one scale
    per row) and K (one scale per 16 keys, anchor subtracted) rotated and quantised, V quantised per channel, then
    attention of the selected query rows (all by default) at scale d^-0.5. Returns fp32 [heads, len(rows), d] and the
    quantised operands."""
    S, d = qkv_bits.shape[0], qkv_bits.shape[-1]
    rot = i8_rotation_for(S, d)
    rows = np.arange(S) if rows is None else np.asarray(rows)
    out = np.zeros((heads, len(rows), d), np.float32)
    parts = {"q8": [], "qs": [], "k8": [], "ks": [], "v8": [], "vs": [], "anchor": []}
    for h in range(heads):
        q, k, v = (np.ascontiguousarray(qkv_bits[:, i, h]) for i in range(3))
        a = i8_anchor(k)
        q8, qs = i8_quant_rows(q, rot)
        k8, ks = i8_quant_rows(k, rot, a, I8_KGROUP)
        v8, vs = i8_quant_v(v)
        out[h] = i8_attention(q8[rows], qs[rows], k8, ks, v8, vs)
        for name, val in zip(parts, (q8, qs, k8, ks, v8, vs, a)):
            parts[name].append(val)
    return out, parts
