"""ctypes mirror of include/lr_mmdit.h: the MMDiT double-stream block forward for torch tensors.

    blk = MMDiTBlock(weights)            # weights: dict of bf16 CUDA tensors (torch nn.Linear layout [out, in])
    blk(txt, img, t, cos, sin)           # in place on txt [St, D], img [Si, D] bf16; t: f32 CUDA tensor [1]

There is no fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from . import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "lr_mmdit.h"

_P, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t


class StreamWeights(ctypes.Structure):
    _fields_ = [("mod", _P), ("qkv", _P), ("out", _P), ("mlp_up", _P), ("mlp_down", _P)]


class Weights(ctypes.Structure):
    _fields_ = [("t1", _P), ("t2", _P), ("q_norm", _P), ("k_norm", _P), ("txt", StreamWeights),
                ("img", StreamWeights)]


SIGNATURES = {
    "lr_mmdit_create": (_I, [ctypes.POINTER(_P)]),
    "lr_mmdit_destroy": (_I, [_P]),
    "lr_mmdit_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "lr_mmdit_plan": (_I, [_P, _I, _I, _I, _I]),
    "lr_mmdit_tune": (_I, [_P, ctypes.POINTER(Weights), _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "lr_mmdit_linear_bf16": (_I, [_P, _P, ctypes.c_int64, _P, _P, ctypes.c_int64, _I, _I, _I, _P, _SZ, _P]),
    "lr_mmdit_block_bf16": (_I, [_P, ctypes.POINTER(Weights), _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P]),
}

STREAM_KEYS = ("mod", "qkv", "out", "mlp_up", "mlp_down")
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


def workspace_bytes(n_txt: int, n_img: int, hidden: int, mlp: int) -> int:
    return int(lib().lr_mmdit_workspace_bytes(n_txt, n_img, hidden, mlp))


def make_weights(hidden: int, mlp: int, device, seed: int = 0, std: float = 0.02, zero_mod: bool = False):
    """Random-init bf16 weights N(0, std) of one block (torch nn.Linear layout), norm weights 1.0."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    D, F = hidden, mlp

    def rnd(*shape):
        return (torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)

    w = {"t1": rnd(D, 256), "t2": rnd(D, D), "q_norm": torch.ones(128, device=device),
         "k_norm": torch.ones(128, device=device)}
    for s in ("txt", "img"):
        w[f"{s}.mod"] = rnd(6 * D, D) * (0 if zero_mod else 1)
        w[f"{s}.qkv"] = rnd(3 * D, D)
        w[f"{s}.out"] = rnd(D, D)
        w[f"{s}.mlp_up"] = rnd(F, D)
        w[f"{s}.mlp_down"] = rnd(D, F)
    return w


class MMDiTBlock:
    """One block's weights bound to a library context (hipBLASLt handle and GEMM plans)."""

    def __init__(self, weights: dict):
        import torch
        self.w = weights
        self.hidden = weights["t2"].shape[0]
        self.mlp = weights["txt.mlp_up"].shape[0]
        for k, v in weights.items():
            want = torch.float32 if k in ("q_norm", "k_norm") else torch.bfloat16
            assert v.is_cuda and v.dtype == want and v.is_contiguous(), k
        self.cw = Weights(t1=weights["t1"].data_ptr(), t2=weights["t2"].data_ptr(),
                          q_norm=weights["q_norm"].data_ptr(), k_norm=weights["k_norm"].data_ptr(),
                          txt=StreamWeights(*[weights[f"txt.{k}"].data_ptr() for k in STREAM_KEYS]),
                          img=StreamWeights(*[weights[f"img.{k}"].data_ptr() for k in STREAM_KEYS]))
        ctx = _P()
        rc = lib().lr_mmdit_create(ctypes.byref(ctx))
        if rc != 0:
            raise _lib.LrError("lr_mmdit_create", rc)
        self.ctx = ctx
        self._ws = None
        self._planned = set()

    def close(self):
        if self.ctx:
            lib().lr_mmdit_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def workspace(self, n_txt: int, n_img: int):
        import torch
        nb = workspace_bytes(n_txt, n_img, self.hidden, self.mlp)
        if nb == 0:
            raise _lib.LrError("lr_mmdit_workspace_bytes", 1)
        if self._ws is None or self._ws.numel() < nb:
            self._ws = torch.empty(nb, dtype=torch.uint8, device=self.w["t1"].device)
        return self._ws

    def tune(self, n_txt: int, n_img: int, candidates: int = 16, stream=None):
        """Pick the fastest of the hipBLASLt candidates for this shape's GEMMs (synchronises)."""
        import torch
        ws = self.workspace(n_txt, n_img)
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().lr_mmdit_tune(self.ctx, ctypes.byref(self.cw), n_txt, n_img, self.hidden, self.mlp, candidates,
                                 ws.data_ptr(), ws.numel(), s)
        if rc != 0:
            raise _lib.LrError("lr_mmdit_tune", rc)
        self._planned.add((n_txt, n_img))

    def plan(self, n_txt: int, n_img: int):
        """Build the GEMM plans of this shape (host only); the block call needs them (lr_mmdit_plan)."""
        if (n_txt, n_img) in self._planned:
            return
        rc = lib().lr_mmdit_plan(self.ctx, n_txt, n_img, self.hidden, self.mlp)
        if rc != 0:
            raise _lib.LrError("lr_mmdit_plan", rc)
        self._planned.add((n_txt, n_img))

    def linear(self, x, w, y, stream=None):
        """y = x w^T through the block's GEMM path (x [M, K], w [N, K], y [M, N] bf16 CUDA tensors, rows may be
        strided). Uses this block's workspace (allocate it with workspace() first)."""
        import torch
        assert self._ws is not None
        M, K = x.shape
        N = w.shape[0]
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().lr_mmdit_linear_bf16(self.ctx, x.data_ptr(), x.stride(0), w.data_ptr(), y.data_ptr(), y.stride(0),
                                        M, N, K, self._ws.data_ptr(), self._ws.numel(), s)
        if rc != 0:
            raise _lib.LrError("lr_mmdit_linear_bf16", rc)

    def __call__(self, txt, img, t, cos, sin, stream=None):
        import torch
        n_txt, n_img = txt.shape[0], img.shape[0]
        assert txt.dtype == img.dtype == torch.bfloat16 and txt.is_contiguous() and img.is_contiguous()
        assert t.dtype == torch.float32 and cos.dtype == sin.dtype == torch.float32
        assert cos.shape == (n_txt + n_img, 64) and sin.shape == cos.shape
        ws = self.workspace(n_txt, n_img)
        self.plan(n_txt, n_img)
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().lr_mmdit_block_bf16(self.ctx, ctypes.byref(self.cw), txt.data_ptr(), img.data_ptr(), n_txt, n_img,
                                       self.hidden, self.mlp, t.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                       ws.data_ptr(), ws.numel(), s)
        if rc != 0:
            raise _lib.LrError("lr_mmdit_block_bf16", rc)
