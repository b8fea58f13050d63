"""Shared helpers for the GPU parity tests: bf16 bit arrays <-> torch tensors, tolerance checks."""
from __future__ import annotations

import numpy as np

# BASELINE's parity bar for bf16 outputs against the fp32/fp64 oracle
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def to_dev(bits: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def from_dev(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def bf16_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def err(got_bits: np.ndarray, ref: np.ndarray):
    d = np.abs(bf16_f32(got_bits).astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float(d.mean())


def assert_close(got_bits: np.ndarray, ref: np.ndarray, max_abs: float = MAX_ABS, mean_abs: float = MEAN_ABS,
                 what: str = ""):
    got = bf16_f32(got_bits)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    mx, mn = err(got_bits, ref)
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} (bar {max_abs}), mean-abs {mn:.3e} (bar {mean_abs})"
    return mx, mn
