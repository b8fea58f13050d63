"""Shared helpers for the GPU parity tests: bf16 bit arrays <-> torch tensors, tolerance checks."""
from __future__ import annotations

import numpy as np

# the parity bar for bf16 outputs against the fp32/fp64 oracle: max-abs and mean-abs (the north star's), and a
# relative L2 bound that a systematic error (a wrong scale, a dropped term) fails even where outputs are small
MAX_ABS = 2e-2
MEAN_ABS = 2e-3
REL_L2 = 3e-3


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


def rel_l2(got_bits: np.ndarray, ref: np.ndarray) -> float:
    d = bf16_f32(got_bits).astype(np.float64) - ref.astype(np.float64)
    den = float(np.linalg.norm(ref.astype(np.float64)))
    return float(np.linalg.norm(d)) / den if den > 0 else float(np.linalg.norm(d))


def assert_close(got_bits: np.ndarray, ref: np.ndarray, max_abs: float = MAX_ABS, mean_abs: float = MEAN_ABS,
                 what: str = "", rel: float = REL_L2):
    got = bf16_f32(got_bits)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    mx, mn = err(got_bits, ref)
    rl = rel_l2(got_bits, ref)
    assert mx <= max_abs and mn <= mean_abs and rl <= rel, \
        f"{what}: max-abs {mx:.3e} (bar {max_abs}), mean-abs {mn:.3e} (bar {mean_abs}), rel-L2 {rl:.3e} (bar {rel})"
    return mx, mn


def bf16_ulps(got_bits: np.ndarray, ref: np.ndarray, floor: float = 2.0 ** -10) -> np.ndarray:
    """|got - ref| in units of the bf16 spacing at |ref| (at least at floor, so that values that cancel to near zero
    are measured against the spacing of the inputs' scale)."""
    r = np.maximum(np.abs(ref.astype(np.float64)), floor)
    ulp = 2.0 ** (np.floor(np.log2(r)) - 7)
    return np.abs(bf16_f32(got_bits).astype(np.float64) - ref.astype(np.float64)) / ulp


# ------------------------------------------------------------------------------------------ tile images
def img_index():
    """Element indices (uint16 units within a 16 KB key tile image) of key r dim d: the layout of tile_image.h restated --
    key fragments f = 8 (r >> 5) + (d >> 4), lane 32 ((d >> 3) & 1) + perm(r & 31) with perm swapping bits 2 and 3."""
    r = np.arange(64)[:, None]
    d = np.arange(128)[None, :]
    m = r & 31
    perm = (m & 0x13) | ((m & 4) << 1) | ((m & 8) >> 1)
    return ((8 * (r >> 5) + (d >> 4)) * 1024 + (32 * ((d >> 3) & 1) + perm) * 16) // 2 + (d & 7)


def decode_images(raw: np.ndarray, Sk: int, HK: int):
    """Workspace bytes -> keys, values uint16 [HK][ceil(Sk/64)*64][128] (rows past Sk included): the key tile images,
    then the value area, rows [tiles * 64][HK][128]."""
    nt = (Sk + 63) // 64
    u = raw[: 2 * HK * nt * 16384].view(np.uint16)
    kimg = u[: HK * nt * 8192].reshape(HK, nt, 8192)
    keys = kimg[:, :, img_index()].reshape(HK, nt * 64, 128)
    vals = u[HK * nt * 8192:].reshape(nt * 64, HK, 128).transpose(1, 0, 2)
    return keys, vals
