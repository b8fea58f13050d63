"""Writes tests/golden/sincos.npz: bits of the engines' portable sincos (src/engines/qwen_image/smath.zig:40-52) on
a fixed set of angles, computed by the reference's own Python statement of it (tools/twin/stk_twin/smath.py, the
twin that smath.zig matches bit for bit, smath.zig:1-2), imported from /root/reference where it lies. Run once in a
container that holds the reference; the fixture holds only inputs and outputs (uint64 bit patterns of f64).

Angles: every fourth point of the reference's own accuracy test (-3000 + 0.7317 i, smath.zig:128-135), the angles of
the Qwen-Image table rows of a 64x64 image grid and its text rows (rope.zig:31-45, ids x omega for the frozen omegas of
kernels/qwen_image/rope_omega.json), and the doubles nearest to k pi / 2 and their neighbours, where the three-part
reduction decides the result.
"""
from __future__ import annotations

import importlib.util
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
TWIN = Path("/root/reference/tools/twin/stk_twin/smath.py")


def angles() -> np.ndarray:
    from localrouter_amd import rope
    grid = -3000.0 + 0.7317 * np.arange(0, 8201, 4, dtype=np.float64)
    grid = grid[grid < 3000.0]
    om = rope.qwen_omegas()
    ids = np.concatenate([rope.qwen_text_ids(4, 0), rope.qwen_image_ids(64, 64, 0)])
    cols = np.concatenate([np.full(d // 2, ax) for ax, d in enumerate(rope.QWEN_AXES)])
    qw = (ids.astype(np.float64)[::37][:, cols] * om[None, :]).ravel()
    near = []
    for k in list(range(-40, 41)) + [1000, 1001, 1910, -1911, 4000, 65535, 2 ** 19]:
        x = k * math.pi / 2
        near += [x, np.nextafter(x, np.inf), np.nextafter(x, -np.inf)]
    return np.unique(np.concatenate([grid, qw, np.array(near)]))


def main() -> None:
    spec = importlib.util.spec_from_file_location("twin_smath", TWIN)
    twin = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(twin)
    x = angles()
    sc = np.array([twin.sincos(float(v)) for v in x], np.float64)
    np.savez_compressed(HERE / "sincos.npz", x=x.view(np.uint64), sin=sc[:, 0].copy().view(np.uint64),
                        cos=sc[:, 1].copy().view(np.uint64))
    print(f"{x.size} angles -> {HERE / 'sincos.npz'}")


if __name__ == "__main__":
    main()
