"""Host-side RoPE tables for the joint-attention path (numpy; built once per shape, then uploaded).

Three families:

* Qwen-Image (src/engines/qwen_image/rope.zig:7-45, tools/twin/stk_twin/dit.py:67-88): ids [N, 3] = (frame or
  position, row, column); axes of 16 / 56 / 56 dims; omega_j = theta^(-2j/d_axis) per axis (the 64 values frozen in
  kernels/qwen_image/rope_omega.json); angle = id * omega in f64, sin/cos in f64 rounded to f32; cos, sin [N, 64]
  fp32, interleaved pairs (LR_TABLE_COSSIN_F32).
* MiniMax H3 (src/engines/minimax_h3/layout.zig:60-134): positions (t, h, w) in f64 for the packed
  [text | cond | audio | video] layout; angle = f32(pos) * inv_freq[j] (16 shared frequencies) in f32, sin/cos in f64
  rounded to f32 then bf16; table [S, 48, 2, 2] = [c, -s, s, c] (LR_TABLE_MAT2_BF16), split-half pairs, rot 96.
* The synthetic BASELINE shapes (the build's own definition, the reference has no such configs): 2D grid tables for
  the 1024-token and 4096-token images, the three-frame edit layout, and the 3D video grid; text tokens un-rotated.

Every table takes its sin / cos from `engine_sincos`, the reference's portable f64 routine
(src/engines/qwen_image/smath.zig:18-52) restated operation for operation, so that the tables are the engines' bits
(numpy's own sin / cos can differ from it in the last f64 bit, and so cross an f32 rounding boundary).
"""
from __future__ import annotations

import numpy as np

QWEN_AXES = (16, 56, 56)
QWEN_THETA = 10000.0
H3_FRAME_PER_TOKEN = (1.0, 4.0, 4.0, 4.0, 4.0)   # layout.zig:12
H3_FRAME_RESCALE = 5.0 / 3.0                      # layout.zig:13


# smath.zig:7-20: pi/2 split in three parts for the Cody-Waite reduction (n * PIO2_1 exact for |n| < 2^20), and the
# kernel polynomials of fdlibm (Sun Microsystems, 1993: k_sin.c, k_cos.c; the reduction constants of e_rem_pio2.c)
INVPIO2 = 6.36619772367581382433e-01
PIO2_1 = 1.57079632673412561417e+00
PIO2_2 = 6.07710050630396597660e-11
PIO2_3 = 2.02226624871116645580e-21
SIN_COEF = (-1.66666666666666324348e-01, 8.33333333332248946124e-03, -1.98412698298579493134e-04,
            2.75573137070700676789e-06, -2.50507602534068634195e-08, 1.58969099521155010221e-10)
COS_COEF = (4.16666666666666019037e-02, -1.38888888888741095749e-03, 2.48015872894767294178e-05,
            -2.75573143513906633035e-07, 2.08757232129817482790e-09, -1.13596475577881948265e-11)


def engine_sincos(x) -> tuple[np.ndarray, np.ndarray]:
    """smath.sincos (smath.zig:40-52) elementwise in float64, the same IEEE operations in the same order: n =
    floor(x 2/pi + 1/2), r = ((x - n pio2_1) - n pio2_2) - n pio2_3, fdlibm's kernel sin and cos of r, quadrant n mod 4.
    Returns (sin, cos)."""
    x = np.asarray(x, np.float64)
    s1, s2, s3, s4, s5, s6 = SIN_COEF
    c1, c2, c3, c4, c5, c6 = COS_COEF
    fn = np.floor(x * INVPIO2 + 0.5)
    n = fn.astype(np.int64)
    r = ((x - fn * PIO2_1) - fn * PIO2_2) - fn * PIO2_3
    z = r * r
    v = z * r
    sv = r + v * (s1 + z * (s2 + z * (s3 + z * (s4 + z * (s5 + z * s6)))))
    cr = z * (c1 + z * (c2 + z * (c3 + z * (c4 + z * (c5 + z * c6)))))
    hz = 0.5 * z
    w = 1.0 - hz
    cv = w + (((1.0 - w) - hz) + z * cr)
    q = n & 3
    sin = np.select([q == 0, q == 1, q == 2], [sv, cv, -sv], -cv)
    cos = np.select([q == 0, q == 1, q == 2], [cv, -sv, -cv], sv)
    return sin, cos


def axis_omegas(d: int, theta: float = QWEN_THETA) -> np.ndarray:
    """omega_j = 1 / theta^(2j/d), j < d/2, in f64."""
    j = np.arange(d // 2, dtype=np.float64)
    return 1.0 / np.power(np.float64(theta), 2.0 * j / d)


# The 64 Qwen-Image frequencies as the engine loads them (f64 bit patterns, big-endian hex; the values of
# kernels/qwen_image/rope_omega.json, read by smath.omegas, smath.zig:112-126). They are torch's float64
# 1 / 10000 ** linspace(0, (d - 2) / d, d / 2) per axis, within 9 f64 ulp of theta^(-2j/d); frozen so that tables
# match the engine's bits.
QWEN_OMEGA_F64_HEX = (
    "3ff0000000000000", "3fd43d136248490f", "3fb999999999999a", "3fa030dc4ea03a72", "3f847ae147ae147b", "3f69e7c6e43390b6",
    "3f50624dd2f1a9fc", "3f34b96be9c2da2c", "3ff0000000000000", "3fe707aa3f9e1202", "3fe093069178d379", "3fd7db4a2009c6e3",
    "3fd12b542ba56564", "3fc8b682a4336478", "3fc1c9194d504805", "3fb999999999999a", "3fb26c8832e4db35", "3faa84d74f27b8c3",
    "3fa315d4e66e38b8", "3f9b7886ac3bd56d", "3f93c53550291d2d", "3f8c74f54880733d", "3f847ae147ae147b", "3f7d7a7384a15eb3",
    "3f753712a5b96096", "3f6e8954a3e38dea", "3f65fa0556964454", "3f5fa1eee6a82eaa", "3f56c3f76d338f61", "3f50624dd2f1a9fc",
    "3f47952936e77efc", "3f40f8dbb7c7807d", "3f386ddd4fe93e54", "3f3194d11211d043", "3f294e58b8868bbb", "3f22365f8a8fa5e7",
    "3ff0000000000000", "3fe707aa3f9e1202", "3fe093069178d379", "3fd7db4a2009c6e3", "3fd12b542ba56564", "3fc8b682a4336478",
    "3fc1c9194d504805", "3fb999999999999a", "3fb26c8832e4db35", "3faa84d74f27b8c3", "3fa315d4e66e38b8", "3f9b7886ac3bd56d",
    "3f93c53550291d2d", "3f8c74f54880733d", "3f847ae147ae147b", "3f7d7a7384a15eb3", "3f753712a5b96096", "3f6e8954a3e38dea",
    "3f65fa0556964454", "3f5fa1eee6a82eaa", "3f56c3f76d338f61", "3f50624dd2f1a9fc", "3f47952936e77efc", "3f40f8dbb7c7807d",
    "3f386ddd4fe93e54", "3f3194d11211d043", "3f294e58b8868bbb", "3f22365f8a8fa5e7",
)


def qwen_omegas(axes=QWEN_AXES, theta: float = QWEN_THETA) -> np.ndarray:
    """The 64 Qwen-Image frequencies, axis by axis: the frozen engine values for the default axes and theta, else
    the closed form theta^(-2j/d)."""
    if tuple(axes) == QWEN_AXES and theta == QWEN_THETA:
        return np.array([np.frombuffer(bytes.fromhex(h), dtype=">f8")[0] for h in QWEN_OMEGA_F64_HEX], np.float64)
    return np.concatenate([axis_omegas(d, theta) for d in axes])


def qwen_text_ids(n: int, first: int = 0) -> np.ndarray:
    """rope.zig:11-13: position p on all three axes."""
    p = np.arange(first, first + n, dtype=np.float32)
    return np.stack([p, p, p], axis=1)


def qwen_image_ids(h: int, w: int, pos: int, target_h: int | None = None, target_w: int | None = None) -> np.ndarray:
    """rope.zig:16-28: frame `pos`, centred rows and columns (half-pixel shifted for odd sides), f32 [h*w, 3]."""
    target_h = h if target_h is None else target_h
    target_w = w if target_w is None else target_w
    fh, fw = np.float32(h), np.float32(w)
    sh = -(fh - np.float32(h // 2)) + np.float32(0.5) * (np.float32(h % 2) - np.float32(target_h % 2))
    sw = -(fw - np.float32(w // 2)) + np.float32(0.5) * (np.float32(w % 2) - np.float32(target_w % 2))
    yy, xx = np.meshgrid(np.arange(h, dtype=np.float32), np.arange(w, dtype=np.float32), indexing="ij")
    ids = np.empty((h * w, 3), dtype=np.float32)
    ids[:, 0] = np.float32(pos)
    ids[:, 1] = (yy + sh).reshape(-1)
    ids[:, 2] = (xx + sw).reshape(-1)
    return ids


def qwen_table(ids: np.ndarray, om: np.ndarray | None = None, axes=QWEN_AXES):
    """rope.zig:31-45: cos, sin [N, 64] f32 from ids [N, 3] (angle = f64(id) * omega in f64)."""
    om = qwen_omegas(axes) if om is None else np.asarray(om, np.float64)
    cols = np.concatenate([np.full(d // 2, ax) for ax, d in enumerate(axes)])
    ang = ids.astype(np.float64)[:, cols] * om[None, :]
    s, c = engine_sincos(ang)
    return c.astype(np.float32), s.astype(np.float32)


def identity_rows(n: int, pairs: int = 64):
    """cos = 1, sin = 0 rows: tokens that are not rotated."""
    return np.ones((n, pairs), np.float32), np.zeros((n, pairs), np.float32)


def grid2d_table(n_text: int, gh: int, gw: int, theta: float = QWEN_THETA):
    """BASELINE's "2D RoPE, split h/w halves": interleaved pairs; pairs 0-31 (dims 0-63) rotate by the grid row r,
    pairs 32-63 (dims 64-127) by the column c, omega_j = theta^(-2j/64) for both; text rows first, un-rotated.
    Returns cos, sin [n_text + gh*gw, 64] f32."""
    om = axis_omegas(64, theta)                                   # 32 values
    r, c = np.meshgrid(np.arange(gh, dtype=np.float64), np.arange(gw, dtype=np.float64), indexing="ij")
    ang = np.concatenate([r.reshape(-1, 1) * om[None, :], c.reshape(-1, 1) * om[None, :]], axis=1)
    tc, ts = identity_rows(n_text)
    s, c = engine_sincos(ang)
    return np.concatenate([tc, c.astype(np.float32)]), np.concatenate([ts, s.astype(np.float32)])


def edit_table(n_text: int, frames: int, gh: int, gw: int):
    """BASELINE's image-edit layout: text (un-rotated), then `frames` gh x gw latents, latent f on frame axis f, rows
    and columns centred as rope.imageIds does; Qwen axes 16/56/56. cos, sin [n_text + frames*gh*gw, 64] f32."""
    ids = np.concatenate([qwen_image_ids(gh, gw, f) for f in range(frames)])
    c, s = qwen_table(ids)
    tc, ts = identity_rows(n_text)
    return np.concatenate([tc, c]), np.concatenate([ts, s])


def video3d_table(n_text: int, t: int, gh: int, gw: int, dims=(32, 48, 48), theta: float = QWEN_THETA):
    """BASELINE's video layout: text (un-rotated), then t x gh x gw tokens (frame-major); t/h/w take 32/48/48 dims
    (16/24/24 interleaved pairs), omega_{a,j} = theta^(-2j/d_a), integer positions. cos, sin [n_text + t*gh*gw, 64]."""
    om = np.concatenate([axis_omegas(d, theta) for d in dims])
    cols = np.concatenate([np.full(d // 2, ax) for ax, d in enumerate(dims)])
    tt, yy, xx = np.meshgrid(np.arange(t, dtype=np.float64), np.arange(gh, dtype=np.float64),
                             np.arange(gw, dtype=np.float64), indexing="ij")
    pos = np.stack([tt.reshape(-1), yy.reshape(-1), xx.reshape(-1)], axis=1)
    n = pos.shape[0]
    cos = np.empty((n_text + n, 64), np.float32)
    sin = np.empty((n_text + n, 64), np.float32)
    cos[:n_text], sin[:n_text] = identity_rows(n_text)
    step = 1 << 16                                                # chunked: 172k x 64 angles at a time is fine,
    for i in range(0, n, step):                                   # but keep the f64 temporaries small
        ang = pos[i:i + step][:, cols] * om[None, :]
        s, c = engine_sincos(ang)
        cos[n_text + i:n_text + i + step] = c
        sin[n_text + i:n_text + i + step] = s
    return cos, sin


# ------------------------------------------------------------------------------------------------ MiniMax H3
def _h3_axis(dim: int, area: float, i: np.ndarray) -> np.ndarray:
    """layout.zig:78-82: (i * (ratio / n) + (1 - ratio) / 2) * 32, ratio = dim / area, n = dim / 2, in f64."""
    ratio = np.float64(dim) / area
    n = np.float64(dim // 2)
    return (i.astype(np.float64) * (ratio / n) + (1.0 - ratio) / 2.0) * 32.0


def h3_positions(l: int, t: int, h: int, w: int, a: int, first_frame: bool = False) -> np.ndarray:
    """layout.zig:85-115: positions [S, 3] f64 (t, h, w) of the packed layout [text | cond | audio | video]."""
    area = np.sqrt(np.float64(h * w))
    hh, ww = np.meshgrid(np.arange(h // 2), np.arange(w // 2), indexing="ij")
    ph, pw = _h3_axis(h, area, hh.reshape(-1)), _h3_axis(w, area, ww.reshape(-1))
    w_lo = _h3_axis(w, area, np.array([0]))[0]
    w_hi = _h3_axis(w, area, np.array([w // 2 - 1]))[0]
    rows = []
    i = np.arange(l, dtype=np.float64)
    rows.append(np.stack([i, np.zeros(l), np.zeros(l)], axis=1))
    cursor = np.float64(l)
    if first_frame:
        rows.append(np.stack([np.full(ph.shape, cursor), ph, pw], axis=1))
    for ch in range(2):
        ai = cursor + np.arange(a, dtype=np.float64)
        rows.append(np.stack([ai, np.zeros(a), np.full(a, w_lo if ch == 0 else w_hi)], axis=1))
    cum = 0.0
    for k in range(t):
        rows.append(np.stack([np.full(ph.shape, cursor + cum), ph, pw], axis=1))
        cum += H3_FRAME_RESCALE * H3_FRAME_PER_TOKEN[k % 5]
    return np.concatenate(rows).astype(np.float64)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round to nearest even, finite inputs (layout.zig:31-34)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def h3_rope_table(pos: np.ndarray, inv_freq: np.ndarray) -> np.ndarray:
    """layout.zig:117-134: bf16 bits [S, 48, 2, 2]: angle = f32(pos) * inv_freq (f32), cos/sin in f64 -> f32 -> bf16;
    entry (r, ax*16 + j) = [c, -s, s, c]."""
    inv = np.asarray(inv_freq, np.float32)
    assert inv.shape == (16,)
    ang = pos.astype(np.float32)[:, :, None] * inv[None, None, :]            # f32 product, [S, 3, 16]
    s, c = engine_sincos(ang.astype(np.float64))
    c = c.astype(np.float32).reshape(-1, 48)
    s = s.astype(np.float32).reshape(-1, 48)
    out = np.empty((pos.shape[0], 48, 2, 2), np.uint16)
    out[..., 0, 0] = f32_to_bf16_bits(c)
    out[..., 0, 1] = f32_to_bf16_bits(-s)
    out[..., 1, 0] = f32_to_bf16_bits(s)
    out[..., 1, 1] = f32_to_bf16_bits(c)
    return out
