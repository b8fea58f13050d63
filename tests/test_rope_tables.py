"""Host RoPE table builders (localrouter_amd.rope) against the reference's own data and test vectors:
kernels/qwen_image/rope_omega.json (committed as tests/golden/rope_omega.json), the image-id test of
src/engines/qwen_image/rope.zig:47-52, the layout tests of src/engines/minimax_h3/layout.zig:186-215, and the engines'
portable sincos (smath.zig:40-52): its own accuracy bound (smath.zig:128-135), relative accuracy at the zeros, where
the three-part reduction decides the result, and its bits on tests/golden/sincos.npz (written by
tests/golden/make_sincos.py from the reference's Python statement of the same routine)."""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest

from localrouter_amd import rope

GOLDEN = Path(__file__).resolve().parent / "golden"


def _frozen_omegas():
    d = json.loads((GOLDEN / "rope_omega.json").read_text())
    assert d["theta"] == 10000.0 and d["axes"] == [16, 56, 56]
    return np.array([struct.unpack(">d", bytes.fromhex(h))[0] for h in d["omega_f64_be_hex"]])


def _sincos_fixture():
    f = np.load(GOLDEN / "sincos.npz")
    return f["x"].view(np.float64), f["sin"], f["cos"]


def test_engine_sincos_bits():
    x, s_bits, c_bits = _sincos_fixture()
    assert x.size > 4000
    s, c = rope.engine_sincos(x)
    assert np.array_equal(s.view(np.uint64), s_bits) and np.array_equal(c.view(np.uint64), c_bits)
    # the fixture tells the routine from libm: numpy's sin and cos differ from it in the last bit on many angles
    assert (np.sin(x).view(np.uint64) != s_bits).sum() > 100


def test_engine_sincos_accuracy_bound():
    """smath.zig:128-135: within 4e-15 of libm over -3000, -3000 + 0.7317, ... < 3000; and special values."""
    x = -3000.0 + 0.7317 * np.arange(8201)
    x = x[x < 3000.0]
    s, c = rope.engine_sincos(x)
    assert np.abs(s - np.sin(x)).max() <= 4e-15 and np.abs(c - np.cos(x)).max() <= 4e-15
    s, c = rope.engine_sincos(np.array([0.0, np.pi / 6, np.pi / 2, np.pi, -np.pi / 2]))
    assert s[0] == 0.0 and c[0] == 1.0
    assert abs(s[1] - 0.5) <= 1.2e-16 and abs(c[2]) <= 1e-16 and c[3] == -1.0 and s[4] == -1.0


def test_engine_sincos_relative_accuracy_at_zeros():
    """The three parts of pi / 2 sum to it within 8.5e-32 (against 60 digits of pi), so near k pi / 2, where the result
    is tiny, the routine is within k 1e-31 + 4 ulp of libm's exactly reduced sin and cos; a reduction that drops the
    third part misses by k 2e-21, a sizeable fraction of results of 1e-18."""
    from fractions import Fraction
    pi = Fraction("3.141592653589793238462643383279502884197169399375105820974944")
    assert abs(pi / 2 - (Fraction(rope.PIO2_1) + Fraction(rope.PIO2_2) + Fraction(rope.PIO2_3))) < Fraction(1, 10 ** 31)
    k = np.concatenate([np.arange(1, 2000), [65535, 2 ** 19]]).astype(np.float64)
    x = k * (np.pi / 2)
    s, c = rope.engine_sincos(x)
    for m, got, ref in ((k % 2 == 0, s, np.sin(x)), (k % 2 == 1, c, np.cos(x))):
        assert (np.abs(got[m] - ref[m]) <= k[m] * 1e-31 + 4 * np.spacing(np.abs(ref[m]))).all()


@pytest.mark.parametrize("name,value", [("PIO2_3", 0.0), ("S6", 0.0), ("C3", 2.48015872894767294178e-04),
                                        ("INVPIO2", 0.6366)])
def test_engine_sincos_planted_mistakes_fail(monkeypatch, name, value):
    """A dropped reduction term, a dropped or mistyped kernel coefficient, a coarse 2/pi: each changes bits of the
    fixture."""
    x, s_bits, c_bits = _sincos_fixture()
    if name in ("S6", "C3"):
        coef = list(rope.SIN_COEF if name == "S6" else rope.COS_COEF)
        coef[5 if name == "S6" else 2] = value
        monkeypatch.setattr(rope, "SIN_COEF" if name == "S6" else "COS_COEF", tuple(coef))
    else:
        monkeypatch.setattr(rope, name, value)
    s, c = rope.engine_sincos(x)
    assert not (np.array_equal(s.view(np.uint64), s_bits) and np.array_equal(c.view(np.uint64), c_bits))


def test_qwen_omegas_are_the_engine_bits():
    assert np.array_equal(rope.qwen_omegas(), _frozen_omegas())


def test_qwen_omegas_recipe_and_closed_form():
    """The fixture's stated recipe (torch float64 1 / 10000 ** linspace(0, (d - 2) / d, d / 2) per axis, as tfimage
    computes it) reproduces every frozen bit; the closed form theta^(-2j/d) agrees to a few f64 ulp (linspace's
    two-sided stepping rounds differently from 2j/d)."""
    torch = pytest.importorskip("torch")
    frozen = _frozen_omegas()
    recipe = np.concatenate([(1.0 / 10000.0 ** torch.linspace(0, (d - 2) / d, d // 2, dtype=torch.float64)).numpy()
                             for d in (16, 56, 56)])
    assert np.array_equal(recipe.view(np.uint64), frozen.view(np.uint64))
    closed = np.concatenate([rope.axis_omegas(d) for d in (16, 56, 56)])
    assert np.all(np.abs(closed - frozen) <= 16 * np.spacing(frozen))
    # a plausible mistake (2j/(d-2) instead of 2j/d, or theta 1e5) is far outside that
    wrong = np.concatenate([1.0 / 10000.0 ** (2 * np.arange(d // 2) / (d - 2)) for d in (16, 56, 56)])
    assert np.abs(wrong - frozen).max() > 1e-3


def test_image_ids_reference_vector():
    """rope.zig:47-52: a 4x3 grid at position 7 starts at (7, -2, -2) and ends at (7, 1, 0)."""
    ids = rope.qwen_image_ids(4, 3, 7, 4, 3)
    assert ids.dtype == np.float32
    assert ids[0].tolist() == [7.0, -2.0, -2.0]
    assert ids[11].tolist() == [7.0, 1.0, 0.0]


def test_text_ids_and_table():
    ids = rope.qwen_text_ids(3, first=5)
    assert ids.tolist() == [[5, 5, 5], [6, 6, 6], [7, 7, 7]]
    c, s = rope.qwen_table(ids)
    om = rope.qwen_omegas()
    assert c.dtype == np.float32 and c.shape == (3, 64)
    ang = 6.0 * om
    assert np.array_equal(c[1], np.cos(ang).astype(np.float32))
    assert np.array_equal(s[1], np.sin(ang).astype(np.float32))


def test_grid2d_table_layout():
    c, s = rope.grid2d_table(3, 4, 5)
    assert c.shape == (3 + 20, 64)
    assert np.all(c[:3] == 1) and np.all(s[:3] == 0)
    om = 1.0 / 10000.0 ** (np.arange(32) * 2 / 64)
    r, col = 2, 3
    row = 3 + r * 5 + col
    assert np.allclose(c[row, :32], np.cos(r * om), atol=1e-7)
    assert np.allclose(s[row, 32:], np.sin(col * om), atol=1e-7)


def test_video3d_table_layout():
    c, s = rope.video3d_table(2, 3, 4, 5)
    assert c.shape == (2 + 60, 64)
    om_t = 1.0 / 10000.0 ** (np.arange(16) * 2 / 32)
    om_h = 1.0 / 10000.0 ** (np.arange(24) * 2 / 48)
    t, h, w = 2, 1, 4
    row = 2 + (t * 4 + h) * 5 + w
    assert np.allclose(c[row, :16], np.cos(t * om_t), atol=1e-7)
    assert np.allclose(s[row, 16:40], np.sin(h * om_h), atol=1e-7)
    assert np.allclose(c[row, 40:], np.cos(w * om_h), atol=1e-7)


def test_edit_table_frames():
    c, s = rope.edit_table(2, 3, 4, 4)
    assert c.shape == (2 + 48, 64)
    # frame axis pairs 0..7 differ between the three latents, the row/column pairs repeat
    assert np.array_equal(c[2 + 0 * 16 + 5, 8:], c[2 + 2 * 16 + 5, 8:])
    assert not np.array_equal(c[2 + 0 * 16 + 5, :8], c[2 + 2 * 16 + 5, :8])


def test_h3_layout_sizes_and_positions():
    """layout.zig:191-214: sizes of two layouts; the condition and target frame zero share positions; audio starts at
    the text length."""
    pos = rope.h3_positions(69, 17, 28, 48, 93)
    assert pos.shape == (69 + 186 + 17 * 14 * 24, 3)
    pos = rope.h3_positions(4, 2, 4, 6, 3, first_frame=True)
    assert pos.shape == (28, 3)
    assert np.array_equal(pos[4], pos[16])
    assert pos[10][0] == 4.0


def test_h3_rope_table_entries():
    pos = rope.h3_positions(4, 2, 4, 6, 3)
    inv = (1.0 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
    tab = rope.h3_rope_table(pos, inv)
    assert tab.shape == (pos.shape[0], 48, 2, 2)
    r, ax, j = 9, 1, 5
    ang = np.float32(pos[r, ax]) * inv[j]
    c = np.float32(np.cos(np.float64(ang)))
    s = np.float32(np.sin(np.float64(ang)))
    bits = lambda x: rope.f32_to_bf16_bits(np.array([x], np.float32))[0]  # noqa: E731
    assert tab[r, ax * 16 + j].tolist() == [[bits(c), bits(-s)], [bits(s), bits(c)]]
