"""The C++ host RoPE builders (include/lr_rope.h, localrouter_amd/csrc/rope_host.cpp) on the CPU: the reference's own
vectors (src/engines/qwen_image/rope.zig:47-52, src/engines/minimax_h3/layout.zig:186-215, the frozen
kernels/qwen_image/rope_omega.json bits) and bit equality with the numpy builders of localrouter_amd.rope, which
tests/test_rope_tables.py pins to the same vectors and closed forms."""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from localrouter_amd import _lib, rope, rope_host


def test_header_and_exports_agree():
    text = re.sub(r"/\*.*?\*/", "", rope_host.HEADER.read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(?:void|int|int64_t)\s+(lr_rope_\w+)\s*\(", text)))
    assert sorted(rope_host.SIGNATURES) == declared
    L = rope_host.lib()
    for name in declared:
        assert hasattr(L, name)


def test_sincos_is_the_engine_bits():
    """The library's sincos (every table builder's) on the bits of tests/golden/sincos.npz, and on the angles of a
    whole Qwen-Image table against the numpy restatement."""
    f = np.load(Path(__file__).resolve().parent / "golden" / "sincos.npz")
    s, c = rope_host.sincos(f["x"].view(np.float64))
    assert np.array_equal(s.view(np.uint64), f["sin"]) and np.array_equal(c.view(np.uint64), f["cos"])
    x = np.random.default_rng(5).uniform(-2e5, 2e5, 200000)
    s, c = rope_host.sincos(x)
    rs, rc = rope.engine_sincos(x)
    assert np.array_equal(s.view(np.uint64), rs.view(np.uint64)) and np.array_equal(c.view(np.uint64), rc.view(np.uint64))
    assert rope_host.lib().lr_rope_sincos(None, 4, None, None) == 1


def test_omegas_are_the_engine_bits():
    assert np.array_equal(rope_host.qwen_omegas().view(np.uint64), rope.qwen_omegas().view(np.uint64))


def test_image_ids_reference_vector():
    """rope.zig:47-52: a 4x3 grid at position 7 starts at (7, -2, -2) and ends at (7, 1, 0)."""
    ids = rope_host.qwen_image_ids(4, 3, 7, 4, 3)
    assert ids[0].tolist() == [7.0, -2.0, -2.0]
    assert ids[11].tolist() == [7.0, 1.0, 0.0]


@pytest.mark.parametrize("h,w,th,tw", [(4, 3, 4, 3), (5, 7, 4, 8), (64, 64, 64, 64), (1, 9, 2, 9)])
def test_image_and_text_ids_match_numpy(h, w, th, tw):
    assert np.array_equal(rope_host.qwen_image_ids(h, w, 3, th, tw), rope.qwen_image_ids(h, w, 3, th, tw))
    assert np.array_equal(rope_host.qwen_text_ids(11, 5), rope.qwen_text_ids(11, 5))


def test_qwen_table_matches_numpy():
    ids = np.concatenate([rope.qwen_text_ids(512), rope.qwen_image_ids(64, 64, 1), rope.qwen_image_ids(5, 7, 2, 6, 6)])
    for om in (None, np.concatenate([rope.axis_omegas(d) for d in (16, 56, 56)])):
        c, s = rope_host.qwen_table(ids, om)
        rc, rs = rope.qwen_table(ids, om)
        assert np.array_equal(c, rc) and np.array_equal(s, rs)


def test_baseline_tables_match_numpy():
    for a, b in [(rope_host.grid2d_table(256, 32, 32), rope.grid2d_table(256, 32, 32)),
                 (rope_host.grid2d_table(512, 64, 64), rope.grid2d_table(512, 64, 64)),
                 (rope_host.edit_table(512, 3, 64, 64), rope.edit_table(512, 3, 64, 64)),
                 (rope_host.video3d_table(512, 5, 44, 80), rope.video3d_table(512, 5, 44, 80))]:
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_h3_layout_reference_vectors():
    """layout.zig:191-214: sizes of two layouts; the condition and target frame zero share positions; audio starts at
    the text length."""
    assert rope_host.h3_rows(69, 17, 28, 48, 93) == 69 + 186 + 17 * 14 * 24
    pos = rope_host.h3_positions(4, 2, 4, 6, 3, first_frame=True)
    assert pos.shape == (28, 3)
    assert np.array_equal(pos[4], pos[16])
    assert pos[10][0] == 4.0


@pytest.mark.parametrize("args", [(4, 2, 4, 6, 3, True), (69, 17, 28, 48, 93, False), (512, 13, 60, 104, 0, True)])
def test_h3_positions_and_table_match_numpy(args):
    pos = rope_host.h3_positions(*args)
    assert np.array_equal(pos, rope.h3_positions(*args[:5], first_frame=args[5]))
    inv = (1.0 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
    assert np.array_equal(rope_host.h3_rope_table(pos, inv), rope.h3_rope_table(pos, inv))


def test_rejects_bad_arguments():
    L = rope_host.lib()
    assert L.lr_rope_qwen_image_ids(None, 4, 4, 0, 4, 4) == 1
    assert L.lr_rope_grid2d_table(-1, 4, 4, 10000.0, None, None) == 1
    assert L.lr_rope_h3_rows(1, 1, 1, 4, 0, 0) == -1
    with pytest.raises(_lib.LrError):
        rope_host.qwen_image_ids(0, 4, 0)
