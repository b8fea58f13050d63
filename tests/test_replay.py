"""The capture reader of the replay gate (CPU): records, notes, refs and the comparison it reports."""
from __future__ import annotations

import numpy as np
import pytest

from localrouter_amd import replay
from tests import capture_util


def test_read_ops_and_refs(tmp_path):
    q = np.arange(3 * 2 * 128, dtype=np.uint16).reshape(1, 3, 2, 128)
    w = np.linspace(-1, 1, 128, dtype=np.float32)
    capture_util.write(tmp_path, [
        {"note": "sigmas", "values": [1.0, 0.5]},
        {"name": "blk0.attn", "kind": "attention", "attrs": {"impl": "stk", "causal": False}, "ins": {"q": q, "k": q,
         "v": q}, "outs": {"y": q.reshape(1, 3, 256)}},
        {"name": "blk0.norm", "kind": "rms_norm_f32", "ins": {"w": w}, "outs": {"y": w}},
    ])
    ops = replay.read_ops(tmp_path)
    assert [o.kind for o in ops] == ["attention", "rms_norm_f32"] and [o.i for o in ops] == [1, 2]
    assert np.array_equal(replay.load_ref(tmp_path, ops[0].ins["q"]), q)
    assert replay.load_ref(tmp_path, ops[0].outs["y"]).shape == (1, 3, 256)
    assert np.array_equal(replay.load_ref(tmp_path, ops[1].ins["w"]), w)
    bad = dict(ops[0].ins["q"], shape=[1, 3, 2, 129])
    with pytest.raises(ValueError):
        replay.load_ref(tmp_path, bad)
    with pytest.raises(ValueError):
        replay.load_ref(tmp_path, dict(ops[0].ins["q"], dtype="complex64"))


def test_compare_reports_equal_within_and_differ():
    a = np.array([0x3F80, 0x4000, 0xBF80] * 4, dtype=np.uint16)      # 1, 2, -1, ...
    assert replay.compare(a, a)[:2] == (True, True)
    b = a.copy(); b[0] = 0x3F81                                       # 1 + 2^-7
    eq, ok, mx, _ = replay.compare(b, a)
    assert not eq and ok and abs(mx - 2 ** -7) < 1e-9                 # mean-abs 2^-7 / 12 is within the bar too
    c = a.copy(); c[1] = 0x4040                                       # 3 instead of 2
    assert replay.compare(c, a)[:2] == (False, False)
    assert replay.compare(a[:2], a)[:2] == (False, False)


def test_classify_mask():
    keep = np.array([True, False, True, True])
    how, k = replay.classify_mask(keep[None, None, None, :], 1, 3, 4)
    assert how == "keys" and np.array_equal(k, keep[None])
    add = np.where(keep, 0.0, -np.inf).astype(np.float32)[None, None, None, :]      # additive form
    assert replay.classify_mask(add, 2, 3, 4)[0] == "keys"
    assert replay.classify_mask(np.tril(np.ones((4, 4), bool))[None, None], 1, 4, 4)[0] == "causal"
    assert replay.classify_mask(np.eye(4, dtype=bool)[None, None], 1, 4, 4)[0] is None
    per_head = np.ones((1, 2, 3, 4), bool); per_head[0, 1, :, 0] = False           # heads differ
    assert replay.classify_mask(per_head, 1, 3, 4)[0] is None


def test_classify_mask_bf16_bits():
    """A bf16 additive mask arrives as uint16 bits: (1 - keep) * -10000 gives -0.0 (0x8000) for kept keys."""
    keep = np.array([True, True, False, True])
    add = ((1.0 - keep) * -10000.0).astype(np.float32)
    assert np.signbit(add[keep]).all()                                              # kept keys are -0.0
    bits = (add.view(np.uint32) >> 16).astype(np.uint16)[None, None, None, :]       # truncated to bf16
    how, k = replay.classify_mask(bits, 1, 3, 4)
    assert how == "keys" and np.array_equal(k, keep[None])
    # a batch that keeps no key is not replayed (SDPA gives NaN rows)
    none_kept = np.full((2, 1, 1, 4), 0xC61C, np.uint16)                            # bf16 -1e4 (truncated) everywhere ...
    none_kept[0] = 0                                                                # ... but batch 0 keeps all
    assert replay.classify_mask(none_kept, 2, 3, 4) == (None, None)
    assert replay.classify_mask(np.zeros((1, 1, 3, 4), bool), 1, 3, 4) == (None, None)

