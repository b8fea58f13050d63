"""The replay gate on the GPU: a capture in the reference's recorder format (tools/twin/stk_twin/rec.py:1-9) with an
unmasked attention, a causal segment (p0, nkeys) with GQA, a q-part rms_rope, SDPA records with a key-padding mask, a
causal mask and an unsupported (diagonal) mask, and a skipped kind; expected outputs from the CPU oracle. Every
replayed op must pass the bar, and a perturbed expected output must be reported."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests import capture_util
from tests._util import bf16_f32

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from localrouter_amd import replay  # noqa: E402


def _capture(root, perturb=False):
    q = oracle.synth_bf16(61, 1, (1, 100, 4, 128))
    k = oracle.synth_bf16(61, 2, (1, 150, 2, 128))
    v = oracle.synth_bf16(61, 3, (1, 150, 2, 128))
    s = 1.0 / np.sqrt(128.0)
    y0 = oracle.attention(bf16_f32(q[0]), bf16_f32(k[0]), bf16_f32(v[0]), scale=s)
    qs = np.ascontiguousarray(q[:, 50:100])
    y1 = oracle.attention(bf16_f32(qs[0]), bf16_f32(k[0]), bf16_f32(v[0]), p0=50, nkeys=150, causal=True, scale=s)
    qkv = oracle.synth_bf16(61, 4, (1, 40, 3, 2, 128))
    w = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(61, 5, (128,)))).astype(np.float32)
    ang = np.random.default_rng(61).uniform(-3, 3, (40, 64))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y2 = oracle.rms_rope(np.ascontiguousarray(qkv[0, :, 0]), w, table_kind=oracle.TABLE_COSSIN_F32, ta=cos, tb=sin,
                         pairing=oracle.PAIR_INTERLEAVED, rot=128, eps=1e-6)
    keep = np.random.default_rng(62).random(150) < 0.7                 # key padding: 30 % of the keys dropped
    kept = np.nonzero(keep)[0]
    yk = oracle.f32_to_bf16(oracle.attention(bf16_f32(q[0]), bf16_f32(k[0][kept]), bf16_f32(v[0][kept]), scale=s))
    yk = yk.reshape(1, 100, 512)
    kq = oracle.synth_bf16(61, 6, (1, 150, 4, 128))
    yc = oracle.f32_to_bf16(oracle.attention(bf16_f32(kq[0]), bf16_f32(k[0]), bf16_f32(v[0]), causal=True, scale=s))
    yc = yc.reshape(1, 150, 512)
    b0 = oracle.f32_to_bf16(y0).reshape(1, 100, 512)
    if perturb:
        b0 = oracle.f32_to_bf16(bf16_f32(b0) + 0.25)
    capture_util.write(root, [
        {"name": "blk0.attn", "kind": "attention", "attrs": {"impl": "stk", "causal": False},
         "ins": {"q": q, "k": k, "v": v}, "outs": {"y": b0}},
        {"note": "segment"},
        {"name": "te.attn.seg1", "kind": "attention", "attrs": {"impl": "stk", "causal": True, "p0": 50, "nkeys": 150},
         "ins": {"q": qs, "k": k, "v": v}, "outs": {"y": oracle.f32_to_bf16(y1).reshape(1, 50, 512)}},
        {"name": "blk0.q_rope", "kind": "rms_rope", "attrs": {"part": 0, "eps": 1e-6},
         "ins": {"qkv": qkv, "w": w, "cos": cos, "sin": sin}, "outs": {"y": oracle.f32_to_bf16(y2)[None]}},
        {"name": "blk0.mlp", "kind": "swiglu", "ins": {"gu": qkv.reshape(40, -1)}, "outs": {"y": qkv.reshape(40, -1)}},
        {"name": "te.attn", "kind": "attention", "attrs": {"impl": "sdpa", "masked": True},
         "ins": {"q": q, "k": k, "v": v, "mask": keep[None, None, None, :]}, "outs": {"y": yk}},
        {"name": "te.attn_causal", "kind": "attention", "attrs": {"impl": "sdpa", "masked": True},
         "ins": {"q": kq, "k": k, "v": v, "mask": np.tril(np.ones((150, 150), bool))[None, None]}, "outs": {"y": yc}},
        {"name": "te.attn_diag", "kind": "attention", "attrs": {"impl": "sdpa", "masked": True},
         "ins": {"q": kq, "k": k, "v": v, "mask": np.eye(150, dtype=bool)[None, None]}, "outs": {"y": yc}},
    ])


def test_replay_capture(tmp_path):
    print("\n[replay] synthetic capture", flush=True)
    _capture(tmp_path)
    st = replay.replay(tmp_path)
    # replayed: two attentions, the rms_rope, the key-padding and the causal SDPA masks; skipped: swiglu, the diagonal
    assert (st.differ, st.skipped) == (0, 2) and st.equal + st.within == 5, st.notes


def test_replay_reports_a_difference(tmp_path):
    print("\n[replay] perturbed capture", flush=True)
    _capture(tmp_path, perturb=True)
    st = replay.replay(tmp_path)
    assert st.differ == 1 and "DIFFERS" in st.notes[0], st.notes


def test_replay_chained(tmp_path):
    """An rms_rope whose recorded output is the q of the next attention (the same blob): chained, the attention reads
    the replayed rms_rope output; both stay within the bar."""
    print("\n[replay] chained", flush=True)
    qkv = oracle.synth_bf16(63, 1, (1, 120, 3, 2, 128))
    w = np.ones(128, np.float32)
    ang = np.random.default_rng(63).uniform(-3, 3, (120, 64))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    qn = oracle.f32_to_bf16(oracle.rms_rope(np.ascontiguousarray(qkv[0, :, 0]), w, table_kind=oracle.TABLE_COSSIN_F32,
                                            ta=cos, tb=sin, rot=128, eps=1e-6))
    k = oracle.synth_bf16(63, 2, (1, 120, 2, 128))
    v = oracle.synth_bf16(63, 3, (1, 120, 2, 128))
    y = oracle.attention(bf16_f32(qn), bf16_f32(k[0]), bf16_f32(v[0]), scale=1.0 / np.sqrt(128.0))
    capture_util.write(tmp_path, [
        {"name": "q_rope", "kind": "rms_rope", "attrs": {"part": 0, "eps": 1e-6},
         "ins": {"qkv": qkv, "w": w, "cos": cos, "sin": sin}, "outs": {"y": qn[None]}},
        {"name": "attn", "kind": "attention", "attrs": {"impl": "stk", "causal": False},
         "ins": {"q": qn[None], "k": k, "v": v}, "outs": {"y": oracle.f32_to_bf16(y).reshape(1, 120, 256)}},
    ])
    for chained in (False, True):
        st = replay.replay(tmp_path, chained=chained)
        assert st.differ == 0 and st.equal + st.within == 2, (chained, st.notes)

