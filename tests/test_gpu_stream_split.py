"""GPU parity of the streaming kernel's split tail (localrouter_amd/csrc/attn_stream.hip): the query blocks past the
last whole round are cut over all workgroups along their key tiles, each piece leaves an fp32 partial (O, m, l), and
the last piece to arrive merges them in piece order. Shapes are chosen so that cut blocks have 2, 3 and 4 pieces, the
whole grid is tail (fewer blocks than CUs), GQA and a ragged last key tile; rows of cut blocks are checked against the
CPU oracle of the reference's chain (tests/_util.py bar). Repeated calls must give identical bits (the merge order
does not depend on which piece arrives last), and overflow inside cut blocks must reach the exact recomputation."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_f32, from_dev, to_dev
from tests.test_stream_schedule import schedule

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from localrouter_amd import ops  # noqa: E402


def _cus():
    return min(torch.cuda.get_device_properties(0).multi_processor_count, 256)


def _case(seed, Sq, Sk, H, HK):
    q = oracle.synth_bf16(seed, 1, (Sq, H, 128))
    k = oracle.synth_bf16(seed, 2, (Sk, HK, 128))
    v = oracle.synth_bf16(seed, 3, (Sk, HK, 128))
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-np.pi, np.pi, size=(max(Sq, Sk), 64))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    return q, k, v, cos, sin


def _run(q, k, v, cos, sin, Sq, Sk):
    tq = (torch.from_numpy(np.ascontiguousarray(cos[:Sq])).cuda(), torch.from_numpy(np.ascontiguousarray(sin[:Sq])).cuda())
    tk = (torch.from_numpy(np.ascontiguousarray(cos[:Sk])).cuda(), torch.from_numpy(np.ascontiguousarray(sin[:Sk])).cuda())
    out = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), table_kind=ops.TABLE_COSSIN_F32, q_table=tq,
                              k_table=tk, eps=1e-6)
    torch.cuda.synchronize()
    return from_dev(out)


def _oracle_rows(q, k, v, cos, sin, Sq, Sk, rows):
    """The reference's chain on the given query rows: q, k normalised and rotated, stored as bf16, then attention over
    every key (the oracle's fp32 flash path)."""
    qh = oracle.rms_rope(np.ascontiguousarray(q[rows]), None, table_kind=oracle.TABLE_COSSIN_F32,
                         ta=np.ascontiguousarray(cos[rows]), tb=np.ascontiguousarray(sin[rows]), eps=1e-6)
    kh = oracle.rms_rope(k, None, table_kind=oracle.TABLE_COSSIN_F32, ta=np.ascontiguousarray(cos[:Sk]),
                         tb=np.ascontiguousarray(sin[:Sk]), eps=1e-6)
    bf = lambda x: oracle.bf16_to_f32(oracle.f32_to_bf16(x))
    return oracle.attention(bf(qh), bf(kh), oracle.bf16_to_f32(v), precise=False)


@pytest.mark.parametrize("Sq,Sk,H,HK", [
    (1280, 1280, 24, 24),     # BASELINE cfg1: 120 blocks, all of them cut over 256 workgroups (2-4 pieces)
    (300, 5000, 2, 2),        # 4 blocks of 79 tiles over 12 workgroups, a partial last query block
    (2048, 2048, 8, 2),       # GQA 4:1, 64 blocks of 32 tiles
    (999, 1100, 7, 7),        # ragged last key tile and query block
    (65792, 512, 1, 1),       # 257 blocks: one whole round, then one block cut over 3 workgroups
    (4608, 4608, 24, 24),     # BASELINE cfg2: 176 of 432 blocks cut, 2-3 pieces each
    (2304, 4000, 24, 6),      # 216 blocks of 63 tiles, all tail, GQA 4:1
])
def test_split_tail_parity(Sq, Sk, H, HK):
    nwg = _cus()
    work, pieces, p = schedule(Sq, H, Sk, nwg)
    assert p["nt"] is not None, "the shape must take the split schedule"
    npieces = sorted({len(ps) for ps in pieces.values()})
    print(f"\n[split] Sq={Sq} Sk={Sk} H={H} HK={HK} cut blocks {len(pieces)} pieces {npieces}", flush=True)
    q, k, v, cos, sin = _case(61, Sq, Sk, H, HK)
    got = _run(q, k, v, cos, sin, Sq, Sk)
    # rows of every cut block of head 0 and of the last head (at most 12 blocks), plus a few rows of the whole blocks
    nqb = (Sq + 255) // 256
    cut = sorted(p["nwhole"] + i for i in pieces)
    rows = set()
    for blk in [b for b in cut if b // nqb in (0, H - 1)][:12]:
        r0 = (blk % nqb) * 256
        rows.update(range(r0, min(r0 + 256, Sq), 3))
    rows.update(np.random.default_rng(1).choice(Sq, size=min(Sq, 64), replace=False).tolist())
    rows = np.array(sorted(rows))
    heads = sorted({0, H - 1})
    ref = _oracle_rows(q, k, v, cos, sin, Sq, Sk, rows)
    for h in heads:
        assert_close(got[rows][:, h], ref[:, h], what=f"split Sq={Sq} head {h}")
    assert np.isfinite(bf16_f32(got)).all()


def test_split_repeats_are_identical():
    """BASELINE cfg2's shape (176 of 432 blocks cut, 2-3 pieces each): three calls, the same bits."""
    Sq = Sk = 4608
    H = 24
    print(f"\n[split repeats] Sq={Sq} H={H}", flush=True)
    q, k, v, cos, sin = _case(62, Sq, Sk, H, H)
    first = _run(q, k, v, cos, sin, Sq, Sk)
    for _ in range(2):
        assert np.array_equal(_run(q, k, v, cos, sin, Sq, Sk), first)


def test_split_overflow_reaches_exact_recomputation():
    """Norm weights 5.0 on sign-ramp inputs (every |x| 1, eps 0: the prepared operands are exact) make the exp2-domain
    scores rise by ~400 along the keys: pieces starting at the first tile overflow against their fixed reference,
    later pieces do not. The merged blocks must come out exact (the merging workgroup recomputes them)."""
    from tests.test_gpu_attention import _sign_ramp, _sign_ramp_expected
    Sq, Sk, H = 2048, 2048, 8
    work, pieces, p = schedule(Sq, H, Sk, _cus())
    assert p["nt"] is not None
    print(f"\n[split overflow] Sq={Sq} Sk={Sk} H={H} cut blocks {len(pieces)}", flush=True)
    q, k = _sign_ramp(Sq, Sk, H)
    v = oracle.synth_bf16(63, 3, (Sk, H, 128))
    w5 = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    out = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=w5, k_norm=w5, table_kind=0, eps=0.0)
    torch.cuda.synchronize()
    got = from_dev(out)
    rows = np.arange(0, Sq, 5)
    exp = _sign_ramp_expected(q[rows], k, v, 5.0, ops.SCALE_128)
    assert_close(got[rows], exp, what="split overflow")


@pytest.mark.parametrize("Sq,Sk,H,HK", [(1280, 4500, 24, 24), (2048, 4096, 8, 2), (999, 4100, 9, 9),
                                        (65792, 4096, 1, 1)])
def test_rows_split_tail_parity(Sq, Sk, H, HK):
    """The split tail over key rows (lr_attention_bf16_ws: the streaming kernel gathering key tiles from the rows, its
    partials and counters in the caller's workspace): rows of cut blocks against the CPU oracle, three calls the same
    bits."""
    work, pieces, p = schedule(Sq, H, Sk, _cus())
    assert p["nt"] is not None, "the shape must take the split schedule"
    print(f"\n[rows split] Sq={Sq} Sk={Sk} H={H} HK={HK} cut blocks {len(pieces)}", flush=True)
    q, k, v, _, _ = _case(64, Sq, Sk, H, HK)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    ws = torch.empty(ops.attention_ws_bytes(Sq, H, Sk), dtype=torch.uint8, device="cuda")
    got = from_dev(ops.attention_ws(dq, dk, dv, workspace=ws))
    for _ in range(2):
        again = from_dev(ops.attention_ws(dq, dk, dv, workspace=ws))
        assert np.array_equal(again, got)
    nqb = (Sq + 255) // 256
    cut = sorted(p["nwhole"] + i for i in pieces)
    rows = set()
    for blk in [b for b in cut if b // nqb in (0, H - 1)][:12]:
        r0 = (blk % nqb) * 256
        rows.update(range(r0, min(r0 + 256, Sq), 3))
    rows.update(np.random.default_rng(2).choice(Sq, size=min(Sq, 64), replace=False).tolist())
    rows = np.array(sorted(rows))
    ref = oracle.attention(bf16_f32(np.ascontiguousarray(q[rows])), bf16_f32(k), bf16_f32(v), precise=False)
    for h in sorted({0, H - 1}):
        assert_close(got[rows][:, h], ref[:, h], what=f"rows split Sq={Sq} head {h}")
    assert np.isfinite(bf16_f32(got)).all()
