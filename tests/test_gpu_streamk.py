"""GPU parity of the stream-K configuration of the joint attention (LR_ATTN_CFG_PAIR_SK_W4: one workgroup per CU over
the blocks' key tiles laid end to end; both parts of a block cut between two workgroups stored as partials in the
workspace's stream-K area and merged by a second kernel).

The schedule runs when the call has at least as many 256-query blocks (ceil(Sq / 256) * H) as the device has CUs
(256 on MI355X) and whole blocks would leave more than 3% of the last round idle; every shape below qualifies. Each
is checked against the oracle (same bar as every attention test) and against the whole-block PAIR_W4 configuration.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_f32, from_dev, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from localrouter_amd import ops  # noqa: E402


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _streamk_runs(Sq, H):
    blocks, n = -(-Sq // 256) * H, min(_cus(), 256)
    rounds = -(-blocks // n)
    return blocks >= n and blocks * 100 < rounds * n * 97


def _inputs(seed, Sq, Sk, H, HK, kind, rot=128):
    q = oracle.synth_bf16(seed, 1, (Sq, H, 128))
    k = oracle.synth_bf16(seed, 2, (Sk, HK, 128))
    v = oracle.synth_bf16(seed, 3, (Sk, HK, 128))
    wq = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(seed, 4, (128,)))).astype(np.float32)
    wk = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(seed, 5, (128,)))).astype(np.float32)
    tabs = None
    if kind == 1:
        rng = np.random.default_rng(seed)
        ang_q = rng.uniform(-3, 3, (Sq, rot // 2)).astype(np.float32)
        ang_k = rng.uniform(-3, 3, (Sk, rot // 2)).astype(np.float32)
        tabs = ((np.cos(ang_q), np.sin(ang_q)), (np.cos(ang_k), np.sin(ang_k)))
    return q, k, v, wq, wk, tabs


def _run(q, k, v, wq, wk, kind, tabs, stream_k, reps=1):
    Sk, HK = k.shape[0], k.shape[1]
    ws = torch.empty(ops.workspace_bytes(Sk, HK, stream_k=True), dtype=torch.uint8, device="cuda")
    cfg = ops.CFG_PAIR_SK_W4 if stream_k else ops.CFG_PAIR_W4
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    kw = {}
    if kind == 1:
        (qa, qb), (ka, kb) = tabs
        kw = dict(q_table=(torch.from_numpy(qa).cuda(), torch.from_numpy(qb).cuda()),
                  k_table=(torch.from_numpy(ka).cuda(), torch.from_numpy(kb).cuda()))
    outs = []
    for _ in range(reps):
        o = ops.joint_attention(dq, dk, dv, q_norm=torch.from_numpy(wq).cuda(), k_norm=torch.from_numpy(wk).cuda(),
                                table_kind=kind, workspace=ws, config=cfg, **kw)
        torch.cuda.synchronize()
        outs.append(from_dev(o))
    return outs


@pytest.mark.parametrize("Sq,Sk,H,HK,kind", [
    (300, 300, 160, 160, 1),    # 320 blocks, 5 key tiles each, partial query block
    (300, 290, 160, 20, 0),     # GQA, ragged last key tile
    (520, 1000, 96, 96, 1),     # 288 blocks of 16 tiles
    (256, 4608, 300, 300, 0),   # long blocks: 72 tiles, a range of 84
])
def test_streamk_matches_oracle_and_whole_blocks(Sq, Sk, H, HK, kind):
    print(f"\n[stream-K] Sq={Sq} Sk={Sk} H={H} HK={HK} kind={kind}", flush=True)
    if not _streamk_runs(Sq, H):
        pytest.skip(f"{_cus()} CUs: the shape does not take the stream-K schedule on this device")
    q, k, v, wq, wk, tabs = _inputs(41, Sq, Sk, H, HK, kind)
    sk = _run(q, k, v, wq, wk, kind, tabs, stream_k=True)[0]
    whole = _run(q, k, v, wq, wk, kind, tabs, stream_k=False)[0]
    # the oracle on a sample of kv heads and their query heads (every block of those heads, cut or not)
    G = H // HK
    kvh = sorted({0, 1, HK // 3, HK // 2, HK - 1})
    heads = [g * G + i for g in kvh for i in range(G)]
    tq = tk = None
    if kind == 1:
        tq, tk = tabs
    ref = oracle.joint_attention(np.ascontiguousarray(q[:, heads]), np.ascontiguousarray(k[:, kvh]),
                                 np.ascontiguousarray(v[:, kvh]), wq=wq, wk=wk, table_kind=kind,
                                 qa=tq[0] if kind else None, qb=tq[1] if kind else None,
                                 ka=tk[0] if kind else None, kb=tk[1] if kind else None, pairing=0, rot=128, eps=1e-6,
                                 precise=True)
    assert_close(sk[:, heads], ref, what="stream-K vs oracle")
    assert_close(whole[:, heads], ref, what="whole blocks vs oracle")
    assert_close(sk, bf16_f32(whole), what="stream-K vs whole blocks (all heads)")
    assert not np.array_equal(sk, whole), "the stream-K merge rounds differently somewhere: the schedule ran"


def test_streamk_repeat_and_shape_change():
    """Flags are consumed and reset per call: the same call repeated gives identical bits, also after a call of
    another shape on the same workspace."""
    print("\n[stream-K repeat]", flush=True)
    a = _inputs(43, 300, 300, 160, 160, 0)
    b = _inputs(44, 520, 700, 96, 96, 0)
    Sk = max(300, 700)
    ws = torch.empty(ops.workspace_bytes(Sk, 160, stream_k=True), dtype=torch.uint8, device="cuda")

    def call(inp):
        q, k, v, wq, wk, _ = inp
        o = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=torch.from_numpy(wq).cuda(),
                                k_norm=torch.from_numpy(wk).cuda(), table_kind=0, workspace=ws,
                                config=ops.CFG_PAIR_SK_W4)
        torch.cuda.synchronize()
        return from_dev(o)

    a1, a2 = call(a), call(a)
    assert np.array_equal(a1, a2), "repeat"
    b1 = call(b)
    a3, b2 = call(a), call(b)
    assert np.array_equal(a1, a3), "after another shape"
    assert np.array_equal(b1, b2)


def test_streamk_overflowing_scores():
    """The overflow construction of the fused tests (scores rising ~260 along the keys in the exp2 domain) at a
    stream-K shape: head parts overflow their first tile's reference, tail parts start at higher scores; the running-
    max launch recomputes every marked block, and the result equals the running-max kernel's."""
    print("\n[stream-K overflow]", flush=True)
    Sq, Sk, H = 300, 330, 160
    u = np.zeros(128, np.float32); u[::2] = 1.0
    w_ = np.zeros(128, np.float32); w_[1::2] = 1.0
    sgn = np.where((np.arange(Sq) // 64) % 2 == 0, 1.0, -1.0).astype(np.float32)
    q = oracle.f32_to_bf16(np.broadcast_to((sgn[:, None] * u[None, :])[:, None, :], (Sq, H, 128)).copy())
    a_ = (2.0 * np.arange(Sk) / Sk - 1.0).astype(np.float32)
    kf = a_[:, None] * u[None, :] + 0.1 * w_[None, :]
    k = oracle.f32_to_bf16(np.broadcast_to(kf[:, None, :], (Sk, H, 128)).copy())
    v = oracle.synth_bf16(45, 3, (Sk, H, 128))
    wq = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    wk = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    if not _streamk_runs(Sq, H):
        pytest.skip(f"{_cus()} CUs: the shape does not take the stream-K schedule on this device")
    outs = []
    for cfg in (ops.CFG_PIPE_W8, ops.CFG_PAIR_SK_W4):
        o = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=wq, k_norm=wk, table_kind=0, config=cfg)
        torch.cuda.synchronize()
        outs.append(from_dev(o))
    assert_close(outs[1], bf16_f32(outs[0]), what="stream-K overflow vs running max")
