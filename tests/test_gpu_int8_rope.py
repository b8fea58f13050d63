"""Kitchen.rmsRope fused into the INT8 prep (lr_int8_attention_prep_rope), on the GPU against the CPU oracle, through
the C ABI.

The H3 chain is rmsRope -> attentionPrep -> attentionKernel (src/engines/minimax_h3/dit.zig:665-671); the fused prep
normalises and rotates q and k in registers while it quantises them. Checked:
  * bit-exact against the oracle chain: oracle.rms_rope(round_norm=True) (bf16 weights, the bf16 [S, 48, 2, 2] table,
    split-half pairs, rot 96) rounded to bf16, then the oracle's anchor and quantisers -- anchor row, int8 Q / K / V,
    every scale, the column sums;
  * bit-exact against the unfused GPU chain (lr_rms_rope_qk_bf16 in place, then lr_int8_attention_prep): the whole
    workspace;
  * the packed qkv is not modified; the attention over the fused workspace equals the one over the unfused workspace;
  * the standalone lr_rms_rope_qk_bf16 itself is bit-exact against the oracle's rounding mode.
Cases: both sides of the H4 / H128 switch (256 keys) and of the 64 / 128 key tile switch (1024), a biased K that
makes the anchor fire (so the anchor row itself is normalised and rotated), the table of H3's own layout
(rope.h3_positions / h3_rope_table), and H3's shape (5,967 tokens x 56 heads, sampled heads)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import bf16_f32, from_dev, to_dev
from tests.test_gpu_int8 import _check_parts, _decode, _oracle_head, _qkv

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from localrouter_amd import ops, rope  # noqa: E402

ROT, EPS = 96, 1e-5   # H3's rmsRope arguments (src/engines/minimax_h3/dit.zig:40, :665)


def _table(S, seed):
    """A bf16 [S, 48, 2, 2] table from H3's own layout arithmetic (positions of a text + video layout, the 16
    frequencies of each axis); rows past the layout's length repeat it."""
    pos = rope.h3_positions(24, 3, 8, 12, 15)
    inv = (1.0 / np.power(10000.0, np.arange(16) / 16.0)).astype(np.float32)
    tab = rope.h3_rope_table(pos, inv).reshape(-1, 192)
    reps = -(-S // tab.shape[0])
    tab = np.tile(tab, (reps, 1))[:S]
    rng = np.random.default_rng(seed)
    return np.ascontiguousarray(np.roll(tab, int(rng.integers(tab.shape[0])), axis=0))


def _weights(seed):
    qn = oracle.f32_to_bf16(1.0 + 0.1 * oracle.bf16_to_f32(oracle.synth_bf16(seed, 7, (128,))))
    kn = oracle.f32_to_bf16(1.0 + 0.1 * oracle.bf16_to_f32(oracle.synth_bf16(seed, 8, (128,))))
    return qn, kn


def _oracle_rope(x, w, tab):
    """The oracle's rmsRope of one head's rows [S, 128] (bf16 bits), rounded to bf16 as the reference stores them."""
    y = oracle.rms_rope(np.ascontiguousarray(x)[:, None, :], None, w_bf16=w, table_kind=oracle.TABLE_MAT2_BF16,
                        ta=tab, pairing=oracle.PAIR_SPLIT_HALF, rot=ROT, eps=EPS, round_norm=True)
    return oracle.f32_to_bf16(y[:, 0, :])


@pytest.mark.parametrize("S,H,bias,heads", [(80, 2, (), None), (256, 2, (1,), None), (300, 3, (0, 2), None),
                                             (1100, 2, (1,), None), (5967, 56, (3,), (0, 3, 55))])
def test_prep_rope_bit_exact(S, H, bias, heads):
    print(f"\n[int8 prep_rope] S={S} H={H} bias={bias}", flush=True)
    qkv = _qkv(40 + S, S, H, bias)
    qn, kn = _weights(S)
    tab = _table(S, S)
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    before = from_dev(dq)
    dqn, dkn, dtab = to_dev(qn), to_dev(kn), to_dev(tab)
    # both workspaces start equal (the prep leaves alignment padding and unused aux bytes as they were)
    ws_f = torch.zeros(ops.int8_workspace_bytes(H, S), dtype=torch.uint8, device="cuda")
    ws_u = torch.zeros_like(ws_f)
    ops.kitchen_attention_prep_rope(dq, ws_f, H, dtab, dqn, dkn, rot=ROT, eps=EPS)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(dq), before), "the fused prep must not modify qkv"
    # the unfused GPU chain: rmsRope in place on a copy, then the prep
    du = dq.clone()
    v3 = du.view(S, 3, H, 128)
    ops.rms_rope_qk(v3[:, 0], v3[:, 1], dqn, dkn, dtab, heads=H, seq=S, rot=ROT, eps=EPS)
    ops.kitchen_attention_prep(du, ws_u, H)
    torch.cuda.synchronize()
    assert torch.equal(ws_f, ws_u), "fused prep != rmsRope + prep (workspace bits)"
    # the oracle chain, head by head
    dec = _decode(ws_f.cpu().numpy(), 1, H, H, S, S)
    roped = from_dev(du).reshape(S, 3, H, 128)
    for h in (range(H) if heads is None else heads):
        qh = _oracle_rope(qkv[:, 0, h], qn, tab)
        kh = _oracle_rope(qkv[:, 1, h], kn, tab)
        assert np.array_equal(roped[:, 0, h], qh) and np.array_equal(roped[:, 1, h], kh), \
            f"head {h}: lr_rms_rope_qk_bf16 != oracle rmsRope (bits)"
        ref = _oracle_head(qh, kh, qkv[:, 2, h], S)
        _check_parts(dec, ref, 0, h, h, S, f"S={S} head {h}")
    # the attention over either workspace: the same bits
    out_f = torch.empty((S, H * 128), dtype=torch.bfloat16, device="cuda")
    out_u = torch.empty_like(out_f)
    ops.kitchen_attention_kernel(out_f, ws_f, H, S, True)
    ops.kitchen_attention_kernel(out_u, ws_u, H, S, True)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_u)
    assert torch.isfinite(out_f.float()).all()


def test_prep_rope_zero_rows_and_partial_rotation():
    """Degenerate rows (all-zero q and k rows: the norm is 0 / sqrt(eps), finite) and a rotation over the first 32 dims
    only: still bit-exact against the oracle chain."""
    S, H, rot = 130, 2, 32
    qkv = _qkv(77, S, H)
    qkv[5, 0, 1] = 0
    qkv[9, 1, 0] = 0
    qn, kn = _weights(77)
    tab = _table(S, 5)[:, :2 * rot].copy()
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    ws = ops.kitchen_attention_prep_rope(dq, None, H, to_dev(tab), to_dev(qn), to_dev(kn), rot=rot, eps=EPS)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S)
    for h in range(H):
        qh, kh = (oracle.f32_to_bf16(oracle.rms_rope(np.ascontiguousarray(qkv[:, i, h])[:, None, :], None, w_bf16=w,
                                                     table_kind=oracle.TABLE_MAT2_BF16, ta=tab,
                                                     pairing=oracle.PAIR_SPLIT_HALF, rot=rot, eps=EPS,
                                                     round_norm=True)[:, 0, :])
                  for i, w in ((0, qn), (1, kn)))
        assert np.isfinite(bf16_f32(qh)).all()
        _check_parts(dec, _oracle_head(qh, kh, qkv[:, 2, h], S), 0, h, h, S, f"rot {rot} head {h}")


def test_prep_rope_gqa_batches():
    """Separate q [B, H, S, 128] and k, v [B, HK, S, 128] tensors: two batches, GQA 4 / 2 (query head h reads kv head
    h // 2); token n of every batch and head uses table row n. Bit-exact against the oracle chain per (batch, head)."""
    B, H, HK, S = 2, 4, 2, 200
    print(f"\n[int8 prep_rope gqa] B={B} H={H} HK={HK} S={S}", flush=True)
    q = oracle.synth_bf16(91, 1, (B, H, S, 128))
    k = oracle.synth_bf16(91, 2, (B, HK, S, 128))
    v = oracle.synth_bf16(91, 3, (B, HK, S, 128))
    qn, kn = _weights(91)
    tab = _table(S, 9)
    ws = ops.int8_attention_prep_rope(to_dev(q), to_dev(k), to_dev(v), to_dev(qn), to_dev(kn), to_dev(tab), rot=ROT,
                                      eps=EPS)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), B, H, HK, S, S)
    for b in range(B):
        kr = [_oracle_rope(k[b, hk], kn, tab) for hk in range(HK)]
        for h in range(H):
            hk = h // (H // HK)
            ref = _oracle_head(_oracle_rope(q[b, h], qn, tab), kr[hk], v[b, hk], S)
            _check_parts(dec, ref, b, h, hk, S, f"b={b} h={h}")


def test_prep_rope_rejects():
    """Head dim 64, Sq != Sk, a misaligned table row stride, rot not a multiple of 16: rejected before any launch."""
    from localrouter_amd import _lib
    L = _lib.load()
    S, H = 64, 1
    qkv = torch.zeros((S, 3 * H * 128), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(ops.int8_workspace_bytes(H, S), dtype=torch.uint8, device="cuda")
    w = torch.ones(128, dtype=torch.bfloat16, device="cuda")
    tab = torch.zeros((S, 256), dtype=torch.bfloat16, device="cuda")
    q, k, v = (qkv.data_ptr() + i * 256 for i in range(3))
    st = (S * 384, 128, 384)

    def call(D=128, Sq=S, Sk=S, rs=256, rot=96):
        return L.lr_int8_attention_prep_rope(q, k, v, ws.data_ptr(), 1, H, H, Sq, Sk, D, *st, *st, *st, w.data_ptr(),
                                             w.data_ptr(), tab.data_ptr(), rs, rot, EPS, None)
    assert call(D=64) == 1 and call(Sq=32) == 1 and call(rs=252) == 1 and call(rot=40) == 1 and call(rs=150) == 1
    assert call() == 0
    torch.cuda.synchronize()
