"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI (liblr_attn.so via ctypes).

Bar (BASELINE): bf16 output within max-abs 2e-2 and mean-abs 2e-3 of the fp64/fp32 oracle on identical seeded inputs.
Edge cases follow what the reference kernel supports (attention.cu:253-444): nkeys not a multiple of the tile, keys
past nkeys ignored, causal with p0 > 0, GQA, strided (packed qkv) rows, partial query blocks.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_f32, from_dev, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from localrouter_amd import ops  # noqa: E402

CONFIGS = [ops.CFG_PIPE_W8, ops.CFG_PIPE_W4, ops.CFG_REGSTAGE_W8, ops.CFG_PINGPONG_W8, ops.CFG_WIDE_W4, ops.CFG_PAIR_W4]
# the fused / prepared calls also run the warp-specialised kernel and the stream-K configuration (packed V^T only)
FUSED_CONFIGS = CONFIGS + [ops.CFG_WS_W8, ops.CFG_PAIR_SK_W4]


def _qkv(seed, W, nk, H, HK):
    q = oracle.synth_bf16(seed, 1, (W, H, 128))
    k = oracle.synth_bf16(seed, 2, (nk, HK, 128))
    v = oracle.synth_bf16(seed, 3, (nk, HK, 128))
    return q, k, v


def _ref(q, k, v, **kw):
    return oracle.attention(bf16_f32(q), bf16_f32(k), bf16_f32(v), precise=True, **kw)


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("W,nk,H,HK", [(1, 1, 1, 1), (37, 100, 2, 2), (300, 300, 4, 1), (513, 129, 2, 2),
                                       (64, 64, 3, 3)])
def test_attention_noncausal(cfg, W, nk, H, HK):
    print(f"\n[attention] cfg={cfg} W={W} nk={nk} H={H} HK={HK}", flush=True)
    q, k, v = _qkv(11, W, nk, H, HK)
    out = ops.attention(to_dev(q), to_dev(k), to_dev(v), config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q, k, v), what=f"cfg{cfg}")


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("W,nk,p0", [(200, 200, 0), (150, 200, 50), (70, 333, 263), (257, 300, 0)])
def test_attention_causal(cfg, W, nk, p0):
    print(f"\n[attention causal] cfg={cfg} W={W} nk={nk} p0={p0}", flush=True)
    q, k, v = _qkv(12, W, nk, 2, 2)
    out = ops.attention(to_dev(q), to_dev(k), to_dev(v), causal=True, p0=p0, config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q, k, v, causal=True, p0=p0), what=f"cfg{cfg}")


@pytest.mark.parametrize("cfg", CONFIGS)
def test_attention_rising_scores(cfg):
    """Scores that rise along the keys by ~65 in the exp2 domain force the running reference up many times (the lazy
    rescale by more than 2^8); queries with the opposite sign keep their maximum in the first tile."""
    print(f"\n[attention rising] cfg={cfg}", flush=True)
    W, nk, H = 96, 300, 2
    sign = np.where(np.arange(W) % 3 == 0, -1.0, 1.0).astype(np.float32)
    q = oracle.f32_to_bf16(np.broadcast_to((2.0 * sign)[:, None, None], (W, H, 128)).copy())
    kk = oracle.f32_to_bf16(np.broadcast_to((2.0 * np.arange(nk) / nk)[:, None, None].astype(np.float32),
                                            (nk, H, 128)).copy())
    v = oracle.synth_bf16(14, 3, (nk, H, 128))
    out = ops.attention(to_dev(q), to_dev(kk), to_dev(v), config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q, kk, v), what=f"cfg{cfg}")


@pytest.mark.parametrize("cfg", CONFIGS)
def test_attention_overflowing_scores(cfg):
    """Scores that rise along the keys by ~260 in the exp2 domain: exp2 relative to the first tile's maximum overflows
    fp32, so a kernel must raise its reference (running max) or recompute the block (the 64-query-per-wave kernel's
    second launch)."""
    print(f"\n[attention overflow] cfg={cfg}", flush=True)
    W, nk, H = 300, 300, 2
    sign = np.where(np.arange(W) % 4 == 0, -1.0, 1.0).astype(np.float32)
    q = oracle.f32_to_bf16(np.broadcast_to((4.0 * sign)[:, None, None], (W, H, 128)).copy())
    kk = oracle.f32_to_bf16(np.broadcast_to((4.0 * np.arange(nk) / nk)[:, None, None].astype(np.float32),
                                            (nk, H, 128)).copy())
    v = oracle.synth_bf16(15, 3, (nk, H, 128))
    out = ops.attention(to_dev(q), to_dev(kk), to_dev(v), config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q, kk, v), what=f"cfg{cfg}")


def test_attention_keys_past_nkeys_ignored():
    """Rows past nkeys hold NaN; the kernel must neither read them into the result nor propagate them."""
    print("\n[attention nkeys] W=100 nk=77 of 128 rows", flush=True)
    q, k, v = _qkv(13, 100, 128, 2, 2)
    k2, v2 = k.copy(), v.copy()
    k2[77:] = 0x7FC0  # bf16 NaN
    v2[77:] = 0x7FC0
    out = ops.attention(to_dev(q), to_dev(k2), to_dev(v2), nkeys=77)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q[:, :, :], k[:77], v[:77]), what="nkeys")


def test_attention_packed_qkv_strides():
    """q, k, v as views of one packed [S, 3, H, 128] buffer (row stride 3*H*128), output into a wider row buffer."""
    print("\n[attention packed] S=190 H=3", flush=True)
    S, H = 190, 3
    qkv = oracle.synth_bf16(14, 1, (S, 3, H, 128))
    d = to_dev(qkv)
    outbuf = torch.zeros((S, 2 * H * 128), dtype=torch.bfloat16, device="cuda")
    out = outbuf[:, H * 128:].view(S, H, 128)
    ops.attention(d[:, 0], d[:, 1], d[:, 2], out)
    torch.cuda.synchronize()
    ref = _ref(np.ascontiguousarray(qkv[:, 0]), np.ascontiguousarray(qkv[:, 1]), np.ascontiguousarray(qkv[:, 2]))
    assert_close(from_dev(out), ref, what="packed")
    assert not outbuf[:, : H * 128].any(), "wrote outside the output rows"


def test_attention_deterministic():
    print("\n[attention determinism] W=600 nk=700 H=4", flush=True)
    q, k, v = _qkv(15, 600, 700, 4, 2)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    a = from_dev(ops.attention(dq, dk, dv))
    b = from_dev(ops.attention(dq, dk, dv))
    assert np.array_equal(a, b)


def test_attention_rejects_bad_args():
    """Rejected arguments return hipErrorInvalidValue and launch nothing."""
    from localrouter_amd import _lib
    q, k, v = _qkv(16, 8, 8, 2, 2)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    out = torch.zeros_like(dq)
    L = _lib.load()
    s = torch.cuda.current_stream().cuda_stream
    sc = ops.SCALE_128
    assert L.lr_attention_bf16(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), 0, 8, 2, 2, 0, 0, sc, 256,
                               256, 256, s) == 1  # nkeys 0
    assert L.lr_attention_bf16(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), 0, 8, 3, 2, 8, 0, sc, 384,
                               256, 384, s) == 1  # H % HK
    assert L.lr_attention_bf16(dq.data_ptr() + 2, dk.data_ptr(), dv.data_ptr(), out.data_ptr(), 0, 8, 2, 2, 8, 0, sc,
                               256, 256, 256, s) == 1  # misaligned
    assert L.lr_attention_bf16(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), 0, 8, 2, 2, 8, 0, -1.0,
                               256, 256, 256, s) == 1  # scale
    torch.cuda.synchronize()
    assert not out.any()


# ------------------------------------------------------------------------------------------ RMSNorm + RoPE
def _tables(kind, S, rot, seed=5):
    rng = np.random.default_rng(seed)
    P = rot // 2
    ang = rng.uniform(-np.pi, np.pi, size=(S, P))
    if kind == ops.TABLE_COSSIN_F32:
        return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    m = np.stack([np.cos(ang), -np.sin(ang), np.sin(ang), np.cos(ang)], axis=-1).astype(np.float32)
    if kind == ops.TABLE_MAT2_F32:
        return m.reshape(S, 4 * P), None
    return oracle.f32_to_bf16(m).reshape(S, 4 * P), None


def _dev_table(t):
    if t is None:
        return None
    if t.dtype == np.uint16:
        return to_dev(t)
    return torch.from_numpy(t).cuda()


@pytest.mark.parametrize("kind,pairing,rot", [(1, 0, 128), (1, 1, 128), (2, 1, 96), (3, 0, 64), (0, 0, 128),
                                              (2, 0, 128), (1, 1, 32)])
@pytest.mark.parametrize("round_norm", [0, 1])
def test_rms_rope(kind, pairing, rot, round_norm):
    print(f"\n[rms_rope] kind={kind} pairing={pairing} rot={rot} round={round_norm}", flush=True)
    S, H = 77, 3
    x = oracle.synth_bf16(21, 1, (S, H, 128))
    w = (1.0 + 0.25 * oracle.bf16_to_f32(oracle.synth_bf16(21, 2, (128,)))).astype(np.float32)
    ta, tb = _tables(kind, S, rot) if kind else (None, None)
    ref = oracle.rms_rope(x, w, table_kind=kind, ta=ta, tb=tb, pairing=pairing, rot=rot, eps=1e-6)
    src = to_dev(x)
    dst = torch.empty_like(src)
    ops.rms_rope(src, dst, torch.from_numpy(w).cuda(), n=S, heads=H, src_row_stride=H * 128, dst_row_stride=H * 128,
                 table_kind=kind, table_a=_dev_table(ta), table_b=_dev_table(tb), rot=rot, pairing=pairing,
                 round_norm=bool(round_norm))
    torch.cuda.synchronize()
    got = bf16_f32(from_dev(dst))
    # two bf16 roundings at most (normalised value, output): |err| <= 2 * 2^-8 * |y| + tiny
    assert np.allclose(got, ref, rtol=1.6e-2, atol=1e-2), np.abs(got - ref).max()


def test_rms_rope_qk_h3_in_place():
    """Kitchen.rmsRope semantics: q and k of a packed qkv, in place, bf16 weights, bf16 [S,48,2,2] table, rot 96."""
    print("\n[rms_rope_qk] H3 packed in place", flush=True)
    from localrouter_amd import rope
    pos = rope.h3_positions(10, 2, 8, 10, 15)
    S, H = pos.shape[0], 4
    qkv = oracle.synth_bf16(22, 1, (S, 3, H, 128))
    qn = oracle.f32_to_bf16(1.0 + 0.1 * oracle.bf16_to_f32(oracle.synth_bf16(22, 2, (128,))))
    kn = oracle.f32_to_bf16(1.0 + 0.1 * oracle.bf16_to_f32(oracle.synth_bf16(22, 3, (128,))))
    inv = (1.0 / np.power(10000.0, np.arange(16) / 16.0)).astype(np.float32)
    tab = rope.h3_rope_table(pos, inv).reshape(S, 192)
    d = to_dev(qkv)
    ops.rms_rope_qk(d[:, 0], d[:, 1], to_dev(qn), to_dev(kn), to_dev(tab), heads=H, seq=S, rot=96, eps=1e-5)
    torch.cuda.synchronize()
    got = from_dev(d)
    for part, wn in ((0, qn), (1, kn)):
        ref = oracle.rms_rope(np.ascontiguousarray(qkv[:, part]), None, w_bf16=wn, table_kind=2, ta=tab, pairing=1,
                              rot=96, eps=1e-5)
        assert np.allclose(bf16_f32(got[:, part]), ref, rtol=1.6e-2, atol=1e-2)
    assert np.array_equal(got[:, 2], qkv[:, 2]), "V must be untouched"


# ------------------------------------------------------------------------------------------ the fused op
@pytest.mark.parametrize("cfg", FUSED_CONFIGS)
@pytest.mark.parametrize("kind,pairing,rot,causal,p0,n_pre,HK", [
    (1, 0, 128, 0, 0, 0, 2),
    (1, 1, 128, 0, 0, 0, 2),
    (2, 1, 96, 0, 0, 0, 1),
    (3, 0, 64, 1, 30, 0, 2),
    (1, 0, 128, 0, 0, 40, 2),
    (0, 0, 128, 1, 0, 0, 2),
])
def test_fused_small(cfg, kind, pairing, rot, causal, p0, n_pre, HK):
    print(f"\n[fused] cfg={cfg} kind={kind} pair={pairing} rot={rot} causal={causal} p0={p0} n_pre={n_pre}", flush=True)
    Sq, Sk, H = 160, 190, 2
    q = oracle.synth_bf16(31, 1, (Sq, H, 128))
    k = oracle.synth_bf16(31, 2, (Sk, HK, 128))
    v = oracle.synth_bf16(31, 3, (Sk, HK, 128))
    wq = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(31, 4, (128,)))).astype(np.float32)
    wk = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(31, 5, (128,)))).astype(np.float32)
    qa = qb = ka = kb = None
    if kind:
        qa, qb = _tables(kind, Sq, rot, seed=6)
        ka, kb = _tables(kind, Sk, rot, seed=7)
    ref = oracle.joint_attention(q, k, v, wq=wq, wk=wk, table_kind=kind, qa=qa, qb=qb, ka=ka, kb=kb, pairing=pairing,
                                 rot=rot, eps=1e-6, p0=p0, causal=bool(causal), n_pre=n_pre, precise=True)
    out = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=torch.from_numpy(wq).cuda(),
                              k_norm=torch.from_numpy(wk).cuda(), table_kind=kind,
                              q_table=(_dev_table(qa), _dev_table(qb)) if kind else None,
                              k_table=(_dev_table(ka), _dev_table(kb)) if kind else None, pairing=pairing, rot=rot,
                              causal=bool(causal), p0=p0, n_pre=n_pre, config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), ref, what="fused")


def test_fused_overflowing_scores():
    """Large norm weights (5.0) make the normalised scores span about +-400 in the exp2 domain. Keys turn from opposing
    u to agreeing with it along the sequence; query rows 0-63, 128-191, ... point along u (relative to the first tile's
    maximum their later P overflow fp32), the others along -u (their maximum is in the first tile). The 64-query-per-
    wave kernel must give the running-max kernel's result on both kinds of rows (both see the same bf16-rounded
    normalised operands; at these score magnitudes the oracle's unrounded operands differ by more than the bar)."""
    print("\n[fused overflow]", flush=True)
    Sq, Sk, H = 260, 330, 2
    u = np.zeros(128, np.float32); u[::2] = 1.0
    w_ = np.zeros(128, np.float32); w_[1::2] = 1.0
    sgn = np.where((np.arange(Sq) // 64) % 2 == 0, 1.0, -1.0).astype(np.float32)
    q = oracle.f32_to_bf16(np.broadcast_to((sgn[:, None] * u[None, :])[:, None, :], (Sq, H, 128)).copy())
    a_ = (2.0 * np.arange(Sk) / Sk - 1.0).astype(np.float32)
    kf = a_[:, None] * u[None, :] + 0.1 * w_[None, :]
    k = oracle.f32_to_bf16(np.broadcast_to(kf[:, None, :], (Sk, H, 128)).copy())
    v = oracle.synth_bf16(32, 3, (Sk, H, 128))
    wq = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    wk = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    outs = []
    for cfg in (ops.CFG_PIPE_W8, ops.CFG_PAIR_W4, ops.CFG_WS_W8):
        o = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=wq, k_norm=wk, table_kind=0, config=cfg)
        torch.cuda.synchronize()
        outs.append(from_dev(o))
    assert_close(outs[1], bf16_f32(outs[0]), what="fused overflow: pair vs running max")
    assert_close(outs[2], bf16_f32(outs[0]), what="fused overflow: warp-specialised vs running max")


# ------------------------------------------------------------------------------------------ the two stages
@pytest.mark.parametrize("Sk,HK,n_pre", [(190, 2, 0), (64, 1, 0), (1, 1, 0), (200, 3, 50)])
def test_kv_prepare_layout_and_prepared_equals_fused(Sk, HK, n_pre):
    """lr_joint_kv_prepare writes the normalised keys [HK][Sk][128] and V^T tiles [HK][ceil(Sk/64)][128][64] (zero past
    Sk, exact copies of V otherwise); lr_joint_attention_prepared over that workspace equals the fused call bit for bit."""
    print(f"\n[kv-prepare] Sk={Sk} HK={HK} n_pre={n_pre}", flush=True)
    Sq, H = 130, 2 * HK
    q = oracle.synth_bf16(41, 1, (Sq, H, 128))
    k = oracle.synth_bf16(41, 2, (Sk, HK, 128))
    v = oracle.synth_bf16(41, 3, (Sk, HK, 128))
    qa, qb = _tables(1, Sq, 128, seed=8)
    ka, kb = _tables(1, Sk, 128, seed=9)
    need = ops.workspace_bytes(Sk, HK)
    ws = torch.full((need,), 0xAB, dtype=torch.uint8, device="cuda")   # stale bytes: all must be overwritten
    ops.joint_kv_prepare(to_dev(k), to_dev(v), ws, k_table=(_dev_table(ka), _dev_table(kb)), n_pre=n_pre)
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    kbytes = (Sk * HK * 256 + 255) // 256 * 256
    nt = (Sk + 63) // 64
    keys = raw[:Sk * HK * 256].view(np.uint16).reshape(HK, Sk, 128)
    vt = raw[kbytes:kbytes + HK * nt * 128 * 64 * 2].view(np.uint16).reshape(HK, nt, 128, 64)
    vpad = np.zeros((nt * 64, HK, 128), np.uint16)
    vpad[:Sk] = v
    expect_vt = vpad.reshape(nt, 64, HK, 128).transpose(2, 0, 3, 1)
    assert np.array_equal(vt, expect_vt), "V^T tiles"
    kref = oracle.rms_rope(k[n_pre:], None, table_kind=oracle.TABLE_COSSIN_F32, ta=ka[:Sk - n_pre], tb=kb[:Sk - n_pre],
                           eps=1e-6) if Sk > n_pre else np.zeros((0, HK, 128), np.float32)
    assert np.array_equal(keys[:, :n_pre].transpose(1, 0, 2), k[:n_pre]), "prefix keys copied"
    if Sk > n_pre:
        assert np.allclose(bf16_f32(keys[:, n_pre:].transpose(1, 0, 2)), kref, rtol=1e-2, atol=1e-2)
    tq = (_dev_table(qa), _dev_table(qb))
    outs = []
    for cfg in (ops.CFG_AUTO, ops.CFG_PIPE_W4, ops.CFG_PAIR_W4, ops.CFG_WS_W8):
        o = ops.joint_attention_prepared(to_dev(q), ws, Sk, HK, q_table=tq, config=cfg)
        f = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_table=tq, k_table=(_dev_table(ka), _dev_table(kb)),
                                n_pre=n_pre, config=cfg)
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(o), from_dev(f)), f"prepared != fused (config {cfg})"
        outs.append(from_dev(o))
    ref = oracle.joint_attention(q, k, v, table_kind=1, qa=qa, qb=qb, ka=ka, kb=kb, eps=1e-6, n_pre=n_pre,
                                 precise=True)
    for o in outs:
        assert_close(o, ref, what="prepared")


def test_prepared_rejects_row_v_configs():
    """Configurations that read V rows cannot run on a prepared workspace (it holds V^T tiles only)."""
    Sk, HK = 64, 1
    ws = torch.zeros(ops.workspace_bytes(Sk, HK), dtype=torch.uint8, device="cuda")
    q = to_dev(oracle.synth_bf16(42, 1, (32, 1, 128)))
    for cfg in (ops.CFG_REGSTAGE_W8, ops.CFG_PINGPONG_W8, ops.CFG_WIDE_W4):
        with pytest.raises(Exception):
            ops.joint_attention_prepared(q, ws, Sk, HK, table_kind=ops.TABLE_NONE, config=cfg)
