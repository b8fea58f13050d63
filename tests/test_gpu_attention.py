"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI (liblr_attn.so via ctypes).

Bar: bf16 output within max-abs 2e-2, mean-abs 2e-3 and relative L2 3e-3 of the fp64/fp32 oracle on identical seeded
inputs (tests/_util.py); RMSNorm + RoPE within 1 bf16 ulp of the oracle in the same rounding mode.
Edge cases follow what the reference kernel supports (attention.cu:253-444): nkeys not a multiple of the tile, keys
past nkeys ignored, causal with p0 > 0, GQA, strided (packed qkv) rows, partial query blocks.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import assert_close, bf16_f32, bf16_ulps, decode_images, from_dev, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from localrouter_amd import ops  # noqa: E402

# attention over key and value rows (lr_attention_bf16_ex): the pipelined kernel's two tile shapes and the streaming
# kernel reading key rows; the fused and prepared calls run the streaming kernel over key tile images
CONFIGS = [ops.CFG_PIPE_W8, ops.CFG_PIPE_W4, ops.CFG_STREAM_W8]
FUSED_CONFIGS = [ops.CFG_AUTO, ops.CFG_STREAM_W8]


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


@pytest.mark.parametrize("p0", [0, 77])
def test_attention_causal_gqa_32_8(p0):
    """Causal attention with 32 query heads over 8 kv heads (groups of 4), p0 = 0 and a shifted diagonal."""
    print(f"\n[attention causal gqa] H=32 HK=8 p0={p0}", flush=True)
    W, nk = 300, 300 + p0
    q, k, v = _qkv(17, W, nk, 32, 8)
    out = ops.attention(to_dev(q), to_dev(k), to_dev(v), causal=True, p0=p0)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q, k, v, causal=True, p0=p0), what="causal gqa 32/8")


def test_attention_head_dim_72_zero_padded():
    """Heads of 72 dims zero-padded to 128 with scale 1/sqrt(72) (a model whose head dim is not 128 running on the
    128-dim kernels): equal to 72-dim attention, and the padded output dims exactly zero."""
    print("\n[attention hd72] W=250 nk=333 H=3", flush=True)
    W, nk, H = 250, 333, 3
    q, k, v = _qkv(18, W, nk, H, H)
    for t in (q, k, v):
        t[..., 72:] = 0
    scale = float(np.float32(1.0 / np.sqrt(72.0)))
    out = from_dev(ops.attention(to_dev(q), to_dev(k), to_dev(v), scale=scale))
    torch.cuda.synchronize()
    ref = oracle.brute_attention(bf16_f32(q), bf16_f32(k), bf16_f32(v), scale=scale)   # zero dims add nothing
    assert_close(out, ref, what="hd72")
    assert not out[..., 72:].any(), "padded dims must stay zero"


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
    fp32, so the kernel must raise its running reference."""
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


@pytest.mark.parametrize("cfg", CONFIGS)
def test_attention_keys_past_nkeys_ignored(cfg):
    """Rows past nkeys hold NaN; the kernel must neither read them into the result nor propagate them."""
    print(f"\n[attention nkeys] cfg={cfg} W=100 nk=77 of 128 rows", flush=True)
    q, k, v = _qkv(13, 100, 128, 2, 2)
    k2, v2 = k.copy(), v.copy()
    k2[77:] = 0x7FC0  # bf16 NaN
    v2[77:] = 0x7FC0
    out = ops.attention(to_dev(q), to_dev(k2), to_dev(v2), nkeys=77, config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q[:, :, :], k[:77], v[:77]), what="nkeys")


@pytest.mark.parametrize("cfg", CONFIGS)
def test_attention_packed_qkv_strides(cfg):
    """q, k, v as views of one packed [S, 3, H, 128] buffer (row stride 3*H*128), output into a wider row buffer."""
    print(f"\n[attention packed] cfg={cfg} S=190 H=3", flush=True)
    S, H = 190, 3
    qkv = oracle.synth_bf16(14, 1, (S, 3, H, 128))
    d = to_dev(qkv)
    outbuf = torch.zeros((S, 2 * H * 128), dtype=torch.bfloat16, device="cuda")
    out = outbuf[:, H * 128:].view(S, H, 128)
    ops.attention(d[:, 0], d[:, 1], d[:, 2], out, config=cfg)
    torch.cuda.synchronize()
    ref = _ref(np.ascontiguousarray(qkv[:, 0]), np.ascontiguousarray(qkv[:, 1]), np.ascontiguousarray(qkv[:, 2]))
    assert_close(from_dev(out), ref, what="packed")
    assert not outbuf[:, : H * 128].any(), "wrote outside the output rows"


@pytest.mark.parametrize("cfg", CONFIGS)
def test_attention_head_major_kv(cfg):
    """k and v head-major ([HK][nkeys][128]: kv-head stride nkeys*128, row stride 128) through lr_attention_bf16_ex,
    GQA 4 / 2, causal with p0 and a ragged last key tile."""
    from localrouter_amd import _lib
    W, nk, H, HK, p0 = 200, 333, 4, 2, 133
    print(f"\n[attention head-major] cfg={cfg} W={W} nk={nk} H={H} HK={HK}", flush=True)
    q, k, v = _qkv(19, W, nk, H, HK)
    dq = to_dev(q)
    dk = to_dev(np.ascontiguousarray(k.transpose(1, 0, 2)))
    dv = to_dev(np.ascontiguousarray(v.transpose(1, 0, 2)))
    out = torch.zeros_like(dq)
    _lib.call("lr_attention_bf16_ex", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), out.data_ptr(), p0, W, H, HK, nk, 1,
              ops.SCALE_128, H * 128, 128, 128, H * 128, nk * 128, nk * 128, cfg,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _ref(q, k, v, causal=True, p0=p0), what=f"head-major cfg{cfg}")


@pytest.mark.parametrize("W,nk,H,HK,causal,p0", [(300, 4100, 17, 17, 0, 0), (513, 4097, 12, 6, 0, 0),
                                                 (700, 999, 3, 1, 1, 299), (64, 4160, 33, 33, 0, 0)])
def test_stream_rows_equal_images(W, nk, H, HK, causal, p0):
    """The streaming kernel over key rows gathers each key tile into the layout of a tile image; over images of the same
    keys (lr_joint_kv_prepare with every key a prefix key: copied unchanged) and the same queries
    (lr_joint_attention_images, which cuts the last partial round of blocks over the workgroups when that pays) the
    output must be the same bits. Non-causal: lr_attention_bf16_ws, which takes the streaming kernel from 4,096 keys and
    33 query blocks on (the same split tail, its partials and counters in the caller's workspace); causal (never
    split): lr_attention_bf16_ex with LR_ATTN_CFG_STREAM_W8."""
    print(f"\n[stream rows = images] W={W} nk={nk} H={H} HK={HK} causal={causal}", flush=True)
    q, k, v = _qkv(20, W, nk, H, HK)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    ws = torch.empty(ops.workspace_bytes(nk, HK), dtype=torch.uint8, device="cuda")
    ops.joint_kv_prepare(dk, dv, ws, table_kind=ops.TABLE_NONE, n_pre=nk)
    img = ops.joint_attention_images(dq, ws, nk, HK, causal=bool(causal), p0=p0)
    if causal:
        rows = ops.attention(dq, dk, dv, causal=True, p0=p0, config=ops.CFG_STREAM_W8)
    else:
        # a workspace of stale bytes: the call clears the counters it needs
        assert ops.attention_ws_bytes(W, H, nk, False) == 69207040   # the streaming kernel's split area
        wsr = torch.full((ops.attention_ws_bytes(W, H, nk, False),), 0x5A, dtype=torch.uint8, device="cuda")
        rows = ops.attention_ws(dq, dk, dv, workspace=wsr)
    torch.cuda.synchronize()
    assert torch.equal(rows, img)
    assert_close(from_dev(rows), _ref(q, k, v, causal=bool(causal), p0=p0), what="stream rows")


@pytest.mark.parametrize("W,nk,H,HK", [(6400, 4100, 12, 12), (6400, 4100, 12, 4), (4608, 4096, 24, 24)])
def test_stream_rows_unsplit_last_pass(W, nk, H, HK):
    """The streaming kernel over key rows without a workspace runs whole 256-query blocks, L, L + 256, ... per
    workgroup, and shares the last partial pass (300 blocks on 256 CUs: 44, five or six per XCD; 432 blocks: 176)
    between the XCDs. Every block must be computed once: the whole output against the pipelined kernel's (an
    independent schedule, to within the parity bar), and the first and last row of every query block of every head
    against the oracle."""
    print(f"\n[stream rows, unsplit last pass] W={W} nk={nk} H={H} HK={HK}", flush=True)
    q, k, v = _qkv(23, W, nk, H, HK)
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    st = ops.attention(dq, dk, dv, config=ops.CFG_STREAM_W8)
    w8 = ops.attention(dq, dk, dv, config=ops.CFG_PIPE_W8)
    torch.cuda.synchronize()
    got = from_dev(st)
    # two bf16 outputs, each rounded once from its own fp32 result: twice the relative-L2 bar (a block left uncomputed
    # or computed from the wrong rows is off by the output's own magnitude)
    assert_close(got, bf16_f32(from_dev(w8)).astype(np.float64), rel=6e-3, what="stream unsplit vs pipelined W8")
    rows = np.unique(np.concatenate([np.arange(0, W, 256), np.minimum(np.arange(255, W + 255, 256), W - 1)]))
    ref = oracle.attention(bf16_f32(q), bf16_f32(k), bf16_f32(v), precise=False, rows=rows)
    assert_close(got[rows], ref, what="stream unsplit vs oracle")


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
    """Within 1 bf16 ulp of the oracle in the same rounding mode (round_norm: the normalised value rounded to bf16
    before the rotation, rms_rope.cu:143-150); the oracle of the other mode is further off on some element."""
    print(f"\n[rms_rope] kind={kind} pairing={pairing} rot={rot} round={round_norm}", flush=True)
    S, H = 77, 3
    x = oracle.synth_bf16(21, 1, (S, H, 128))
    w = (1.0 + 0.25 * oracle.bf16_to_f32(oracle.synth_bf16(21, 2, (128,)))).astype(np.float32)
    ta, tb = _tables(kind, S, rot) if kind else (None, None)
    ref = oracle.rms_rope(x, w, table_kind=kind, ta=ta, tb=tb, pairing=pairing, rot=rot, eps=1e-6,
                          round_norm=bool(round_norm))
    src = to_dev(x)
    dst = torch.empty_like(src)
    ops.rms_rope(src, dst, torch.from_numpy(w).cuda(), n=S, heads=H, src_row_stride=H * 128, dst_row_stride=H * 128,
                 table_kind=kind, table_a=_dev_table(ta), table_b=_dev_table(tb), rot=rot, pairing=pairing,
                 round_norm=bool(round_norm))
    torch.cuda.synchronize()
    got = from_dev(dst)
    u = bf16_ulps(got, ref)
    assert u.max() <= 1.0, f"{u.max():.2f} ulp"
    if kind and round_norm:
        other = oracle.rms_rope(x, w, table_kind=kind, ta=ta, tb=tb, pairing=pairing, rot=rot, eps=1e-6)
        assert bf16_ulps(got, other).max() > 1.0, "the test cannot tell the two rounding modes apart"


def test_rms_rope_qk_h3_in_place():
    """Kitchen.rmsRope semantics: q and k of a packed qkv, in place, bf16 weights, bf16 [S,48,2,2] table, rot 96, the
    normalised value rounded to bf16 before the rotation: the oracle's rounding mode bit for bit (the norm in double,
    the rotation's products exact), and farther from the other mode."""
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
                              rot=96, eps=1e-5, round_norm=True)
        u = bf16_ulps(np.ascontiguousarray(got[:, part]), ref)
        assert u.max() <= 1.0, f"part {part}: {u.max():.2f} ulp"
        assert np.array_equal(got[:, part], oracle.f32_to_bf16(ref)), f"part {part}: not the oracle's bits"
    assert np.array_equal(got[:, 2], qkv[:, 2]), "V must be untouched"


# ------------------------------------------------------------------------------------------ the fused op
def _fused_case(seed, Sq, Sk, H, HK, kind, pairing, rot):
    q = oracle.synth_bf16(seed, 1, (Sq, H, 128))
    k = oracle.synth_bf16(seed, 2, (Sk, HK, 128))
    v = oracle.synth_bf16(seed, 3, (Sk, HK, 128))
    wq = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(seed, 4, (128,)))).astype(np.float32)
    wk = (1.0 + 0.2 * oracle.bf16_to_f32(oracle.synth_bf16(seed, 5, (128,)))).astype(np.float32)
    qa = qb = ka = kb = None
    if kind:
        qa, qb = _tables(kind, Sq, rot, seed=6)
        ka, kb = _tables(kind, Sk, rot, seed=7)
    return q, k, v, wq, wk, qa, qb, ka, kb


@pytest.mark.parametrize("cfg", FUSED_CONFIGS)
@pytest.mark.parametrize("Sq,Sk,H,kind,pairing,rot,causal,p0,n_pre,HK", [
    (160, 190, 2, 1, 0, 128, 0, 0, 0, 2),
    (160, 190, 2, 1, 1, 128, 0, 0, 0, 2),
    (160, 190, 2, 2, 1, 96, 0, 0, 0, 1),
    (160, 190, 2, 3, 0, 64, 1, 30, 0, 2),
    (160, 190, 2, 1, 0, 128, 0, 0, 40, 2),
    (160, 190, 2, 0, 0, 128, 1, 0, 0, 2),
    (1, 1, 1, 1, 0, 128, 0, 0, 0, 1),           # one query, one key
    (600, 64, 4, 1, 0, 128, 0, 0, 0, 1),        # one key tile, GQA 4:1, three query blocks (the last partial)
    (300, 700, 8, 2, 1, 96, 1, 400, 0, 2),      # causal, p0 > 0, GQA 4:1, many key tiles
    (257, 65, 2, 1, 0, 128, 0, 0, 65, 2),       # every key a prefix key (n_pre = Sk)
])
def test_fused_small(cfg, Sq, Sk, H, kind, pairing, rot, causal, p0, n_pre, HK):
    """Against the fp64 oracle of the reference's chain (prepared q and k stored as bf16, then attention)."""
    print(f"\n[fused] cfg={cfg} Sq={Sq} Sk={Sk} H={H} HK={HK} kind={kind} pair={pairing} rot={rot} causal={causal} "
          f"p0={p0} n_pre={n_pre}", flush=True)
    q, k, v, wq, wk, qa, qb, ka, kb = _fused_case(31, Sq, Sk, H, HK, kind, pairing, rot)
    ref = oracle.joint_attention(q, k, v, wq=wq, wk=wk, table_kind=kind, qa=qa, qb=qb, ka=ka, kb=kb, pairing=pairing,
                                 rot=rot, eps=1e-6, p0=p0, causal=bool(causal), n_pre=n_pre, precise=True,
                                 round_prepared=True)
    out = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=torch.from_numpy(wq).cuda(),
                              k_norm=torch.from_numpy(wk).cuda(), table_kind=kind,
                              q_table=(_dev_table(qa), _dev_table(qb)) if kind else None,
                              k_table=(_dev_table(ka), _dev_table(kb)) if kind else None, pairing=pairing, rot=rot,
                              causal=bool(causal), p0=p0, n_pre=n_pre, config=cfg)
    torch.cuda.synchronize()
    assert_close(from_dev(out), ref, what="fused")


def test_fused_in_place():
    """q_raw may be the output buffer itself: the result equals the out-of-place call bit for bit."""
    print("\n[fused in place] Sq=300 Sk=200 H=4 HK=2", flush=True)
    q, k, v, wq, wk, qa, qb, ka, kb = _fused_case(33, 300, 200, 4, 2, 1, 0, 128)
    kw = dict(q_norm=torch.from_numpy(wq).cuda(), k_norm=torch.from_numpy(wk).cuda(), table_kind=1,
              q_table=(_dev_table(qa), _dev_table(qb)), k_table=(_dev_table(ka), _dev_table(kb)))
    dq = to_dev(q)
    ref = from_dev(ops.joint_attention(dq, to_dev(k), to_dev(v), **kw))
    ops.joint_attention(dq, to_dev(k), to_dev(v), dq, **kw)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(dq), ref)


def _sign_ramp(Sq, Sk, H):
    """Inputs whose prepared operands the kernels produce exactly (eps 0, every |x| 1: the norm is 1 exactly): q rows
    +-1 (blocks of 64 rows alternating sign), key j +1 on its first m_j dims and -1 on the rest, m_j rising 0..128."""
    sgn = np.where((np.arange(Sq) // 64) % 2 == 0, 1.0, -1.0).astype(np.float32)
    q = oracle.f32_to_bf16(np.broadcast_to(sgn[:, None, None], (Sq, H, 128)).copy())
    m = np.rint(128.0 * np.arange(Sk) / max(Sk - 1, 1)).astype(np.int64)
    kf = np.where(np.arange(128)[None, :] < m[:, None], 1.0, -1.0).astype(np.float32)
    k = oracle.f32_to_bf16(np.broadcast_to(kf[:, None, :], (Sk, H, 128)).copy())
    return q, k


def _sign_ramp_expected(q, k, v, wn, scale):
    """The kernels' prepared operands, restated: with |x| = 1 everywhere and eps 0 the norm is 1, so queries and keys
    become bf16(x * w) = x * w exactly for w = 5; then the fp64 oracle over them."""
    assert bf16_f32(oracle.f32_to_bf16(np.array([wn], np.float32)))[0] == wn, "w must be a bf16 value"
    return oracle.attention(bf16_f32(q) * wn, bf16_f32(k) * wn, bf16_f32(v), scale=scale, precise=True)


def test_fused_overflowing_scores():
    """Norm weights 5.0 make the exp2-domain scores span about +-400: relative to a block's first-tile maximum the
    later P of the +u query rows overflow fp32 (the kernel's exact recomputation of those rows), the -u rows keep
    their maximum in the first tile. Checked against the fp64 oracle on the prepared operands (exact here)."""
    print("\n[fused overflow] Sq=260 Sk=330 H=2", flush=True)
    Sq, Sk, H = 260, 330, 2
    q, k = _sign_ramp(Sq, Sk, H)
    v = oracle.synth_bf16(32, 3, (Sk, H, 128))
    w5 = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    out = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=w5, k_norm=w5, table_kind=0, eps=0.0)
    torch.cuda.synchronize()
    assert_close(from_dev(out), _sign_ramp_expected(q, k, v, 5.0, ops.SCALE_128), what="fused overflow")


def test_fused_overflow_in_every_block_of_a_workgroup():
    """More overflowing blocks per persistent workgroup than its list of blocks to recompute holds (16 blocks of
    256 rows per CU, half the waves of each overflowing): the kernel must recompute all of them."""
    print("\n[fused overflow, many blocks] Sq=131072 Sk=128 H=8", flush=True)
    H = 8
    Sq = 16 * 256 * (256 // H)      # 4096 blocks of 256 rows: 16 per workgroup on a 256-CU device
    Sk = 128
    q1, k = _sign_ramp(128, Sk, H)  # rows 0-63 +u, 64-127 -u; the pattern repeats every 128 rows
    v = oracle.synth_bf16(34, 3, (Sk, H, 128))
    dq = to_dev(q1).repeat(Sq // 128, 1, 1)
    w5 = torch.full((128,), 5.0, dtype=torch.float32, device="cuda")
    out = ops.joint_attention(dq, to_dev(k), to_dev(v), q_norm=w5, k_norm=w5, table_kind=0, eps=0.0)
    torch.cuda.synchronize()
    exp = _sign_ramp_expected(q1, k, v, 5.0, ops.SCALE_128)          # [128, H, 128]: every 128-row period
    got = from_dev(out).reshape(Sq // 128, 128, H, 128)
    for i in (0, 1, 2, Sq // 256, Sq // 128 - 1):
        assert_close(got[i], exp, what=f"period {i}")
    assert (got == got[0:1]).all(), "every 128-row period must give the same bits"


# ------------------------------------------------------------------------------------------ the two stages
@pytest.mark.parametrize("Sk,HK,n_pre", [(190, 2, 0), (64, 1, 0), (1, 1, 0), (200, 3, 50)])
def test_kv_prepare_layout_and_prepared_equals_fused(Sk, HK, n_pre):
    """lr_joint_kv_prepare writes the normalised keys as tile images and the values as rows into the workspace (zero
    past Sk, exact copies of V and of the prefix keys); lr_joint_attention_prepared over that workspace equals the
    fused call (which reads the caller's value rows) bit for bit."""
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
    keys, vals = decode_images(ws.cpu().numpy(), Sk, HK)
    assert np.array_equal(vals[:, :Sk], v.transpose(1, 0, 2)), "value rows"
    assert not vals[:, Sk:].any() and not keys[:, Sk:].any(), "rows past Sk must be zero"
    assert np.array_equal(keys[:, :n_pre], k[:n_pre].transpose(1, 0, 2)), "prefix keys copied"
    if Sk > n_pre:
        kref = oracle.rms_rope(k[n_pre:], None, table_kind=oracle.TABLE_COSSIN_F32, ta=ka[:Sk - n_pre],
                               tb=kb[:Sk - n_pre], eps=1e-6)
        u = bf16_ulps(np.ascontiguousarray(keys[:, n_pre:Sk].transpose(1, 0, 2)), kref)
        assert u.max() <= 1.0, f"prepared keys {u.max():.2f} ulp from the oracle"
    tq = (_dev_table(qa), _dev_table(qb))
    o = ops.joint_attention_prepared(to_dev(q), ws, Sk, HK, q_table=tq)
    o2 = ops.joint_attention_prepared(to_dev(q), ws, Sk, HK, q_table=tq)      # the workspace is only read
    f = ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_table=tq, k_table=(_dev_table(ka), _dev_table(kb)),
                            n_pre=n_pre)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(o), from_dev(f)), "prepared != fused"
    assert np.array_equal(from_dev(o), from_dev(o2)), "second prepared call differs"
    ref = oracle.joint_attention(q, k, v, table_kind=1, qa=qa, qb=qb, ka=ka, kb=kb, eps=1e-6, n_pre=n_pre,
                                 precise=True, round_prepared=True)
    assert_close(from_dev(o), ref, what="prepared")


@pytest.mark.parametrize("causal,p0", [(0, 0), (1, 90)])
def test_three_launches_equal_fused(causal, p0):
    """lr_joint_kv_prepare + lr_joint_q_prepare + lr_joint_attention_images (queries prepared apart from out, and in
    place into out) give the fused call's bits."""
    print(f"\n[three launches] causal={causal} p0={p0}", flush=True)
    Sq, Sk, H, HK = 300, 333, 4, 2
    q, k, v, wq, wk, qa, qb, ka, kb = _fused_case(35, Sq, Sk, H, HK, 1, 1, 128)
    tq, tk = (_dev_table(qa), _dev_table(qb)), (_dev_table(ka), _dev_table(kb))
    dwq, dwk = torch.from_numpy(wq).cuda(), torch.from_numpy(wk).cuda()
    fused = from_dev(ops.joint_attention(to_dev(q), to_dev(k), to_dev(v), q_norm=dwq, k_norm=dwk, q_table=tq,
                                         k_table=tk, pairing=1, causal=bool(causal), p0=p0))
    ws = torch.empty(ops.workspace_bytes(Sk, HK), dtype=torch.uint8, device="cuda")
    ops.joint_kv_prepare(to_dev(k), to_dev(v), ws, k_norm=dwk, k_table=tk, pairing=1)
    qp = ops.joint_q_prepare(to_dev(q), q_norm=dwq, q_table=tq, pairing=1)
    apart = from_dev(ops.joint_attention_images(qp, ws, Sk, HK, causal=bool(causal), p0=p0))
    inplace = from_dev(ops.joint_attention_images(qp, ws, Sk, HK, qp, causal=bool(causal), p0=p0))
    torch.cuda.synchronize()
    assert np.array_equal(apart, fused) and np.array_equal(inplace, fused)


@pytest.mark.parametrize("kind,pairing,rot,n_pre,offset", [
    (1, 0, 128, 0, 0),      # cos / sin rows 16-byte aligned: 16-byte table loads
    (1, 0, 128, 0, 1),      # tables offset by one float: the per-pair loads
    (1, 1, 64, 30, 0),      # split-half, partial rot, a prefix
    (2, 1, 96, 0, 0),       # bf16 2x2 table (H3 form)
    (1, 0, 128, 333, 0),    # every key a prefix key: keys and queries in two launches
])
def test_one_launch_prepare_equals_the_stages(kind, pairing, rot, n_pre, offset):
    """lr_joint_prepare (queries, keys and values in one launch: the fused call's first launch, plus the value rows
    copied into the workspace) writes the same prepared queries, key images and value rows, bit for bit, as
    lr_joint_q_prepare + lr_joint_kv_prepare."""
    Sq, Sk, H, HK = 300, 333, 4, 2
    print(f"\n[one-launch prepare] kind={kind} pairing={pairing} rot={rot} n_pre={n_pre} offset={offset}", flush=True)
    q, k, v, wq, wk, qa, qb, ka, kb = _fused_case(36, Sq, Sk, H, HK, kind, pairing, rot)

    def tab(t):   # the table on the device, starting `offset` floats into its allocation (same row stride)
        if t is None:
            return None
        d = _dev_table(t)
        if offset == 0:
            return d
        flat = torch.zeros(d.numel() + 8, dtype=d.dtype, device="cuda")
        view = flat[offset:offset + d.numel()].view(d.shape)
        view.copy_(d)
        return view
    tq, tk = (tab(qa), tab(qb)), (tab(ka), tab(kb))
    dwq, dwk = torch.from_numpy(wq).cuda(), torch.from_numpy(wk).cuda()
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    ws1 = torch.zeros(ops.workspace_bytes(Sk, HK), dtype=torch.uint8, device="cuda")
    ws2 = torch.full_like(ws1, 0x5A)
    ops.joint_kv_prepare(dk, dv, ws1, k_norm=dwk, table_kind=kind, k_table=tk, pairing=pairing, rot=rot, n_pre=n_pre)
    qp1 = ops.joint_q_prepare(dq, q_norm=dwq, table_kind=kind, q_table=tq, pairing=pairing, rot=rot)
    qp2 = ops.joint_prepare(dq, dk, dv, ws2, q_norm=dwq, k_norm=dwk, table_kind=kind, q_table=tq, k_table=tk,
                            pairing=pairing, rot=rot, n_pre=n_pre)
    torch.cuda.synchronize()
    img = 2 * HK * ((Sk + 63) // 64) * 16384
    assert np.array_equal(from_dev(qp2), from_dev(qp1)), "prepared queries differ"
    assert torch.equal(ws2[:img], ws1[:img]), "tile images differ"
    assert not ws2[-1024:].view(torch.int32).any(), "the arrival counters are zeroed"


def test_prepared_rejects_plain_configs():
    """The prepared call runs the streaming kernel only: the plain-attention configurations are rejected."""
    Sk, HK = 64, 1
    ws = torch.zeros(ops.workspace_bytes(Sk, HK), dtype=torch.uint8, device="cuda")
    q = to_dev(oracle.synth_bf16(42, 1, (32, 1, 128)))
    for cfg in (ops.CFG_PIPE_W8, ops.CFG_PIPE_W4, 3, 8):
        with pytest.raises(Exception):
            ops.joint_attention_prepared(q, ws, Sk, HK, table_kind=ops.TABLE_NONE, config=cfg)
