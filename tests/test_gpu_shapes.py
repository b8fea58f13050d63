"""GPU parity at BASELINE's own shapes, through the C ABI (lr_joint_attention_fused).

  cfg1  256 text + 1024 image tokens (32x32 grid), 24 heads x 128      -- every query row checked
  cfg2  512 text + 4096 image tokens (64x64 grid), 24 heads x 128      -- every query row checked
  cfg4  512 text + 3 x 4096 image tokens (3-frame edit layout)          -- sampled query rows
  cfg5  512 text + 49 x 44 x 80 video tokens (172,992), one pass        -- sampled query rows
  qwen21  4096 image queries x 32 heads over an 80-key cached prefix + 4096 keys (the reference's own call shape,
          dit.zig:252-293)                                              -- sampled query rows

Per-head QK-RMSNorm eps 1e-6 with weights 1.0, RoPE theta 10000 (text rows un-rotated), scale f32(1/sqrt(128)),
non-causal. The oracle is the CPU fp32 flash-style path (oracle/lro.c, pinned against fp64 and torch SDPA on the
CPU). Bar: max-abs 2e-2, mean-abs 2e-3, relative L2 3e-3 on the bf16 output.
"""
from __future__ import annotations

import time

import numpy as np
import pytest

import oracle
from tests._util import assert_close, from_dev, to_dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from localrouter_amd import ops, rope  # noqa: E402

H = 24


def _run_fused(q, k, v, cos, sin, config=ops.CFG_AUTO):
    tc, ts = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    out = ops.joint_attention(q, k, v, table_kind=ops.TABLE_COSSIN_F32, q_table=(tc, ts), eps=1e-6, config=config)
    torch.cuda.synchronize()
    return out


def _bf16(x):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(x))


def _oracle_rows(qb, kb, vb, cos, sin, rows):
    """fp32 oracle output for the given query rows: q/k normalised and rotated and stored as bf16 (the reference's
    chain, dit.zig:252-263), then attention over every key."""
    qh = oracle.rms_rope(np.ascontiguousarray(qb[rows]), None, table_kind=oracle.TABLE_COSSIN_F32,
                         ta=np.ascontiguousarray(cos[rows]), tb=np.ascontiguousarray(sin[rows]), eps=1e-6)
    kh = oracle.rms_rope(kb, None, table_kind=oracle.TABLE_COSSIN_F32, ta=cos, tb=sin, eps=1e-6)
    return oracle.attention(_bf16(qh), _bf16(kh), oracle.bf16_to_f32(vb), precise=False)


@pytest.mark.parametrize("cfg", [ops.CFG_AUTO])
@pytest.mark.parametrize("name,n_text,grid", [("cfg1", 256, (32, 32)), ("cfg2", 512, (64, 64))])
def test_baseline_image_shapes_all_rows(name, n_text, grid, cfg):
    cos, sin = rope.grid2d_table(n_text, *grid)
    S = cos.shape[0]
    print(f"\n[{name}] S={S} H={H} config={cfg}", flush=True)
    qb = oracle.synth_bf16(100, 1, (S, H, 128))
    kb = oracle.synth_bf16(100, 2, (S, H, 128))
    vb = oracle.synth_bf16(100, 3, (S, H, 128))
    out = from_dev(_run_fused(to_dev(qb), to_dev(kb), to_dev(vb), cos, sin, config=cfg))
    ref = _oracle_rows(qb, kb, vb, cos, sin, np.arange(S))
    mx, mn = assert_close(out, ref, what=name)
    print(f"[{name}] max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)


def test_edit_shape_sampled_rows():
    cos, sin = rope.edit_table(512, 3, 64, 64)
    S = cos.shape[0]
    assert S == 12800
    print(f"\n[cfg4] S={S} H={H}", flush=True)
    qb = oracle.synth_bf16(104, 1, (S, H, 128))
    kb = oracle.synth_bf16(104, 2, (S, H, 128))
    vb = oracle.synth_bf16(104, 3, (S, H, 128))
    out = from_dev(_run_fused(to_dev(qb), to_dev(kb), to_dev(vb), cos, sin))
    rows = np.sort(np.random.default_rng(4).choice(S, size=768, replace=False))
    rows[:4] = [0, 511, 512, S - 1]   # text / first image token / last token
    rows = np.unique(rows)
    ref = _oracle_rows(qb, kb, vb, cos, sin, rows)
    mx, mn = assert_close(out[rows], ref, what="cfg4")
    print(f"[cfg4] {len(rows)} rows: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)


def test_qwen21_reference_shape_sampled_rows():
    """The reference's own call shape (Qwen-Image 2.1, src/engines/qwen_image/dit.zig:252-293, the shape of its
    published pattn2 / cuDNN timings): 4,096 image queries x 32 heads over an 80-row cached text prefix (keys already
    rotated, used as given: n_pre = 80) plus the 4,096 image keys, whose k-table row is j - 80."""
    n_pre, gh, gw, Hq = 80, 64, 64, 32
    cos_all, sin_all = rope.grid2d_table(n_pre, gh, gw)
    cos, sin = np.ascontiguousarray(cos_all[n_pre:]), np.ascontiguousarray(sin_all[n_pre:])
    Sq = cos.shape[0]
    Sk = n_pre + Sq
    print(f"\n[qwen21] Sq={Sq} Sk={Sk} n_pre={n_pre} H={Hq}", flush=True)
    qb = oracle.synth_bf16(108, 1, (Sq, Hq, 128))
    kb = oracle.synth_bf16(108, 2, (Sk, Hq, 128))
    vb = oracle.synth_bf16(108, 3, (Sk, Hq, 128))
    tc, ts = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    out = from_dev(ops.joint_attention(to_dev(qb), to_dev(kb), to_dev(vb), table_kind=ops.TABLE_COSSIN_F32,
                                       q_table=(tc, ts), eps=1e-6, n_pre=n_pre))
    rows = np.unique(np.concatenate([[0, 63, 64, Sq - 1],
                                     np.random.default_rng(8).choice(Sq, size=380, replace=False)]))
    qh = oracle.rms_rope(np.ascontiguousarray(qb[rows]), None, table_kind=oracle.TABLE_COSSIN_F32,
                         ta=np.ascontiguousarray(cos[rows]), tb=np.ascontiguousarray(sin[rows]), eps=1e-6)
    kh = oracle.rms_rope(np.ascontiguousarray(kb[n_pre:]), None, table_kind=oracle.TABLE_COSSIN_F32, ta=cos, tb=sin,
                         eps=1e-6)
    kall = np.concatenate([oracle.bf16_to_f32(kb[:n_pre]), _bf16(kh)])
    ref = oracle.attention(_bf16(qh), kall, oracle.bf16_to_f32(vb), precise=False)
    mx, mn = assert_close(out[rows], ref, what="qwen21")
    print(f"[qwen21] {len(rows)} rows: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)


@pytest.mark.slow
def test_video_shape_single_pass_sampled_rows():
    """172,992 tokens x 24 heads in one call; inputs drawn on the GPU (torch Philox, seed 5), copied to the host for
    the oracle on 96 sampled query rows over all keys."""
    t0 = time.time()
    cos, sin = rope.video3d_table(512, 49, 44, 80)
    S = cos.shape[0]
    assert S == 172992
    print(f"\n[cfg5] S={S} H={H}: generating inputs", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    q = torch.randn((S, H, 128), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((S, H, 128), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((S, H, 128), generator=g, device="cuda").to(torch.bfloat16)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    out = _run_fused(q, k, v, cos, sin)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    print(f"[cfg5] one pass {ms:.1f} ms ({4.0 * S * S * 128 * H / ms / 1e9:.1f} TFLOP/s)", flush=True)
    assert torch.isfinite(out.float()).all()
    rows = np.unique(np.concatenate([[0, 511, 512, S - 1],
                                     np.random.default_rng(5).choice(S, size=92, replace=False)]))
    qb = from_dev(q[torch.from_numpy(rows).cuda()])
    kb, vb = from_dev(k), from_dev(v)
    del q, k, v
    got = from_dev(out[torch.from_numpy(rows).cuda()])
    del out
    torch.cuda.empty_cache()
    print(f"[cfg5] oracle on {len(rows)} rows ({time.time() - t0:.0f} s so far)", flush=True)
    qh = oracle.rms_rope(qb, None, table_kind=oracle.TABLE_COSSIN_F32, ta=np.ascontiguousarray(cos[rows]),
                         tb=np.ascontiguousarray(sin[rows]), eps=1e-6)
    kh = oracle.rms_rope(kb, None, table_kind=oracle.TABLE_COSSIN_F32, ta=cos, tb=sin, eps=1e-6)
    del kb
    ref = oracle.attention(_bf16(qh), _bf16(kh), oracle.bf16_to_f32(vb), precise=False)
    mx, mn = assert_close(got, ref, what="cfg5")
    print(f"[cfg5] max-abs {mx:.3e} mean-abs {mn:.3e} ({time.time() - t0:.0f} s)", flush=True)


def test_fused_matches_plain_attention_over_rotated_operands():
    """Two product paths compute the same function: the fused call (streaming kernel over tile images, queries scaled
    before their bf16 rounding) and lr_rms_rope_bf16 + lr_attention_bf16 (value rows, running maximum) agree to the
    bar at a mid-size shape."""
    cos, sin = rope.grid2d_table(64, 16, 16)
    S = cos.shape[0]
    print(f"\n[fused vs plain] S={S} H=4", flush=True)
    qb = oracle.synth_bf16(106, 1, (S, 4, 128))
    kb = oracle.synth_bf16(106, 2, (S, 4, 128))
    vb = oracle.synth_bf16(106, 3, (S, 4, 128))
    tc, ts = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    fused = from_dev(ops.joint_attention(to_dev(qb), to_dev(kb), to_dev(vb), table_kind=ops.TABLE_COSSIN_F32,
                                         q_table=(tc, ts)))
    qh, kh = torch.empty_like(to_dev(qb)), torch.empty_like(to_dev(kb))
    for src, dst in ((to_dev(qb), qh), (to_dev(kb), kh)):
        ops.rms_rope(src, dst, None, n=S, heads=4, src_row_stride=4 * 128, dst_row_stride=4 * 128,
                     table_kind=ops.TABLE_COSSIN_F32, table_a=tc, table_b=ts)
    plain = from_dev(ops.attention(qh, kh, to_dev(vb)))
    torch.cuda.synchronize()
    # two bf16 implementations against each other: each carries its own P and output roundings, so the relative L2
    # bar is sqrt(2) times the one against the oracle
    assert_close(fused, (plain.astype(np.uint32) << 16).view(np.float32), what="fused vs plain", rel=4.3e-3)
