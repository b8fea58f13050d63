"""lr_joint_attention_fused_noalloc (no workspace argument, a static scratch array per GPU) against
lr_joint_attention_fused, through the C ABI: the same bits on two calls in a row (the second smaller), and the size
limit rejected before anything is launched."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import from_dev, to_dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

from localrouter_amd import _lib, ops  # noqa: E402

HIP_ERROR_OUT_OF_MEMORY = 2


def _case(seed, Sq, Sk, H, HK):
    q = to_dev(oracle.synth_bf16(seed, 1, (Sq, H, 128)))
    k = to_dev(oracle.synth_bf16(seed, 2, (Sk, HK, 128)))
    v = to_dev(oracle.synth_bf16(seed, 3, (Sk, HK, 128)))
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-np.pi, np.pi, size=(max(Sq, Sk), 64))
    cos = torch.from_numpy(np.cos(ang).astype(np.float32)).cuda()
    sin = torch.from_numpy(np.sin(ang).astype(np.float32)).cuda()
    wq = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)).cuda()
    wk = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)).cuda()
    return q, k, v, cos, sin, wq, wk


def _noalloc(q, k, v, out, cos, sin, wq, wk, Sq, Sk, H, HK, causal=0, p0=0, n_pre=0):
    rs_q, rs_k, rs_o = H * 128, HK * 128, H * 128
    return _lib.load().lr_joint_attention_fused_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), wq.data_ptr(), wk.data_ptr(), ops.TABLE_COSSIN_F32,
        cos.data_ptr(), sin.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.stride(0), ops.PAIR_INTERLEAVED, 128, 1e-6,
        Sq, Sk, H, HK, p0, causal, ops.SCALE_128, rs_q, rs_k, rs_k, rs_o, n_pre,
        torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("first,second", [((1000, 1100, 4, 2, 0, 0), (300, 257, 2, 1, 1, 40)),
                                          ((4608, 4608, 24, 24, 0, 0), (64, 65, 1, 1, 0, 0))])
def test_noalloc_equals_fused_twice(first, second):
    assert _lib.load().lr_attn_init() == 0
    for seed, (Sq, Sk, H, HK, causal, p0) in ((51, first), (52, second)):
        print(f"\n[noalloc] Sq={Sq} Sk={Sk} H={H} HK={HK} causal={causal} p0={p0}", flush=True)
        q, k, v, cos, sin, wq, wk = _case(seed, Sq, Sk, H, HK)
        out = torch.full((Sq, H, 128), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert _noalloc(q, k, v, out, cos, sin, wq, wk, Sq, Sk, H, HK, causal, p0) == 0
        ref = ops.joint_attention(q, k, v, q_norm=wq, k_norm=wk, table_kind=ops.TABLE_COSSIN_F32, q_table=(cos, sin),
                                  k_table=(cos, sin), causal=bool(causal), p0=p0)
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out), from_dev(ref)), "no-alloc result differs from the fused call's"


def test_noalloc_rejects_beyond_its_scratch():
    """HK 24 with Sk 5441 needs 86 tiles per head, past the 2048 tiles of 2 x 16 KB the 64 MiB array holds: the call
    returns hipErrorOutOfMemory and writes nothing."""
    Sq, Sk, H, HK = 64, 5441, 24, 24
    q, k, v, cos, sin, wq, wk = _case(53, Sq, Sk, H, HK)
    out = torch.zeros((Sq, H, 128), dtype=torch.bfloat16, device="cuda")
    assert _noalloc(q, k, v, out, cos, sin, wq, wk, Sq, Sk, H, HK) == HIP_ERROR_OUT_OF_MEMORY
    torch.cuda.synchronize()
    assert not out.any()
    # the largest size that fits runs
    Sk = 5440
    q, k, v, cos, sin, wq, wk = _case(54, Sq, Sk, H, HK)
    assert _noalloc(q, k, v, out, cos, sin, wq, wk, Sq, Sk, H, HK) == 0
    ref = ops.joint_attention(q, k, v, q_norm=wq, k_norm=wk, table_kind=ops.TABLE_COSSIN_F32, q_table=(cos, sin),
                              k_table=(cos, sin))
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(out), from_dev(ref))
