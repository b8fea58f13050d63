"""Kandinsky-6's attention calls (src/engines/kandinsky6/dit/launch.zig:239-300) through this library: the four
unmasked shapes of its flash dispatch (visual self 50,220 x 32 heads, video-from-audio 50,220 <- 218, audio-from-video
218 <- 50,220 x 16 heads, audio self 218 x 16 heads; rows of heads x 128, scale 1/sqrt(128)) via lr_attention_bf16,
and the key-padding-masked calls (attention.zig:21-27) via lr_attention_kmask_bf16. Checked against the fp32 / fp64
oracle (sampled query rows for the 50k shapes), at the bar of every parity test here (tests/_util.py): max-abs 2e-2,
mean-abs 2e-3 and relative L2 3e-3 on the bf16 output."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle  # noqa: E402
from tests._util import assert_close  # noqa: E402

pytestmark = pytest.mark.gpu
SCALE = float(np.float32(1.0) / np.sqrt(np.float32(128.0)))


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _f32(t):
    return oracle.bf16_to_f32(_bits(t))


def _rand(shape, g, dev):
    return torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)


@pytest.mark.parametrize("W,S,H", [(50220, 50220, 32), (50220, 218, 32), (218, 50220, 16), (218, 218, 16)])
def test_k6_flash_shapes(W, S, H):
    from localrouter_amd import ops
    dev = torch.device("cuda", 0)
    print(f"k6 shape: W {W} nkeys {S} heads {H}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(W + S + H)
    q, k, v = _rand((W, H, 128), g, dev), _rand((S, H, 128), g, dev), _rand((S, H, 128), g, dev)
    out = ops.attention(q, k, v, scale=SCALE)
    torch.cuda.synchronize()
    rows = np.unique(np.linspace(0, W - 1, min(W, 48)).astype(np.int64))
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), scale=SCALE, precise=False, rows=rows)
    mx, mn = assert_close(_bits(out)[rows], ref, what=f"k6 {W}x{S}x{H}")
    print(f"  max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)


@pytest.mark.parametrize("W,S,H,keep", [(300, 218, 4, 0.7), (64, 218, 32, 0.3), (130, 1000, 2, 0.95)])
def test_kmask_random(W, S, H, keep):
    from localrouter_amd import ops
    dev = torch.device("cuda", 0)
    print(f"kmask: W {W} nkeys {S} heads {H} keep {keep}", flush=True)
    g = torch.Generator(device=dev)
    g.manual_seed(W * 7 + S)
    q, k, v = _rand((W, H, 128), g, dev), _rand((S, H, 128), g, dev), _rand((S, H, 128), g, dev)
    rng = np.random.default_rng(S + H)
    m = (rng.random(S) < keep).astype(np.uint8)
    m[rng.integers(S)] = 1
    kmask = torch.from_numpy(m).to(dev)
    out = ops.attention_kmask(q, k, v, kmask, n_valid=int(m.sum()), scale=SCALE)
    torch.cuda.synchronize()
    keep_idx = np.nonzero(m)[0]
    ref = oracle.attention(_f32(q), _f32(k)[keep_idx], _f32(v)[keep_idx], scale=SCALE)
    mx, mn = assert_close(_bits(out), ref, what=f"kmask {W}x{S}x{H}")
    print(f"  kept {len(keep_idx)}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)


def test_kmask_all_and_one():
    """All keys kept: the same bits as the unmasked call. One key kept: every output row is that key's value row."""
    from localrouter_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    W, S, H = 100, 218, 4
    q, k, v = _rand((W, H, 128), g, dev), _rand((S, H, 128), g, dev), _rand((S, H, 128), g, dev)
    full = ops.attention_kmask(q, k, v, torch.ones(S, dtype=torch.uint8, device=dev), scale=SCALE)
    plain = ops.attention(q, k, v, scale=SCALE)
    one = torch.zeros(S, dtype=torch.uint8, device=dev)
    one[117] = 1
    single = ops.attention_kmask(q, k, v, one, n_valid=1, scale=SCALE)
    torch.cuda.synchronize()
    assert torch.equal(full, plain)
    assert torch.equal(single, v[117].unsqueeze(0).expand(W, H, 128))


def test_kmask_fewer_kept_than_declared_is_memory_safe():
    """A caller error (n_valid above the mask's count) leaves slots without a key: they become zero rows, no read out
    of bounds; the result is then that of attention with zero keys added."""
    from localrouter_amd import ops
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    W, S, H = 16, 64, 2
    q, k, v = _rand((W, H, 128), g, dev), _rand((S, H, 128), g, dev), _rand((S, H, 128), g, dev)
    m = torch.zeros(S, dtype=torch.uint8, device=dev)
    m[:10] = 1
    ws = torch.full((int(ops._lib.load().lr_attention_kmask_workspace_bytes(12, H)),), 0x7f, dtype=torch.uint8,
                    device=dev)
    out = ops.attention_kmask(q, k, v, m, n_valid=12, scale=SCALE, workspace=ws)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("W,S,H,HK", [(218, 50220, 16, 16), (100, 4000, 4, 2), (256, 1000, 3, 3), (37, 1100, 8, 1)])
def test_key_split_attention(W, S, H, HK):
    """lr_attention_bf16_ws splits few-query calls over the keys; the merged result meets the same bar as the unsplit
    call (sampled rows at the K6 shape, every row otherwise)."""
    from localrouter_amd import _lib, ops
    dev = torch.device("cuda", 0)
    nb = int(_lib.load().lr_attention_ws_bytes(W, H, S, 0))
    print(f"key split: W {W} nkeys {S} heads {H}/{HK} workspace {nb}", flush=True)
    assert nb > 0
    g = torch.Generator(device=dev)
    g.manual_seed(W + S)
    q, k, v = _rand((W, H, 128), g, dev), _rand((S, HK, 128), g, dev), _rand((S, HK, 128), g, dev)
    out = ops.attention_ws(q, k, v, scale=SCALE)
    plain = ops.attention(q, k, v, scale=SCALE)
    torch.cuda.synchronize()
    rows = np.arange(W)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), scale=SCALE, precise=False, rows=rows)
    dp = np.abs(_f32(out) - _f32(plain))
    mx, mn = assert_close(_bits(out), ref, what=f"key split {W}x{S}x{H}/{HK}")
    print(f"  max-abs {mx:.3e} mean-abs {mn:.3e}; vs unsplit max {dp.max():.3e}", flush=True)
