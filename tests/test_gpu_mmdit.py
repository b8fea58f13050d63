"""The MMDiT block forward (include/lr_mmdit.h) on the GPU against its fp32 oracle (oracle/mmdit.py).

Bar: the outputs (bf16 residual streams, values of order 1) within max-abs 6.25e-2 and mean-abs 2e-3 of the oracle,
which rounds at the same points; and the block's update (output - input) within 3 % relative L2 of the oracle's,
which a wrong gate, modulation chunk or branch would miss by far. The composition has no reference block to be
pinned to (parity unpinned beyond the oracle's own checks in tests/test_oracle_mmdit.py)."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle  # noqa: E402
from oracle import mmdit as om  # noqa: E402

pytestmark = pytest.mark.gpu


def _rope(n_txt, gh, gw):
    from localrouter_amd import rope_host
    return rope_host.grid2d_table(n_txt, gh, gw)


def _to_np_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _run(n_txt, gh, gw, D, F, std, seed=0, zero_mod=False, tval=0.5, tune=False):
    from localrouter_amd import mmdit
    dev = torch.device("cuda", 0)
    n_img = gh * gw
    print(f"mmdit block: n_txt {n_txt} n_img {n_img} D {D} F {F} std {std} zero_mod {zero_mod}", flush=True)
    w = mmdit.make_weights(D, F, dev, seed=seed, std=std, zero_mod=zero_mod)
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    txt = torch.randn((n_txt, D), generator=g, device=dev).to(torch.bfloat16)
    img = torch.randn((n_img, D), generator=g, device=dev).to(torch.bfloat16)
    cos_np, sin_np = _rope(n_txt, gh, gw)
    cos, sin = torch.from_numpy(cos_np).to(dev), torch.from_numpy(sin_np).to(dev)
    t = torch.tensor([tval], dtype=torch.float32, device=dev)
    txt0, img0 = _to_np_bits(txt), _to_np_bits(img)
    blk = mmdit.MMDiTBlock(w)
    if tune:
        blk.tune(n_txt, n_img, candidates=8)
    blk(txt, img, t, cos, sin)
    torch.cuda.synchronize()
    got_t, got_i = oracle.bf16_to_f32(_to_np_bits(txt)), oracle.bf16_to_f32(_to_np_bits(img))
    wn = {k: (_to_np_bits(v) if v.dtype == torch.bfloat16 else v.cpu().numpy()) for k, v in w.items()}
    blk.close()
    return (txt0, img0), (got_t, got_i), wn, cos_np, sin_np, tval


def _check(case):
    (txt0, img0), (got_t, got_i), wn, cos_np, sin_np, tval = case
    ref_t, ref_i = om.mmdit_block(txt0, img0, wn, tval, cos_np, sin_np)
    got = np.concatenate([got_t, got_i])
    ref = np.concatenate([ref_t, ref_i])
    x0 = oracle.bf16_to_f32(np.concatenate([txt0, img0]))
    err = np.abs(got - ref)
    rel = np.linalg.norm((got - x0) - (ref - x0)) / max(np.linalg.norm(ref - x0), 1e-30)
    print(f"  max-abs {err.max():.3e} mean-abs {err.mean():.3e} update rel-L2 {rel:.3e} "
          f"|update| mean {np.abs(ref - x0).mean():.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err.max() <= 6.25e-2 and err.mean() <= 2e-3
    assert rel <= 0.03


def test_block_small():
    _check(_run(16, 6, 8, 256, 512, 0.05))


def test_block_image_only_and_odd_rows():
    _check(_run(0, 5, 9, 384, 1024, 0.05, seed=3, tval=0.81))


def test_block_adaln_zero_is_identity():
    """Zero modulation weights: every gate is 0, both streams come back bit for bit."""
    (txt0, img0), (got_t, got_i), *_ = _run(24, 4, 10, 256, 768, 0.05, seed=5, zero_mod=True)
    assert np.array_equal(got_t, oracle.bf16_to_f32(txt0)) and np.array_equal(got_i, oracle.bf16_to_f32(img0))


def test_block_cfg3_full_shape():
    """512 text + 4096 image tokens (64 x 64 grid), hidden 3072, 24 heads, MLP 12288, weights
    N(0, 0.02), activations N(0, 1); GEMM candidates tuned first, as bench.py runs it."""
    _check(_run(512, 64, 64, 3072, 12288, 0.02, seed=7, tune=True))


def test_block_tuned_small():
    _check(_run(40, 8, 12, 512, 1536, 0.05, seed=11, tune=True))


def test_block_repeated_calls_reuse_plans():
    """A second call of the same shape on the same context gives the same bits as the first on fresh inputs."""
    from localrouter_amd import mmdit
    dev = torch.device("cuda", 0)
    D, F, n_txt, gh, gw = 256, 512, 8, 4, 4
    w = mmdit.make_weights(D, F, dev, seed=9, std=0.05)
    blk = mmdit.MMDiTBlock(w)
    cos_np, sin_np = _rope(n_txt, gh, gw)
    cos, sin = torch.from_numpy(cos_np).to(dev), torch.from_numpy(sin_np).to(dev)
    t = torch.tensor([0.3], dtype=torch.float32, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(10)
    txt = torch.randn((n_txt, D), generator=g, device=dev).to(torch.bfloat16)
    img = torch.randn((gh * gw, D), generator=g, device=dev).to(torch.bfloat16)
    outs = []
    for _ in range(2):
        a, b = txt.clone(), img.clone()
        blk(a, b, t, cos, sin)
        outs.append((a, b))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    blk.close()


def test_block_needs_its_plans_and_launches_nothing_without_them():
    """The block call does no planning of its own (it may be recorded under graph capture): on a context whose shape
    was not planned it returns hipErrorNotReady (600) before any launch, and after lr_mmdit_plan the same call runs."""
    import ctypes
    from localrouter_amd import mmdit
    dev = torch.device("cuda", 0)
    D, F, n_txt, gh, gw = 256, 512, 8, 4, 4
    n_img = gh * gw
    w = mmdit.make_weights(D, F, dev, seed=13, std=0.05)
    blk = mmdit.MMDiTBlock(w)
    g = torch.Generator(device=dev)
    g.manual_seed(14)
    txt = torch.randn((n_txt, D), generator=g, device=dev).to(torch.bfloat16)
    img = torch.randn((n_img, D), generator=g, device=dev).to(torch.bfloat16)
    cos_np, sin_np = _rope(n_txt, gh, gw)
    cos, sin = torch.from_numpy(cos_np).to(dev), torch.from_numpy(sin_np).to(dev)
    t = torch.tensor([0.5], dtype=torch.float32, device=dev)
    ws = blk.workspace(n_txt, n_img)
    before = (_to_np_bits(txt), _to_np_bits(img))
    call = lambda: mmdit.lib().lr_mmdit_block_bf16(blk.ctx, ctypes.byref(blk.cw), txt.data_ptr(), img.data_ptr(),
                                                   n_txt, n_img, D, F, t.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                                   ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert call() == 600
    torch.cuda.synchronize()
    assert np.array_equal(_to_np_bits(txt), before[0]) and np.array_equal(_to_np_bits(img), before[1])
    assert mmdit.lib().lr_mmdit_plan(blk.ctx, n_txt, n_img, D, F) == 0
    assert call() == 0
    torch.cuda.synchronize()
    assert not np.array_equal(_to_np_bits(img), before[1])
    blk.close()


def test_block_modulation_chunk_meanings():
    """The oracle's chunk-meaning identities (tests/test_oracle_mmdit.py) on the GPU block: on zero inputs a scale
    changes no bit, a shift does, and a zero gate shuts its own branch (the output is exactly 0)."""
    from localrouter_amd import mmdit
    from tests.test_oracle_mmdit import (MEANING_D, MEANING_F, MEANING_GRID, MEANING_ST, chunk_weights,
                                         meaning_cases)
    dev = torch.device("cuda", 0)
    D, F, St, (gh, gw) = MEANING_D, MEANING_F, MEANING_ST, MEANING_GRID
    cos_np, sin_np = _rope(St, gh, gw)
    cos, sin = torch.from_numpy(cos_np).to(dev), torch.from_numpy(sin_np).to(dev)
    t = torch.zeros(1, dtype=torch.float32, device=dev)
    rng = np.random.default_rng(11)
    for name, a, b, extra, outcome in meaning_cases(rng):
        seed = int(rng.integers(1 << 30))
        print(f"mmdit chunk meaning: {name} -> {outcome}", flush=True)
        outs = []
        for chunks in (a, b):
            wn = chunk_weights(np.random.default_rng(seed), D, F, {"txt": chunks, "img": chunks}, **extra)
            w = {k: (torch.from_numpy(v.view(np.int16)).to(dev).view(torch.bfloat16) if v.dtype == np.uint16
                     else torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(dev)) for k, v in wn.items()}
            txt = torch.zeros((St, D), dtype=torch.bfloat16, device=dev)
            img = torch.zeros((gh * gw, D), dtype=torch.bfloat16, device=dev)
            blk = mmdit.MMDiTBlock(w)
            blk(txt, img, t, cos, sin)
            torch.cuda.synchronize()
            outs.append(np.concatenate([_to_np_bits(txt), _to_np_bits(img)]))
            blk.close()
        same = np.array_equal(outs[0], outs[1])
        if outcome == "zero":
            assert same and not np.any(oracle.bf16_to_f32(outs[0])), name
        elif outcome == "same":
            assert same and np.any(outs[0]), name
        else:
            assert not same, name

