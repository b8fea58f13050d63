"""The MMDiT block oracle (oracle/mmdit.py) pinned on the CPU: closed forms and special values of its elementwise
pieces, the LayerNorm moments, the linear layout against a brute-force loop, the adaLN-zero identity, and the meaning
of each modulation chunk (identities on zero inputs that planted shift/scale and gate swaps fail)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from oracle import mmdit as om


def test_sinusoid_closed_form():
    """t = 0: cos 1 / sin 0. Other t: cos / sin of 1000 t (after the reference's two bf16 roundings) times
    exp(-ln(1e4) i / 128), to bf16 rounding."""
    e0 = om.sinusoid(0.0)
    assert np.all(e0[:128] == 1.0) and np.all(e0[128:] == 0.0)
    for t in (0.25, 0.5, 0.937):
        tr = float(om.bf16r(np.array([om.bf16r(np.array([t * 1000.0], np.float32))[0] / 1000.0], np.float32))[0])
        tr *= 1000.0
        i = np.arange(128)
        freq = np.exp(-math.log(10000.0) * i / 128.0)
        ref = np.concatenate([np.cos(tr * freq), np.sin(tr * freq)])
        assert np.abs(om.sinusoid(t) - ref).max() <= 2.0 ** -8 * 1.01
    # 0.5 -> 500 is exact in bf16; 0.937 -> 937 is not (bf16 keeps 8 bits): the rounding shows in the angle
    assert float(om.bf16r(np.array([937.0], np.float32))[0]) == 936.0


def test_gelu_tanh_closed_form():
    x = np.linspace(-6, 6, 1001).astype(np.float32)
    ref = 0.5 * x.astype(np.float64) * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x.astype(np.float64) ** 3)))
    assert np.abs(om.gelu_tanh(x) - ref).max() < 2e-6
    assert om.gelu_tanh(np.zeros(1, np.float32))[0] == 0.0
    # odd part: gelu(x) - gelu(-x) = x
    assert np.abs(om.gelu_tanh(x) - om.gelu_tanh(-x) - x).max() < 2e-6
    # the tanh approximation stays within 1e-3 of the exact (erf) GELU
    from scipy.special import erf
    exact = 0.5 * x * (1 + erf(x / np.sqrt(2)))
    assert np.abs(om.gelu_tanh(x) - exact).max() < 1e-3


def test_layer_norm_moments():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((8, 3072)) * 3 + 1.5).astype(np.float32)
    y = om.layer_norm_modulate(x, np.zeros(3072, np.float32), np.zeros(3072, np.float32))
    assert np.abs(y.mean(axis=1)).max() < 1e-3
    assert np.abs(y.std(axis=1) - 1).max() < 2e-3
    # shift and scale: y' = y (1 + s) + b
    b, s = np.full(3072, 0.5, np.float32), np.full(3072, -0.25, np.float32)
    y2 = om.layer_norm_modulate(x, b, s)
    assert np.abs(y2 - (y * 0.75 + 0.5)).max() < 2e-2


def test_linear_layout_brute_force():
    rng = np.random.default_rng(1)
    x = om.bf16r(rng.standard_normal((3, 5)).astype(np.float32))
    w = om.bf16r(rng.standard_normal((4, 5)).astype(np.float32))   # [out, in]
    y = om.linear(x, w)
    for m in range(3):
        for n in range(4):
            assert y[m, n] == om.bf16r(np.array([sum(float(x[m, k]) * float(w[n, k]) for k in range(5))],
                                                np.float32))[0]


def test_gated_residual_is_fma():
    x = np.array([[1.0, -2.0, 3.0]], np.float32)
    a = np.array([[0.5, 0.25, -1.0]], np.float32)
    g = np.array([2.0, 0.0, 0.5], np.float32)
    assert om.gated_residual(x, a, g).tolist() == [[2.0, -2.0, 2.5]]


def _small_weights(rng, D, F, zero_mod=False, std=0.05):
    # std 0.05 at D = 256 gives gates of about 0.2: at 0.02 they would be ~0.01 and most updates would round away
    def rnd(*shape):
        return oracle.f32_to_bf16((rng.standard_normal(shape) * std).astype(np.float32))
    w = {"t1": rnd(D, 256), "t2": rnd(D, D), "q_norm": np.ones(128, np.float32), "k_norm": np.ones(128, np.float32)}
    for s in ("txt", "img"):
        w[f"{s}.mod"] = rnd(6 * D, D) * (0 if zero_mod else 1)
        w[f"{s}.qkv"], w[f"{s}.out"] = rnd(3 * D, D), rnd(D, D)
        w[f"{s}.mlp_up"], w[f"{s}.mlp_down"] = rnd(F, D), rnd(D, F)
    return w


def test_adaln_zero_identity_and_branches():
    """Zero modulation weights make every gate 0: the block returns its input bit for bit. With the modulation on,
    both streams change, by about the gate times the branch outputs."""
    from localrouter_amd import rope
    rng = np.random.default_rng(2)
    D, F, St, Si = 256, 512, 16, 48
    cos, sin = rope.grid2d_table(St, 6, 8)
    txt = oracle.f32_to_bf16(rng.standard_normal((St, D)).astype(np.float32))
    img = oracle.f32_to_bf16(rng.standard_normal((Si, D)).astype(np.float32))
    yt, yi = om.mmdit_block(txt, img, _small_weights(rng, D, F, zero_mod=True), 0.5, cos, sin)
    assert np.array_equal(yt, oracle.bf16_to_f32(txt)) and np.array_equal(yi, oracle.bf16_to_f32(img))
    yt, yi = om.mmdit_block(txt, img, _small_weights(rng, D, F), 0.5, cos, sin)
    dt, di = yt - oracle.bf16_to_f32(txt), yi - oracle.bf16_to_f32(img)
    assert 1e-2 < np.abs(dt).mean() < 2 and 1e-2 < np.abs(di).mean() < 2


def chunk_weights(rng, D, F, chunks, std=0.05, zero_out=False, zero_down=False):
    """Weights whose modulation chunks are exactly the given values at t = 0: the sinusoid is 1 (cos) on its first
    128 entries, t1 row 0 sums those to 64 (bf16: 128 * 0.5), silu(64) = 64 in fp32 (exp(-64) vanishes next to 1),
    t2 passes it on to entry 0 of the time vector, silu again 64, and every other entry is silu(0) = 0; so chunk row
    r of a stream is 64 * mod[r, 0], set to value / 64 (exact in bf16 for values of 8 significant bits).
    chunks[s][i]: the value (scalar or [D]) of chunk i of stream s."""
    w = _small_weights(rng, D, F, std=std)
    t1 = np.zeros((D, 256), np.float32)
    t1[0, :128] = 0.5
    t2 = np.zeros((D, D), np.float32)
    t2[0, 0] = 1.0
    w["t1"], w["t2"] = oracle.f32_to_bf16(t1), oracle.f32_to_bf16(t2)
    for s in ("txt", "img"):
        mod = oracle.bf16_to_f32(w[f"{s}.mod"])
        col = np.concatenate([np.broadcast_to(np.asarray(v, np.float32), (D,)) for v in chunks[s]]) / 64.0
        mod[:, 0] = col
        w[f"{s}.mod"] = oracle.f32_to_bf16(mod)
        assert np.array_equal(oracle.bf16_to_f32(w[f"{s}.mod"])[:, 0], col.astype(np.float32))
        if zero_out:
            w[f"{s}.out"] = np.zeros_like(w[f"{s}.out"])
        if zero_down:
            w[f"{s}.mlp_down"] = np.zeros_like(w[f"{s}.mlp_down"])
    return w


def _b(rng, D, lo=-1.0, hi=1.0):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(rng.uniform(lo, hi, D).astype(np.float32)))


MEANING_D, MEANING_F, MEANING_ST, MEANING_GRID = 256, 512, 8, (4, 6)


def meaning_cases(rng):
    """Four pairs of weights on zero inputs, each pair differing in one chunk, with the outcome the chunk meanings
    fix: 'same' (the two blocks return the same bits) or 'zero' (both return zeros), or 'differ'."""
    D, F = MEANING_D, MEANING_F
    g, sh = (lambda: _b(rng, D, 0.25, 1.0)), (lambda: _b(rng, D))
    cases = []
    # attention half live, MLP gated off: the attention scale multiplies LayerNorm(0) = 0, the shift is the input
    base = [sh(), _b(rng, D), g(), sh(), _b(rng, D), 0.0]
    for i, outcome in ((1, "same"), (0, "differ")):
        other = list(base)
        other[i] = _b(rng, D)
        cases.append((f"attention chunk {i}", base, other, {}, outcome))
    # attention gated off (the stream stays 0), MLP live: the same for the MLP's scale and shift
    base = [sh(), _b(rng, D), 0.0, sh(), _b(rng, D), g()]
    for i, outcome in ((4, "same"), (3, "differ")):
        other = list(base)
        other[i] = _b(rng, D)
        cases.append((f"mlp chunk {i}", base, other, {}, outcome))
    # the MLP's down projection zero and the attention gate zero: nothing reaches the stream, whatever the MLP gate
    base = [sh(), _b(rng, D), 0.0, sh(), _b(rng, D), g()]
    other = list(base)
    other[5] = g()
    cases.append(("attention gate 0", base, other, {"zero_down": True}, "zero"))
    # the output projection zero and the MLP gate zero: likewise, whatever the attention gate
    base = [sh(), _b(rng, D), g(), sh(), _b(rng, D), 0.0]
    other = list(base)
    other[2] = g()
    cases.append(("mlp gate 0", base, other, {"zero_out": True}, "zero"))
    return cases


def _meaning_holds(chunk_order):
    from localrouter_amd import rope
    rng = np.random.default_rng(11)
    D, F, St, (gh, gw) = MEANING_D, MEANING_F, MEANING_ST, MEANING_GRID
    cos, sin = rope.grid2d_table(St, gh, gw)
    txt = np.zeros((St, D), np.uint16)
    img = np.zeros((gh * gw, D), np.uint16)
    ok = []
    for name, a, b, extra, outcome in meaning_cases(rng):
        seed = int(rng.integers(1 << 30))
        outs = []
        for chunks in (a, b):
            w = chunk_weights(np.random.default_rng(seed), D, F, {"txt": chunks, "img": chunks}, **extra)
            outs.append(np.concatenate(om.mmdit_block(txt, img, w, 0.0, cos, sin, chunk_order=chunk_order)))
        same = np.array_equal(outs[0], outs[1])
        zero = same and not np.any(outs[0])
        ok.append({"same": same and np.any(outs[0]), "differ": not same, "zero": zero}[outcome])
    return ok


def test_modulation_chunk_meanings():
    """On zero inputs the LayerNorm is 0, so each chunk's meaning fixes an outcome: scales change nothing, shifts do,
    a zero gate shuts its own branch and only that one."""
    assert all(_meaning_holds((0, 1, 2, 3, 4, 5)))


@pytest.mark.parametrize("order,what", [((1, 0, 2, 3, 4, 5), "attention shift <-> scale"),
                                        ((0, 1, 2, 4, 3, 5), "mlp shift <-> scale"),
                                        ((0, 1, 5, 3, 4, 2), "gate_attn <-> gate_mlp")])
def test_planted_chunk_swaps_fail(order, what):
    assert not all(_meaning_holds(order)), what


def test_block_flops_cfg3():
    """512 + 4096 tokens, hidden 3072, MLP 12288."""
    f = om.block_flops(512, 4096, 3072, 12288)
    assert f == pytest.approx(2 * 4608 * 3072 * 36864 + 4 * 4608 ** 2 * 3072 + 2 * (256 * 3072 + 3072 ** 2
                                                                                      + 12 * 3072 ** 2))
