"""Pins of the INT8-chain oracle (oracle/lro_int8.c), on the CPU only.

Each part is checked against something it does not share code with:
  * the rotations: the signed H128 equals the closed form (-1)^popcount(i & j) / sqrt(128) times the reference's sign
    vector (the constants of kernels/cuda/minimax/kitchen/quant_qk_int8.cu:93-97), H4 is block-diagonal with the
    4-point Sylvester Hadamard, both are orthogonal and leave dot products of rotated pairs unchanged;
  * the K anchor: three key sets whose outcome the criterion of quant_qk_int8.cu:461-596 fixes in closed form
    (accepted at a known sample, declined on energy, declined on the abs-max cap), with planted slips in the rule
    failing them, and an independent numpy restatement on random heads where both outcomes occur;
  * the quantisers: scale = absmax / 127 + 1e-7 (Q, K) and absmax / 127 per channel (V), the largest magnitude maps to
    +-127, every element within half a step, ties to even;
  * the attention over quantised operands: an independent numpy fp64 softmax over the dequantised operands, and the
    whole chain against exact attention of the unquantised inputs within the quantisation error.
"""
from __future__ import annotations

import numpy as np

import oracle

SCALE = float(np.frombuffer(np.uint32(0x3DB504F3).tobytes(), np.float32)[0])
SIGNS = [0x1035997B, 0x8087F5EE, 0xEE2E4E1A, 0x71132418]


def _sign_vector():
    out = np.ones(128)
    for j in range(128):
        lane, c = j // 4, j % 4
        flip = ((SIGNS[lane >> 3] >> ((lane & 7) * 4 + c)) & 1) ^ 1
        out[j] = -1.0 if flip else 1.0
    return out


def _rotation_matrix(kind, d=128):
    # row i of the result is the rotation of basis vector e_i, so its transpose maps inputs to outputs
    return oracle.i8_rotate(np.eye(d, dtype=np.float32), kind).T.astype(np.float64)


def test_signed_h128_closed_form():
    M = _rotation_matrix(128)
    pc = np.array([[bin(i & j).count("1") & 1 for j in range(128)] for i in range(128)])
    closed = np.where(pc == 1, -1.0, 1.0) / np.sqrt(128.0) * _sign_vector()[None, :]
    assert np.abs(M - closed).max() < 1e-7
    assert np.abs(M @ M.T - np.eye(128)).max() < 1e-6
    # a wrong sign word would be caught: the sign vector has both signs in every word's lanes
    assert (_sign_vector() < 0).sum() not in (0, 128)


def test_plain_h64_closed_form():
    """Head dim 64 (convrot64, quant_qk_int8.cu:110-129): the Sylvester-Hadamard matrix of order 64, entries
    (-1)^popcount(i & j) / 8, no sign flip; orthogonal."""
    M = _rotation_matrix(64, 64)
    pc = np.array([[bin(i & j).count("1") & 1 for j in range(64)] for i in range(64)])
    assert np.abs(M - np.where(pc == 1, -1.0, 1.0) / 8.0).max() < 1e-7
    assert np.abs(M @ M.T - np.eye(64)).max() < 1e-6


def test_h4_blocks():
    h4 = 0.5 * np.array([[1, 1, 1, 1], [1, -1, 1, -1], [1, 1, -1, -1], [1, -1, -1, 1]], np.float64)
    for d in (128, 64):
        assert np.array_equal(_rotation_matrix(4, d), np.kron(np.eye(d // 4), h4))


def test_rotation_keeps_dot_products():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((5, 128)).astype(np.float32)
    k = rng.standard_normal((7, 128)).astype(np.float32)
    for kind in (4, 128):
        qr, kr = oracle.i8_rotate(q, kind), oracle.i8_rotate(k, kind)
        assert np.allclose(qr @ kr.T, q @ k.T, atol=1e-4)
    q, k = q[:, :64].copy(), k[:, :64].copy()
    for kind in (4, 64):
        qr, kr = oracle.i8_rotate(q, kind), oracle.i8_rotate(k, kind)
        assert np.allclose(qr @ kr.T, q @ k.T, atol=1e-4)


def _anchor_numpy(k):
    """Independent restatement: 9 samples at i (L-1)/8, argmin of ||9 s_j - sum s||^2, accepted when the residual
    energy drops and the residual abs-max grows by at most 12.5 %."""
    L = k.shape[0]
    idx = [i * (L - 1) // 8 for i in range(9)]
    s = k[idx].astype(np.float64)
    dist = ((9 * s - s.sum(0)[None]) ** 2).sum(1)
    best = int(np.argmin(dist))
    r = s - s[best][None]
    ok = (r ** 2).sum() < (s ** 2).sum() and np.abs(r).max() <= np.abs(s).max() * 1.125
    return idx[best] if ok else -1


def test_anchor_against_numpy():
    rng = np.random.default_rng(1)
    seen = set()
    for trial in range(40):
        L = int(rng.integers(9, 400))
        base = rng.standard_normal(128) * (4.0 if trial % 2 else 0.0)
        k = base[None] + rng.standard_normal((L, 128)) * (0.3 if trial % 2 else 1.0)
        bits = oracle.f32_to_bf16(k.astype(np.float32))
        got = oracle.i8_anchor(bits)
        assert got == _anchor_numpy(oracle.bf16_to_f32(bits)), trial
        seen.add(got >= 0)
    assert seen == {True, False}, "both outcomes must occur"


def _anchor_cases(L=101, d=128):
    """Keys whose anchor outcome the criterion fixes in closed form (all values exact in bf16). The 9 samples are rows
    i (L-1) // 8; the other rows are noise that the rule never reads.
      accept: samples = c + delta_j, delta in +- pairs and one zero at sample 3, c large: sample 3 is exactly the mean
              (distance 0), the residuals are the deltas (energy drops, abs-max shrinks) -> row 3 (L-1) // 8;
      energy: the same deltas with c = 0: subtracting the zero sample changes nothing (energy equal) -> -1;
      absmax: delta = +8A at sample 0, -A at the other 8 (sum 0), c0 = -4A: the energy drops (216 A^2 -> 81 A^2) but
              the abs-max grows from 5A to 9A (> 12.5 %) -> -1."""
    rng = np.random.default_rng(7)
    idx = [i * (L - 1) // 8 for i in range(9)]
    v = [np.zeros(d) for _ in range(4)]
    for m in range(4):
        v[m][8 * m:8 * m + 8] = 2.0 ** (m - 2)
    deltas = [v[0], -v[0], v[1], np.zeros(d), -v[1], v[2], -v[2], v[3], -v[3]]
    cases = {}
    for name, c in (("accept", np.full(d, 6.0)), ("energy", np.zeros(d))):
        k = rng.standard_normal((L, d)).round(2)
        for j, i in enumerate(idx):
            k[i] = c + deltas[j]
        cases[name] = (k, idx[3] if name == "accept" else -1)
    A = 0.5
    k = rng.standard_normal((L, d)).round(2)
    for j, i in enumerate(idx):
        k[i] = 0.0
        k[i][0] = -4 * A + (8 * A if j == 0 else -A)
    cases["absmax"] = (k, -1)
    return cases


def test_anchor_closed_forms():
    for name, (k, want) in _anchor_cases().items():
        bits = oracle.f32_to_bf16(k.astype(np.float32))
        assert np.array_equal(oracle.bf16_to_f32(bits)[[i * 100 // 8 for i in range(9)]],
                              k[[i * 100 // 8 for i in range(9)]].astype(np.float32)), "samples exact in bf16"
        assert oracle.i8_anchor(bits) == want, name
        assert _anchor_numpy(oracle.bf16_to_f32(bits)) == want, name


def test_anchor_planted_mistakes_fail():
    """Each plausible slip in the criterion changes the outcome of one closed-form case."""
    def variant(k, no_cap=False, bad_index=False, le_energy=False):
        L = k.shape[0]
        idx = [i * L // 9 for i in range(9)] if bad_index else [i * (L - 1) // 8 for i in range(9)]
        s = k[idx].astype(np.float64)
        best = int(np.argmin(((9 * s - s.sum(0)[None]) ** 2).sum(1)))
        r = s - s[best][None]
        e_ok = (r ** 2).sum() <= (s ** 2).sum() if le_energy else (r ** 2).sum() < (s ** 2).sum()
        m_ok = True if no_cap else np.abs(r).max() <= np.abs(s).max() * 1.125
        return idx[best] if e_ok and m_ok else -1
    cases = {n: (oracle.bf16_to_f32(oracle.f32_to_bf16(k.astype(np.float32))), w) for n, (k, w) in _anchor_cases().items()}
    assert all(variant(k) == w for k, w in cases.values())
    for slip in ({"no_cap": True}, {"bad_index": True}, {"le_energy": True}):
        assert any(variant(k, **slip) != w for k, w in cases.values()), slip


def test_quantisers():
    rng = np.random.default_rng(2)
    x = oracle.f32_to_bf16((rng.standard_normal((70, 128)) * 3).astype(np.float32))
    xf = oracle.bf16_to_f32(x)
    for rot, group in ((128, 1), (4, 16), (0, 16)):
        q8, sc = oracle.i8_quant_rows(x, rot, -1, group)
        xr = oracle.i8_rotate(xf, rot) if rot else xf
        for g in range(len(sc)):
            blk = xr[g * group:(g + 1) * group]
            assert sc[g] == np.float32(np.float32(np.abs(blk).max()) / np.float32(127.0) + np.float32(1e-7))
            qb = q8[g * group:(g + 1) * group].astype(np.float64)
            assert np.abs(qb * sc[g] - blk).max() <= 0.5 * sc[g] * (1 + 1e-5)
            assert np.abs(qb).max() == 127
    v8, vs = oracle.i8_quant_v(x)
    assert np.allclose(vs, np.abs(xf).max(0) / 127.0, rtol=1e-6)
    assert np.all(np.abs(v8.astype(np.float64) * vs[None] - xf) <= 0.5 * vs[None] * (1 + 1e-5))


def test_attention_over_quantised_operands():
    rng = np.random.default_rng(3)
    W, nk = 20, 77
    q8 = rng.integers(-127, 128, (W, 128)).astype(np.int8)
    k8 = rng.integers(-127, 128, (nk, 128)).astype(np.int8)
    v8 = rng.integers(-127, 128, (nk, 128)).astype(np.int8)
    qs = rng.uniform(0.005, 0.02, W).astype(np.float32)
    ks = rng.uniform(0.005, 0.02, (nk + 15) // 16).astype(np.float32)
    vs = rng.uniform(0.005, 0.02, 128).astype(np.float32)
    got = oracle.i8_attention(q8, qs, k8, ks, v8, vs)
    kd = k8.astype(np.float64) * np.repeat(ks.astype(np.float64), 16)[:nk, None]
    s = (q8.astype(np.float64) * qs[:, None]) @ kd.T * SCALE
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    ref = p @ (v8.astype(np.float64) * vs[None])
    assert np.abs(got - ref).max() < 1e-6


def test_chain_close_to_exact_attention():
    """Quantisation error only: the chain against fp64 attention of the bf16 inputs, both with the anchor and without
    (an anchor shifts every score of a query equally, which softmax ignores)."""
    S, H = 300, 2
    qkv = oracle.synth_bf16(7, 1, (S, 3, H, 128))
    # give head 1 a large common key offset so that its anchor is used
    f = oracle.bf16_to_f32(qkv)
    f[:, 1, 1] += 3.0 * oracle.bf16_to_f32(oracle.synth_bf16(7, 2, (1, 128)))
    qkv = oracle.f32_to_bf16(f)
    out, parts = oracle.int8_attention(qkv, H)
    assert parts["anchor"][1] >= 0
    qf = oracle.bf16_to_f32(qkv)
    for h in range(H):
        exact = oracle.brute_attention(qf[:, 0, h][:, None], qf[:, 1, h][:, None], qf[:, 2, h][:, None])[:, 0]
        d = np.abs(out[h] - exact)
        assert d.max() < 2e-2 and d.mean() < 2e-3, (h, d.max(), d.mean())


def _p8_numpy(q8, qs, k8, ks, v8, vs, cta):
    """Independent restatement of the u8 P rounding: per row and per cta-key tile, P = round(255 * exp(s - max_tile s))
    (the kernel's exp2(x - max + 7.9943534) with the offset's fp32 value), the row sum over the rounded P, tiles
    combined with weights exp(max_tile - max_row)."""
    nk = k8.shape[0]
    kd = k8.astype(np.float64) * np.repeat(ks.astype(np.float64), 16)[:nk, None]
    x = (q8.astype(np.float64) * qs[:, None]) @ kd.T * SCALE * np.log2(np.e)
    off = float(np.float32(7.9943534))
    num = np.zeros((q8.shape[0], 128))
    den = np.zeros((q8.shape[0], 1))
    tiles = [(t, min(t + cta, nk)) for t in range(0, nk, cta)]
    mt = np.stack([x[:, a:b].max(1) - off for a, b in tiles], 1)
    M = mt.max(1, keepdims=True)
    for i, (a, b) in enumerate(tiles):
        p = np.clip(np.rint(np.exp2(x[:, a:b] - mt[:, i:i + 1])), 0, 255)
        w = np.exp2(mt[:, i:i + 1] - M)
        num += w * (p @ v8[a:b].astype(np.float64))
        den += w * p.sum(1, keepdims=True)
    return num / den * vs[None].astype(np.float64)


# P of a key whose score sits k log2 steps below its tile's maximum: the nearest integer to 2^(7.9943534 - k) =
# 254.99997 / 2^k (the offset's fp32 value), i.e. to 255 / 2^k; k = 1 (127.49998) is left out as a near-tie
P8_AT_STEP = {0: 255, 2: 64, 3: 32, 4: 16, 5: 8, 6: 4, 7: 2, 8: 1, 9: 0, 10: 0}


def test_p8_closed_form_at_log2_steps():
    """Scores at exact log2 steps (qs = 1 / (scale log2 e) in fp32, key scales 1, q a unit vector, so x_j = -k_j to
    1e-7): every P is known in closed form, every tile's weight is 2^-(its maximum's step), and the output is the
    P-weighted mean of V. Three tiles of 64 keys (the last one partial) with maxima at steps 0, 3 and 2; row 1 doubles
    the steps of another column."""
    qs1 = np.float32(1.0 / (SCALE * np.log2(np.e)))
    nk, cta = 170, 64
    rng = np.random.default_rng(12)
    tiles = [(0, 64, 0), (64, 128, 3), (128, 170, 2)]
    steps0 = np.zeros(nk, np.int64)
    for a, b, lo in tiles:
        rel = rng.choice(list(P8_AT_STEP), b - a)
        rel[0] = 0
        steps0[a:b] = lo + rel
    steps1 = rng.integers(0, 6, nk)
    for a, b, _ in tiles:
        steps1[a] = 0
    q8 = np.zeros((2, 128), np.int8)
    q8[0, 0], q8[1, 1] = 1, 2
    k8 = rng.integers(-127, 128, (nk, 128)).astype(np.int8)
    k8[:, 0], k8[:, 1] = -steps0, -steps1
    v8 = rng.integers(-127, 128, (nk, 128)).astype(np.int8)
    vs = rng.uniform(0.005, 0.02, 128).astype(np.float32)
    got = oracle.i8_attention_p8(q8, np.full(2, qs1), k8, np.ones((nk + 15) // 16, np.float32), v8, vs, cta)
    for row, steps, mult in ((0, steps0, 1), (1, steps1, 2)):
        num, den = np.zeros(128), 0.0
        for a, b, _ in tiles:
            x = mult * steps[a:b]
            top = x.min()
            p = np.array([P8_AT_STEP[int(k)] for k in x - top], np.float64)
            num += 2.0 ** -top * (p @ v8[a:b].astype(np.float64))
            den += 2.0 ** -top * p.sum()
        exp = num / den * vs
        assert np.abs(got[row] - exp).max() <= 1e-6 * np.abs(exp).max(), row
    # the closed form is not the exact softmax: the rounding shows
    assert np.abs(got - oracle.i8_attention(q8, np.full(2, qs1), k8, np.ones((nk + 15) // 16, np.float32), v8,
                                            vs)).max() > 1e-4


def test_p8_rounding_against_numpy():
    rng = np.random.default_rng(4)
    for W, nk, cta in ((7, 200, 64), (5, 300, 128), (3, 64, 64), (4, 65, 64)):
        q8 = rng.integers(-127, 128, (W, 128)).astype(np.int8)
        k8 = rng.integers(-127, 128, (nk, 128)).astype(np.int8)
        v8 = rng.integers(-127, 128, (nk, 128)).astype(np.int8)
        qs = rng.uniform(0.01, 0.05, W).astype(np.float32)
        ks = rng.uniform(0.01, 0.05, (nk + 15) // 16).astype(np.float32)
        vs = rng.uniform(0.005, 0.02, 128).astype(np.float32)
        got = oracle.i8_attention_p8(q8, qs, k8, ks, v8, vs, cta)
        ref = _p8_numpy(q8, qs, k8, ks, v8, vs, cta)
        assert np.abs(got - ref).max() < 1e-6, (W, nk, cta)
        # the rounding is a perturbation of the exact softmax: within a few u8 steps of it, not equal to it
        exact = oracle.i8_attention(q8, qs, k8, ks, v8, vs)
        d = np.abs(got - exact)
        assert 0 < d.max() < 4 * 127 * vs.max() / 255, (W, nk, cta, d.max())
    assert oracle.i8_cta_for(1024) == 64 and oracle.i8_cta_for(1025) == 128


def test_chain_head_dim_64_close_to_exact_attention():
    """Head dim 64 at scale 1/8: the chain (H64 or H4, anchor, per-row / per-16-key / per-channel scales, cta 64)
    within BASELINE's bar of fp64 attention of the bf16 inputs; P rounded per 64-key tile within a few u8 steps."""
    rng = np.random.default_rng(21)
    for S, H in ((300, 3), (200, 2)):
        x = (rng.standard_normal((S, 3, H, 64)) * np.array([1.0, 1.0, 1.0])[None, :, None, None]).astype(np.float32)
        qkv = oracle.f32_to_bf16(x)
        out, parts = oracle.int8_attention(qkv, H)
        assert out.shape == (H, S, 64) and oracle.i8_rotation_for(S, 64) == (4 if S <= 256 else 64)
        xf = oracle.bf16_to_f32(qkv).astype(np.float64)
        for h in range(H):
            s = xf[:, 0, h] @ xf[:, 1, h].T / 8.0
            p = np.exp(s - s.max(1, keepdims=True))
            exact = (p / p.sum(1, keepdims=True)) @ xf[:, 2, h]
            d = np.abs(out[h] - exact)
            assert d.max() < 2e-2 and d.mean() < 2e-3, (S, h, d.max(), d.mean())
            args = [parts[n][h] for n in ("q8", "qs", "k8", "ks", "v8", "vs")]
            p8 = oracle.i8_attention_p8(*args, oracle.i8_cta_for(S, 64))
            assert np.abs(p8 - out[h]).max() < 4 * 127 * parts["vs"][h].max() / 255
    assert oracle.i8_cta_for(5000, 64) == 64 and oracle.i8_scale(64) == 0.125

