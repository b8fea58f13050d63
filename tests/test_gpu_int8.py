"""GPU parity of the INT8 attention chain (MiniMax H3's quantised attention) against the CPU oracle (oracle/lro_int8.c),
through the C ABI.

  * the prep is bit-exact: anchor row, int8 Q / K / V, every scale, the per-tile column sums;
  * the attention is checked three ways: against the oracle's emulation of the reference's u8 P rounding (tight: the
    only differences are fp32 vs fp64 exponent arithmetic and the bf16 output rounding), against fp64 attention over
    the same quantised operands, and against exact attention of the bf16 inputs at the BASELINE bar (2e-2 / 2e-3);
  * the rows output equals the [H, S, D] output transposed, bit for bit; the one-call entry point equals prep + kernel.
Cases follow the reference's own gate (tools/twin/stk_twin/h3/test_kitchen.py:22-100): packed qkv views, S on both
sides of the H4 / H128 switch (256) and of the 64 / 128 key tile switch (1024), a biased K that makes the anchor fire,
GQA and batches, and H3's shape (5,967 tokens x 56 heads); at head dim 64 (the wheel's other case,
kitchen_launch.cu:196-241: H4 or the plain H64, 64-key tiles, scale 1/8) the gate's 1,797 x 32 x 64 and small cases.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests._util import MAX_ABS, MEAN_ABS, bf16_f32, from_dev, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from localrouter_amd import ops  # noqa: E402


# ------------------------------------------------------------------------------------------ workspace layout, restated
def _k_swz(r, d=128):
    if d == 64:
        return ((r >> 1) & 1) | (((r >> 4) & 1) << 1)
    return ((r >> 2) & 4) | ((((r >> 2) ^ r) & 1) << 1) | ((r >> 1) & 1)


def _v_swz(d, cta):
    return (((d >> 1) & 7) ^ ((d & 1) << 2)) if cta == 128 else (((d >> 1) ^ (d >> 3)) & 3)


def _decode(ws: np.ndarray, B, H, HK, Sq, Sk, d=128) -> dict:
    cta = oracle.i8_cta_for(Sk, d)
    nt = -(-Sk // cta)
    skp, nvc = nt * cta, -(-Sk // 256)
    sizes = [B * H * Sq * d, B * HK * skp * d, B * HK * skp * d, B * HK * nt * 1024, B * H * Sq * 4,
             B * HK * d * 4, B * HK * nvc * d * 4, B * HK * 4, B * HK * d * 2]
    off, at = [], 0
    for s in sizes:
        off.append(at)
        at += -(-s // 256) * 256
    part = lambda i: ws[off[i]:off[i] + sizes[i]]  # noqa: E731
    r = np.arange(skp)
    kst = part(1).view(np.int8).reshape(B, HK, skp, d // 16, 16)
    kidx = np.arange(d // 16)[None, :] ^ np.array([_k_swz(x & 31, d) for x in r])[:, None]
    k8 = np.take_along_axis(kst, kidx[None, None, :, :, None], axis=3).reshape(B, HK, skp, d)
    cpr = cta // 16
    vst = part(2).view(np.int8).reshape(B, HK, nt, d, cpr, 16)
    vidx = np.arange(cpr)[None, :] ^ np.array([_v_swz(c, cta) for c in range(d)])[:, None]
    vt = np.take_along_axis(vst, vidx[None, None, None, :, :, None], axis=4).reshape(B, HK, nt, d, cta)
    v8 = vt.transpose(0, 1, 2, 4, 3).reshape(B, HK, skp, d)
    aux = part(3).reshape(B, HK, nt, 1024)
    db = d // 32
    cs = aux[..., :128 * db].copy().view(np.int16).reshape(B, HK, nt, 2, 32, db)
    cs = cs.transpose(0, 1, 2, 3, 5, 4).reshape(B, HK, nt, 2, d)            # [half][dim]
    nb = cta // 32
    ks = aux[..., 512:512 + 8 * nb].copy().view(np.float32).reshape(B, HK, nt, 2, nb)
    ks = ks.transpose(0, 1, 2, 4, 3).reshape(B, HK, nt * 2 * nb)              # group order 2 kb + half per tile
    return dict(cta=cta, skp=skp, q8=part(0).view(np.int8).reshape(B, H, Sq, d),
                qs=part(4).view(np.float32).reshape(B, H, Sq), k8=k8, ks=ks, v8=v8, cs=cs,
                vs=part(5).view(np.float32).reshape(B, HK, d), anchor=part(7).view(np.int32).reshape(B, HK),
                arow=part(8).view(np.uint16).reshape(B, HK, d))


# ------------------------------------------------------------------------------------------ inputs and the oracle
def _qkv(seed, S, H, bias_heads=(), d=128):
    """Packed qkv bits [S, 3, H, d] ~ N(0, 1); heads in bias_heads get a large common key offset (anchor fires)."""
    qkv = oracle.synth_bf16(seed, 1, (S, 3, H, d))
    if bias_heads:
        f = bf16_f32(qkv)
        off = 3.0 * bf16_f32(oracle.synth_bf16(seed, 2, (1, d)))
        for h in bias_heads:
            f[:, 1, h] += off[0]
        qkv = oracle.f32_to_bf16(f)
    return qkv


def _oracle_head(q, k, v, Sk):
    """The oracle's quantised operands of one (query head, kv head) pair: bf16 bits [Sq, d], [Sk, d], [Sk, d]."""
    rot = oracle.i8_rotation_for(Sk, q.shape[-1])
    a = oracle.i8_anchor(k)
    q8, qs = oracle.i8_quant_rows(q, rot)
    k8, ks = oracle.i8_quant_rows(k, rot, a, oracle.I8_KGROUP)
    v8, vs = oracle.i8_quant_v(v)
    arow = np.asarray(k[a], np.uint16) if a >= 0 else np.zeros(k.shape[-1], np.uint16)
    return dict(anchor=a, arow=arow, q8=q8, qs=qs, k8=k8, ks=ks, v8=v8, vs=vs)


def _check_parts(dec, ref, b, h, hk, Sk, what):
    cta = dec["cta"]
    assert dec["anchor"][b, hk] == ref["anchor"], f"{what}: anchor"
    assert np.array_equal(dec["arow"][b, hk], ref["arow"]), f"{what}: anchor row"
    assert np.array_equal(dec["q8"][b, h], ref["q8"]), f"{what}: q8"
    assert np.array_equal(dec["qs"][b, h].view(np.uint32), ref["qs"].view(np.uint32)), f"{what}: q scales"
    assert np.array_equal(dec["k8"][b, hk, :Sk], ref["k8"]), f"{what}: k8"
    # padding rows repeat real keys: row r > Sk - 1 holds key min(16 gL + r % 16, Sk - 1), gL = (Sk - 1) // 16, so
    # that its score equals a real score; groups past gL carry gL's scale
    last, gl = Sk - 1, (Sk - 1) // 16
    src = [min(gl * 16 + r % 16, last) for r in range(Sk, dec["skp"])]
    assert np.array_equal(dec["k8"][b, hk, Sk:], ref["k8"][src]), f"{what}: k8 padding"
    ng = len(ref["ks"])
    assert np.array_equal(dec["ks"][b, hk, :ng].view(np.uint32), ref["ks"].view(np.uint32)), f"{what}: k scales"
    assert np.all(dec["ks"][b, hk, ng:] == ref["ks"][gl]), f"{what}: padded k scales"
    assert np.array_equal(dec["v8"][b, hk, :Sk], ref["v8"]), f"{what}: v8"
    assert not dec["v8"][b, hk, Sk:].any(), f"{what}: v8 padding"
    assert np.array_equal(dec["vs"][b, hk].view(np.uint32), ref["vs"].view(np.uint32)), f"{what}: v scales"
    d = ref["v8"].shape[1]
    v8p = np.zeros((dec["skp"], d), np.int64)
    v8p[:Sk] = ref["v8"]
    halves = v8p.reshape(-1, 2, cta // 2, d).sum(2)
    assert np.array_equal(dec["cs"][b, hk].astype(np.int64), halves), f"{what}: column sums"


def _check_out(got_bits, ref, rows, what):
    """got: bf16 [Sq_sel, d] of one head; ref: the oracle's quantised operands of that head."""
    got = bf16_f32(got_bits).astype(np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite"
    args = (ref["q8"][rows], ref["qs"][rows], ref["k8"], ref["ks"], ref["v8"], ref["vs"])
    emu = oracle.i8_attention_p8(*args, oracle.i8_cta_for(len(ref["k8"]), ref["q8"].shape[1])).astype(np.float64)
    # the emulation differs only by fp32 exponent arithmetic (a u8 step flips now and then: <= 2 * max|v| / rowsum)
    # and the bf16 output rounding (<= 2^-9 relative)
    d = np.abs(got - emu)
    bound = 2.0 ** -8 * np.abs(emu) + 2e-3
    assert np.all(d <= bound), f"{what}: vs u8-P emulation max {d.max():.3e} at {np.unravel_index(d.argmax(), d.shape)}"
    # bf16 rounding alone is <= 2^-9 |x| per element, so its mean is <= 2^-9 mean|x|; flips add little on average
    assert d.mean() <= 2.0 ** -9 * np.abs(emu).mean() + 5e-5, f"{what}: vs u8-P emulation mean {d.mean():.3e}"
    exact_q = oracle.i8_attention(*args).astype(np.float64)
    d2 = np.abs(got - exact_q)
    assert d2.max() <= MAX_ABS and d2.mean() <= MEAN_ABS, f"{what}: vs fp64 quantised {d2.max():.3e} {d2.mean():.3e}"
    return d.max(), d.mean(), d2.max(), d2.mean()


CASES = [(80, 2, ()), (256, 2, (1,)), (300, 2, (0,)), (1024, 2, ()), (1100, 3, (2,)), (777, 1, (0,))]


@pytest.mark.parametrize("S,H,bias", CASES)
def test_int8_packed_qkv(S, H, bias):
    """Kitchen.attention on a packed qkv buffer: prep bit-exact, attention within the bars, rows == transpose."""
    print(f"\n[int8 qkv] S={S} H={H} bias={bias}", flush=True)
    qkv = _qkv(21, S, H, bias)
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    ws = ops.kitchen_attention_prep(dq, None, H)
    out = ops.kitchen_attention_kernel(torch.empty((H, S, 128), dtype=torch.bfloat16, device="cuda"), ws, H, S, False)
    rows = ops.kitchen_attention_kernel(torch.empty((S, H * 128), dtype=torch.bfloat16, device="cuda"), ws, H, S, True)
    one = ops.kitchen_attention(dq, H)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S)
    got, got_rows, got_one = from_dev(out), from_dev(rows), from_dev(one)
    assert np.array_equal(got_rows.reshape(S, H, 128).transpose(1, 0, 2), got), "rows != [H, S, D] transposed"
    assert np.array_equal(got_one, got), "one call != prep + kernel"
    qf = bf16_f32(qkv)
    for h in range(H):
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        if h in bias:
            assert ref["anchor"] >= 0, "the biased head must use its anchor"
        _check_parts(dec, ref, 0, h, h, S, f"S={S} h={h}")
        stats = _check_out(got[h], ref, np.arange(S), f"S={S} h={h}")
        exact = oracle.brute_attention(qf[:, 0, h][:, None], qf[:, 1, h][:, None], qf[:, 2, h][:, None])[:, 0]
        d = np.abs(bf16_f32(got[h]).astype(np.float64) - exact)
        print(f"  h={h} anchor={ref['anchor']} emu {stats[0]:.2e}/{stats[1]:.2e} fp64q {stats[2]:.2e}/{stats[3]:.2e} "
              f"exact {d.max():.2e}/{d.mean():.2e}", flush=True)
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, f"S={S} h={h}: vs exact {d.max():.3e} {d.mean():.3e}"


def test_int8_prep_nonfinite_values():
    """NaN and infinities in q, k and v: the quantisers' NaN -> 0 and saturation (float_utils.cuh:40-51; the
    kernels convert through v_cvt_i32_f32, which maps NaN to 0 and saturates), the abs-max that skips NaN (fmaxf),
    and the infinite scales: the prep still bit-exact against the oracle. The planted rows are not anchor samples."""
    S, H = 300, 2
    print(f"\n[int8 non-finite] S={S} H={H}", flush=True)
    qkv = _qkv(61, S, H)
    nan, pinf, ninf = np.uint16(0x7FC0), np.uint16(0x7F80), np.uint16(0xFF80)
    qkv[5, 0, 0, 3] = nan         # a query row that becomes NaN throughout (the rotation mixes it): all zeros
    qkv[50, 0, 1, 77] = pinf      # a query row of infinities: scale inf, every value 0 or saturated
    qkv[120, 1, 0, 10] = ninf     # a key scale group with an infinite scale
    qkv[6, 1, 1, 0] = nan         # a key row of NaN inside a finite group
    qkv[77, 2, 0, 5] = nan        # one NaN value of V (skipped by the channel abs-max, quantised to 0)
    qkv[200, 2, 1, 100] = ninf    # an infinite V channel scale
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    ws = ops.kitchen_attention_prep(dq, None, H)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S)
    for h in range(H):
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        _check_parts(dec, ref, 0, h, h, S, f"non-finite h={h}")
    assert not dec["q8"][0, 0, 5].any(), "a NaN query row quantises to zeros"
    assert np.isinf(dec["vs"][0, 1, 100]), "an infinite V value makes its channel scale infinite"


def test_int8_anchor_closed_forms():
    """The prep's anchor on keys whose outcome the criterion fixes in closed form (tests/test_oracle_int8.py
    _anchor_cases): accepted at sample 3's row, declined on energy, declined on the 12.5 % abs-max cap; the other
    prep parts bit-exact against the oracle."""
    from tests.test_oracle_int8 import _anchor_cases
    cases = _anchor_cases()
    S, H = 101, len(cases)
    print(f"\n[int8 anchor closed forms] S={S} H={H}", flush=True)
    qkv = bf16_f32(_qkv(31, S, H))
    for h, (name, (k, want)) in enumerate(cases.items()):
        qkv[:, 1, h] = k
    qkv = oracle.f32_to_bf16(qkv)
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    ws = ops.kitchen_attention_prep(dq, None, H)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S)
    for h, (name, (k, want)) in enumerate(cases.items()):
        assert dec["anchor"][0, h] == want, f"{name}: anchor {dec['anchor'][0, h]}, closed form {want}"
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        _check_parts(dec, ref, 0, h, h, S, f"anchor case {name}")


@pytest.mark.parametrize("B,H,HK,Sq,Sk", [(2, 4, 2, 200, 333), (1, 3, 1, 513, 1500), (2, 2, 2, 1, 70)])
def test_int8_gqa_batch_cross(B, H, HK, Sq, Sk):
    """Separate q [B,H,Sq,D] and k, v [B,HK,Sk,D] tensors: GQA (query head h reads kv head h // (H / HK)), batches,
    Sq != Sk, a single query."""
    print(f"\n[int8 gqa] B={B} H={H} HK={HK} Sq={Sq} Sk={Sk}", flush=True)
    q = oracle.synth_bf16(22, 1, (B, H, Sq, 128))
    k = oracle.synth_bf16(22, 2, (B, HK, Sk, 128))
    v = oracle.synth_bf16(22, 3, (B, HK, Sk, 128))
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    ws = ops.int8_attention_prep(dq, dk, dv)
    out = ops.int8_attention_kernel(ws, torch.empty((B, H, Sq, 128), dtype=torch.bfloat16, device="cuda"), batch=B,
                                    heads=H, kv_heads=HK, sq=Sq, sk=Sk)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), B, H, HK, Sq, Sk)
    got = from_dev(out)
    G = H // HK
    for b in range(B):
        for h in range(H):
            hk = h // G
            ref = _oracle_head(q[b, h], k[b, hk], v[b, hk], Sk)
            _check_parts(dec, ref, b, h, hk, Sk, f"b={b} h={h}")
            _check_out(got[b, h], ref, np.arange(Sq), f"b={b} h={h}")


@pytest.mark.parametrize("B,H,HK,Sq,Sk,d", [(1, 4, 2, 2100, 2100, 128), (2, 3, 3, 600, 2200, 128),
                                             (1, 4, 4, 2100, 2100, 64)])
def test_int8_split_last_round(B, H, HK, Sq, Sk, d):
    """Query blocks that fill at most half a round of the compute units, over at least 16 key tiles: the kernel cuts
    each block into key ranges (starting on 4-tile boundaries; the last range holds the partial last tile and its P
    mask), and a second launch merges the ranges' rows. Every row of every head against the u8-P emulation and the
    fp64 attention over the quantised operands; the rows output equals the head-major one bit for bit, and a second
    call over the same workspace gives the same bits."""
    print(f"\n[int8 split] B={B} H={H} HK={HK} Sq={Sq} Sk={Sk} d={d}", flush=True)
    q = oracle.synth_bf16(24, 1, (B, H, Sq, d))
    k = oracle.synth_bf16(24, 2, (B, HK, Sk, d))
    v = oracle.synth_bf16(24, 3, (B, HK, Sk, d))
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    ws = ops.int8_attention_prep(dq, dk, dv)
    kw = dict(batch=B, heads=H, kv_heads=HK, sq=Sq, sk=Sk, head_dim=d)
    out = ops.int8_attention_kernel(ws, torch.empty((B, H, Sq, d), dtype=torch.bfloat16, device="cuda"), **kw)
    again = ops.int8_attention_kernel(ws, torch.empty((B, H, Sq, d), dtype=torch.bfloat16, device="cuda"), **kw)
    got = from_dev(out)
    assert np.array_equal(from_dev(again), got), "second call over the same workspace"
    if B == 1:
        rows = ops.int8_attention_kernel(ws, torch.empty((Sq, H * d), dtype=torch.bfloat16, device="cuda"), rows=True,
                                         **kw)
        assert np.array_equal(from_dev(rows).reshape(Sq, H, d).transpose(1, 0, 2), got[0]), "rows != head-major"
    G = H // HK
    for b in range(B):
        for h in range(H):
            ref = _oracle_head(q[b, h], k[b, h // G], v[b, h // G], Sk)
            st = _check_out(got[b, h], ref, np.arange(Sq), f"b={b} h={h}")
            print(f"  b={b} h={h} emu {st[0]:.2e}/{st[1]:.2e} fp64q {st[2]:.2e}/{st[3]:.2e}", flush=True)


def test_int8_degenerate_inputs():
    """Zero query rows (uniform attention), identical keys (the anchor removes everything: all scores 0), constant V
    channels, on a tail tile: the masked keys past Sk must not enter the row sums."""
    S, H = 333, 2
    print(f"\n[int8 degenerate] S={S}", flush=True)
    qkv = bf16_f32(_qkv(23, S, H))
    qkv[::7, 0, 0] = 0.0                       # zero query rows
    qkv[:, 1, 1] = qkv[0, 1, 1][None]          # one key repeated
    qkv[:, 2, 0, :4] = 1.5                     # constant value channels
    qkv = oracle.f32_to_bf16(qkv)
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    out = ops.kitchen_attention(dq, H)
    torch.cuda.synchronize()
    got = from_dev(out)
    qf = bf16_f32(qkv)
    for h in range(H):
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        _check_out(got[h], ref, np.arange(S), f"h={h}")
        exact = oracle.brute_attention(qf[:, 0, h][:, None], qf[:, 1, h][:, None], qf[:, 2, h][:, None])[:, 0]
        d = np.abs(bf16_f32(got[h]).astype(np.float64) - exact)
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, f"h={h}: vs exact {d.max():.3e} {d.mean():.3e}"
    # uniform attention of a zero query row over a repeated-key head: the mean of V exactly as the oracle has it
    assert np.all(np.isfinite(bf16_f32(got)))


def test_int8_h3_shape():
    """H3's attention: 5,967 tokens x 56 heads from one packed qkv buffer, the [H, S, D] and rows outputs. The oracle
    checks two heads (every prep part, 96 query rows each, first, last and a spread between)."""
    S, H = 5967, 56
    print(f"\n[int8 h3] S={S} H={H}", flush=True)
    qkv = _qkv(24, S, H, bias_heads=(55,))
    dq = to_dev(qkv.reshape(S, 3 * H * 128))
    ws = torch.empty(ops.int8_workspace_bytes(H, S), dtype=torch.uint8, device="cuda")
    out = ops.kitchen_attention(dq, H, workspace=ws)
    rows = ops.kitchen_attention(dq, H, workspace=ws, rows=True)
    torch.cuda.synchronize()
    got = from_dev(out)
    assert np.array_equal(from_dev(rows).reshape(S, H, 128).transpose(1, 0, 2), got)
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S)
    sel = np.unique(np.concatenate([np.arange(32), np.linspace(32, S - 33, 32).astype(int), np.arange(S - 32, S)]))
    for h in (0, 55):
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        if h == 55:
            assert ref["anchor"] >= 0
        _check_parts(dec, ref, 0, h, h, S, f"h={h}")
        stats = _check_out(got[h][sel], ref, sel, f"h={h}")
        print(f"  h={h} emu {stats[0]:.2e}/{stats[1]:.2e} fp64q {stats[2]:.2e}/{stats[3]:.2e}", flush=True)


def _exact_bar_d64(ref, rows, exact):
    """Against exact attention at head dim 64: BASELINE's bar, or 1.25x the error the reference's algorithm itself
    makes (fp64 attention over the oracle's quantised operands) where that is larger: 64 channels and few keys leave
    more quantisation error than the bar allows."""
    args = (ref["q8"][rows], ref["qs"][rows], ref["k8"], ref["ks"], ref["v8"], ref["vs"])
    e = np.abs(oracle.i8_attention(*args).astype(np.float64) - exact)
    return max(MAX_ABS, 1.25 * e.max()), max(MEAN_ABS, 1.25 * e.mean())


@pytest.mark.parametrize("S,H,bias", [(80, 2, ()), (300, 2, (1,)), (1100, 2, (0,))])
def test_int8_head_dim_64(S, H, bias):
    """Head dim 64: H4 up to 256 keys, else the plain H64; 64-key tiles at every length; scale 1/8. Prep bit-exact,
    attention within the bars, against exact attention too; rows == transpose; one call == prep + kernel."""
    print(f"\n[int8 d64] S={S} H={H} bias={bias}", flush=True)
    qkv = _qkv(25, S, H, bias, d=64)
    dq = to_dev(qkv.reshape(S, 3 * H * 64))
    ws = ops.kitchen_attention_prep(dq, None, H, head_dim=64)
    out = ops.kitchen_attention_kernel(torch.empty((H, S, 64), dtype=torch.bfloat16, device="cuda"), ws, H, S, False,
                                       head_dim=64)
    rows = ops.kitchen_attention_kernel(torch.empty((S, H * 64), dtype=torch.bfloat16, device="cuda"), ws, H, S, True,
                                        head_dim=64)
    one = ops.kitchen_attention(dq, H, head_dim=64)
    torch.cuda.synchronize()
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S, d=64)
    got, got_rows, got_one = from_dev(out), from_dev(rows), from_dev(one)
    assert np.array_equal(got_rows.reshape(S, H, 64).transpose(1, 0, 2), got), "rows != [H, S, D] transposed"
    assert np.array_equal(got_one, got), "one call != prep + kernel"
    qf = bf16_f32(qkv)
    for h in range(H):
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        if h in bias:
            assert ref["anchor"] >= 0, "the biased head must use its anchor"
        _check_parts(dec, ref, 0, h, h, S, f"d64 S={S} h={h}")
        stats = _check_out(got[h], ref, np.arange(S), f"d64 S={S} h={h}")
        exact = oracle.brute_attention(qf[:, 0, h][:, None], qf[:, 1, h][:, None], qf[:, 2, h][:, None], scale=0.125)[:, 0]
        d = np.abs(bf16_f32(got[h]).astype(np.float64) - exact)
        bar = _exact_bar_d64(ref, np.arange(S), exact)
        print(f"  h={h} anchor={ref['anchor']} emu {stats[0]:.2e}/{stats[1]:.2e} fp64q {stats[2]:.2e}/{stats[3]:.2e} "
              f"exact {d.max():.2e}/{d.mean():.2e} (bar {bar[0]:.2e}/{bar[1]:.2e})", flush=True)
        assert d.max() <= bar[0] and d.mean() <= bar[1], f"d64 S={S} h={h}: vs exact {d.max():.3e} {d.mean():.3e}"


def test_int8_head_dim_64_gate_shape():
    """The reference gate's head-dim-64 case (tools/twin/stk_twin/h3/test_kitchen.py:22): 1,797 tokens x 32 heads x 64
    from one packed qkv buffer, rows output. The oracle checks three heads (every prep part, 96 query rows each)."""
    S, H = 1797, 32
    print(f"\n[int8 d64 gate] S={S} H={H}", flush=True)
    qkv = _qkv(26, S, H, bias_heads=(31,), d=64)
    dq = to_dev(qkv.reshape(S, 3 * H * 64))
    ws = torch.empty(ops.int8_workspace_bytes(H, S, head_dim=64), dtype=torch.uint8, device="cuda")
    rows = ops.kitchen_attention(dq, H, workspace=ws, rows=True, head_dim=64)
    torch.cuda.synchronize()
    got = from_dev(rows).reshape(S, H, 64).transpose(1, 0, 2)
    dec = _decode(ws.cpu().numpy(), 1, H, H, S, S, d=64)
    sel = np.unique(np.concatenate([np.arange(32), np.linspace(32, S - 33, 32).astype(int), np.arange(S - 32, S)]))
    qf = bf16_f32(qkv)
    for h in (0, 17, 31):
        ref = _oracle_head(*(np.ascontiguousarray(qkv[:, i, h]) for i in range(3)), S)
        if h == 31:
            assert ref["anchor"] >= 0
        _check_parts(dec, ref, 0, h, h, S, f"d64 gate h={h}")
        stats = _check_out(got[h][sel], ref, sel, f"d64 gate h={h}")
        exact = oracle.brute_attention(qf[sel, 0, h][:, None], qf[:, 1, h][:, None], qf[:, 2, h][:, None], scale=0.125)[:, 0]
        d = np.abs(bf16_f32(got[h][sel]).astype(np.float64) - exact)
        bar = _exact_bar_d64(ref, sel, exact)
        print(f"  h={h} emu {stats[0]:.2e}/{stats[1]:.2e} fp64q {stats[2]:.2e}/{stats[3]:.2e} "
              f"exact {d.max():.2e}/{d.mean():.2e} (bar {bar[0]:.2e}/{bar[1]:.2e})", flush=True)
        assert d.max() <= bar[0] and d.mean() <= bar[1], f"d64 gate h={h}: vs exact {d.max():.3e} {d.mean():.3e}"
    assert np.all(np.isfinite(bf16_f32(got)))
