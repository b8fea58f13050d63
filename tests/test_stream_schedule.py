"""The streaming kernel's work partition, restated on the host and checked exhaustively over many shapes.

localrouter_amd/csrc/attn_stream.hip computes, per workgroup: whole query blocks logical, logical + nwg, ... below
nwhole = (nblk // nwg) * nwg; with a split tail, the remaining rem = nblk % nwg blocks laid end to end as U = rem * T
key tiles, tail workgroup L < nt taking tiles [L U // nt, (L + 1) U // nt); the owner of tail tile u is
ceil((u + 1) nt / U) - 1; a piece's partial slot is 2 L + (0 for the first block of L's range, 1 for the second).
launch_stream's split rule (stream_split_params): non-causal, rem > 0 and T (nwg - rem) >= 4 nwg; nt = min(nwg, U,
3 rem). These tests replay the same integer arithmetic and check what the kernel relies on: every key tile of every
block is computed exactly once, a workgroup has at most two tail pieces, a cut block has 2 to 4 pieces, piece slots are
unique, the owner formula agrees with the ranges, and the counts match the merge's piece order."""
from __future__ import annotations

import itertools

import numpy as np

import pytest

SBM, PMAX, MAX_WG = 256, 4, 256


def split_params(W, H, nkeys, causal, nwg):
    nblk = (W + SBM - 1) // SBM * H
    rem = nblk % nwg
    T = (nkeys + 63) // 64
    if causal or rem == 0 or T * (nwg - rem) < 4 * nwg:
        return None
    return min(nwg, rem * T, rem * (PMAX - 1))


def schedule(W, H, nkeys, nwg, causal=False):
    """Per workgroup: list of (block, t0, t1, tail_index or None, slot or None); and per cut block its piece owners."""
    nqb = (W + SBM - 1) // SBM
    nblk = nqb * H
    T = (nkeys + 63) // 64
    nt = split_params(W, H, nkeys, causal, nwg)
    split = nt is not None
    nwhole = (nblk // nwg) * nwg if split else nblk
    U = (nblk - nwhole) * T
    grid = nwg if split else min(nblk, nwg)
    owner = (lambda u: -(-((u + 1) * nt) // U) - 1) if split else None
    work, pieces = {}, {}
    for L in range(grid):
        items = [(blk, 0, T, None, None) for blk in range(L, nwhole, nwg)]
        if split and L < nt:
            u0, u1 = L * U // nt, (L + 1) * U // nt
            n_p = (u1 - 1) // T - u0 // T + 1 if u1 > u0 else 0
            for k in range(n_p):
                i = u0 // T + k
                t0 = u0 - i * T if k == 0 else 0
                t1 = min(T, u1 - i * T)
                items.append((nwhole + i, t0, t1, i, 2 * L + k))
                pieces.setdefault(i, []).append((L, t0, t1, 2 * L + k))
                lf, ll = owner(i * T), owner((i + 1) * T - 1)
                assert lf <= L <= ll
        work[L] = items
    return work, pieces, dict(nblk=nblk, T=T, nt=nt, nwhole=nwhole, U=U, owner=owner)


SHAPES = [(4608, 24, 4608), (1280, 24, 1280), (12800, 24, 12800), (172992, 24, 172992), (65792, 1, 512),
          (300, 2, 5000), (4096, 16, 4096), (2048, 3, 777), (256 * 300, 1, 4096), (999, 7, 1100), (64, 1, 65)]


@pytest.mark.parametrize("W,H,nkeys", SHAPES)
@pytest.mark.parametrize("nwg", [256, 255, 128, 80, 8])
def test_every_tile_once(W, H, nkeys, nwg):
    work, pieces, p = schedule(W, H, nkeys, nwg)
    T = p["T"]
    ranges = {}
    for L, items in work.items():
        assert sum(1 for it in items if it[3] is not None) <= 2, "at most two tail pieces per workgroup"
        for blk, t0, t1, _, _ in items:
            assert 0 <= t0 < t1 <= T
            ranges.setdefault(blk, []).append((t0, t1))
    assert sorted(ranges) == list(range(p["nblk"]))
    for blk, rs in ranges.items():   # the ranges of a block tile [0, T) without gaps or overlaps
        rs.sort()
        assert rs[0][0] == 0 and rs[-1][1] == T and all(x[1] == y[0] for x, y in zip(rs, rs[1:]))
    slots = [s for ps in pieces.values() for (_, _, _, s) in ps]
    assert len(slots) == len(set(slots)) and all(0 <= s < 2 * MAX_WG for s in slots)
    for i, ps in pieces.items():
        owners = [L for (L, _, _, _) in ps]
        lf, ll = p["owner"](i * T), p["owner"]((i + 1) * T - 1)
        # the merge takes piece j from workgroup lf + j with slot 2 (lf + j) + (0 if block i is the first of its range)
        assert owners == list(range(lf, ll + 1)), "pieces are consecutive workgroups in order"
        assert 2 <= len(ps) <= PMAX
        for j, (L, t0, t1, s) in enumerate(ps):
            first_blk = (L * p["U"] // p["nt"]) // T
            assert s == 2 * L + (0 if i == first_blk else 1)
            assert t0 == (ps[j - 1][2] if j else 0) and (j < len(ps) - 1 or t1 == T)


def test_split_balances_the_qwen_step():
    """cfg2 on 256 CUs: 432 blocks of 72 tiles; whole rounds give 144 tiles to the busiest workgroup, the split tail
    122 (the balanced load is 121.5)."""
    work, pieces, p = schedule(4608, 24, 4608, 256)
    loads = [sum(t1 - t0 for _, t0, t1, _, _ in items) for items in work.values()]
    assert p["nt"] == 256 and p["nwhole"] == 256 and max(loads) == 122 and min(loads) == 121
    assert max(len(ps) for ps in pieces.values()) == 3
    # cfg1: 120 blocks of 20 tiles over all 256 workgroups instead of 120
    work, pieces, p = schedule(1280, 24, 1280, 256)
    assert p["nwhole"] == 0 and max(sum(t1 - t0 for _, t0, t1, _, _ in w) for w in work.values()) == 10


@pytest.mark.parametrize("W,H,nkeys,nwg", [(4608, 24, 4608, 256), (64, 1, 65, 256), (2048, 8, 2048, 256)])
def test_no_split_when_it_does_not_pay(W, H, nkeys, nwg):
    """Causal calls keep whole blocks, and so do calls whose balancing would save less than 4 key tiles per workgroup
    (2 tiles a block); 64 blocks of 32 tiles on 256 workgroups are split."""
    nt = split_params(W, H, nkeys, True, nwg)
    assert nt is None
    if (W, H) == (64, 1):
        assert split_params(W, H, nkeys, False, nwg) is None       # 2 tiles: balancing saves less than 4
    if (W, H) == (2048, 8):
        assert split_params(W, H, nkeys, False, nwg) is not None   # 64 blocks of 32 tiles over 256 workgroups


def test_owner_formula_matches_ranges():
    for U, nt in itertools.product([1, 5, 96, 1000, 12672, 7 * 2703], [1, 3, 7, 100, 256]):
        if nt > U:
            continue
        owner = lambda u: -(-((u + 1) * nt) // U) - 1
        for L in range(nt):
            for u in {L * U // nt, (L + 1) * U // nt - 1}:
                assert owner(u) == L


# ---- the value tile in LDS (attn_stream.hip: vt_offset, vt_lane_row, vt_lane_chunk, vt_lane), restated
def vt_offset(r, c):
    return 256 * (4 * (r >> 2) + (c >> 2)) + 64 * (r & 3) + 16 * (c & 3)


def vt_lane_row(l):
    return (l >> 2) & 3


def vt_lane_chunk(l):
    return 4 * (l >> 4) + (l & 3)


def vt_lane(l):
    return 2048 * (l >> 5) + 64 * ((l >> 2) & 3) + 32 * ((l >> 4) & 1) + 8 * (l & 3)


def _ds_read_tr16_b64(lds_u16, addr_bytes):
    """ds_read_b64_tr_b16 on 64 lanes: in each group of 16 lanes, lane 4 j + q supplies four 16-bit elements (its 8
    bytes) as columns 4 q .. 4 q + 3 of row j of a 4 x 16 block; lane s of the group receives column s of rows 0-3."""
    out = np.zeros((64, 4), dtype=lds_u16.dtype)
    for g in range(4):
        block = np.zeros((4, 16), dtype=lds_u16.dtype)
        for s in range(16):
            a = addr_bytes[16 * g + s]
            assert a % 8 == 0
            block[s >> 2, 4 * (s & 3):4 * (s & 3) + 4] = lds_u16[a // 2:a // 2 + 4]
        for s in range(16):
            out[16 * g + s] = block[:, s]
    return out


def test_value_rows_lds_layout_gives_the_pv_operand():
    """The direct loads of a value tile (wave w, load i, lane l: LDS bytes 2048 w + 1024 i + 16 l <- row
    8 w + 4 i + vt_lane_row(l), chunk vt_lane_chunk(l)) fill every 16-byte unit of the slot once, at vt_offset; and two
    transposed reads at vt_lane(l) + 4096 kk + 256 db (+ 1024) give lane l = 32 hf + n the A operand of the P V MFMA:
    keys 16 kk + 8 hf .. +7 of dim 32 db + n. The eight-byte addresses of one read fall on distinct banks in each
    half-wave (64 banks of 4 bytes: the read takes the minimum two passes)."""
    rng = np.random.default_rng(0)
    V = rng.integers(0, 1 << 16, size=(64, 128), dtype=np.uint16)
    lds = np.full(8192, 0xFFFF, dtype=np.uint16)
    seen = set()
    for w in range(8):
        for i in range(2):
            for l in range(64):
                o = 2048 * w + 1024 * i + 16 * l
                r, c = 8 * w + 4 * i + vt_lane_row(l), vt_lane_chunk(l)
                assert vt_offset(r, c) == o
                seen.add((r, c))
                lds[o // 2:o // 2 + 8] = V[r, 8 * c:8 * c + 8]
    assert len(seen) == 64 * 16
    lanes = np.arange(64)
    for kk in range(4):
        for db in range(4):
            parts = []
            for p in range(2):
                addr = np.array([vt_lane(l) + 4096 * kk + 256 * db + 1024 * p for l in lanes])
                for half in (addr[:32], addr[32:]):
                    banks = set()
                    for a in half:
                        for b in (a // 4 % 64, a // 4 % 64 + 1):
                            assert b not in banks, "bank conflict"
                            banks.add(b)
                parts.append(_ds_read_tr16_b64(lds, addr))
            frag = np.concatenate(parts, axis=1)
            for l in lanes:
                hf, n = l >> 5, l & 31
                want = V[16 * kk + 8 * hf:16 * kk + 8 * hf + 8, 32 * db + n]
                assert np.array_equal(frag[l], want), (kk, db, l)
