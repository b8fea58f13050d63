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
