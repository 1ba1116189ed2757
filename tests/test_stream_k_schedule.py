"""CPU: the four-wave stream-K schedule's unit bookkeeping.

gemm_w4sk_kernel splits the last L stages of each of T tiles over Gt tail
workgroups: tail j owns units [j*Ut/Gt, (j+1)*Ut/Gt) of the Ut = T*L
(tile, stage) pairs, walks them tile by tile as pieces, stores piece (j, t)
in slot j + t and counts it on tile t; the main workgroup of tile t waits
for owner(t*L + L - 1) - owner(t*L) + 1 pieces and reads slots owner(t*L) + t
and owner(t*L + L - 1) + t.  This walks the schedule as the kernel does (the
integer expressions of csrc/gemm.hip's w4sk_start / w4sk_owner) and checks
what its correctness rests on, over every (T, Gt) the planner can produce on
a 256-CU device and a range of L: every unit is covered exactly once, each
tile has one or two pieces, the pieces the main workgroup expects are exactly
the ones stored (lower K range first), slots are distinct and below
T + Gt - 1.  A schedule with Gt > T (more tails than tiles) breaks the
two-piece bound, which the planner excludes; the test checks that too.
"""

from __future__ import annotations

import pytest


def start(j: int, ut: int, gt: int) -> int:
    return j * ut // gt


def owner(v: int, ut: int, gt: int) -> int:
    return ((v + 1) * gt - 1) // ut


def walk(T: int, L: int, gt: int):
    """{tile: [(tail, first stage, length, slot)]} as the tails store them."""
    ut = T * L
    pieces: dict[int, list] = {}
    for j in range(gt):
        v, vend = start(j, ut, gt), start(j + 1, ut, gt)
        while v < vend:
            t, r = divmod(v, L)
            n = min(L - r, vend - v)
            pieces.setdefault(t, []).append((j, r, n, j + t))
            v += n
    return pieces


def plans(cus: int = 256):
    """(T, Gt) pairs the planner forms: T*16 > 11*cus, Gt = min(T, cus - T
    rounded up to 8) rounded down to 8, Gt >= 8."""
    for T in range(cus * 11 // 16 + 1, cus):
        t8 = -(-T // 8) * 8
        gt = min(T, cus - t8) // 8 * 8
        if gt >= 8:
            yield T, gt


@pytest.mark.parametrize("L", [4, 7, 11, 28, 32, 64])
def test_every_unit_once_and_two_pieces_at_most(L):
    for T, gt in plans():
        pieces = walk(T, L, gt)
        slots = set()
        for t in range(T):
            ps = pieces[t]
            assert 1 <= len(ps) <= 2, (T, gt, L, t, ps)
            # K order along the tile, contiguous, covering [0, L)
            assert [p[1] for p in ps] == sorted(p[1] for p in ps)
            assert ps[0][1] == 0 and sum(p[2] for p in ps) == L
            if len(ps) == 2:
                assert ps[1][1] == ps[0][2]
            # what the main workgroup expects
            ut = T * L
            j0, j1 = owner(t * L, ut, gt), owner(t * L + L - 1, ut, gt)
            assert j1 - j0 + 1 == len(ps)
            assert [p[3] for p in ps] == ([j0 + t] if j0 == j1 else [j0 + t, j1 + t])
            for p in ps:
                assert p[3] not in slots and 0 <= p[3] < T + gt - 1
                slots.add(p[3])


def test_more_tails_than_tiles_breaks_the_two_piece_bound():
    pieces = walk(16, 4, 40)
    assert max(len(p) for p in pieces.values()) > 2


def test_baseline_down_proj_schedule():
    """M = 3100, N = 4096, K = 12288 on 256 CUs: 208 tiles, 48 tails, 192
    stages of 64, ks = the even share + 4 = 160."""
    T, gt, KT = 208, 48, 192
    ks = (T * KT + (T + gt) // 2) // (T + gt) + 4
    assert ks == 160
    pieces = walk(T, KT - ks, gt)
    # 47 tail boundaries at j * 6656 / 48 = j * 13 * 32 / 3 units: the 15 with
    # j divisible by 3 fall on a tile edge, the other 32 split a tile
    assert sum(len(p) == 2 for p in pieces.values()) == 32
    assert max(p[3] for ps in pieces.values() for p in ps) == T + gt - 2
