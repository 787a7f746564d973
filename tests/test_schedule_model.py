"""The drop-in launch's schedule (attention.hip: sched_inverse, sched_count,
sched_scan, sched_fill), restated in numpy from its index arithmetic and
checked for what the launches rely on: every window the order names lands in
exactly one slot (team list or one-wave slot), every slot is written, every
write stays inside its buffer, heavier classes come first within each XCD
share, and each share holds a contiguous index range of each class.  The
kernels themselves meet the oracle on the GPU (test_gpu_parity, test_gpu_fuzz);
this pins the arithmetic on the CPU, including orders with invalid, repeated
and missing entries and inverse arrays holding stale values.  CPU only."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rng

C, B, X, TEAM_CAP = 64, 1024, 8, 512   # classes, windows per block, XCDs, team list


def heavy_tiles(T: int, W: int) -> int:
    mean = (T + W - 1) // W if W else 0
    return max(8 * mean, 1024)


def schedule(offs: np.ndarray, order: np.ndarray | None, stale: np.ndarray | None,
             team_cap: int = TEAM_CAP):
    """Returns (team list, one-wave slots, class position of each window)."""
    W = len(offs) - 1
    T = int(offs[-1])
    nb = (W + B - 1) // B
    L = ((W + X - 1) // X + C + 3) // 4 * 4
    # sched_inverse: scattered positions; repeated windows keep any of theirs
    inv = stale.copy() if stale is not None else np.full(W, -7, np.int64)
    if order is not None:
        ok = (order >= 0) & (order < W)
        inv[order[ok]] = np.nonzero(ok)[0]
    # sched_count: class position q of every window (-1: not named)
    w = np.arange(nb * B)
    tiles = np.full(nb * B, -1, np.int64)
    tiles[:W] = np.diff(np.clip(offs, 0, T))
    named = w < W
    if order is not None:
        p = np.where(named, inv[np.minimum(w, W - 1)], -1)
        good = (p >= 0) & (p < W)
        named &= good & (order[np.clip(p, 0, W - 1)] == w)
    octave = np.where(tiles > 0, np.floor(np.log2(np.maximum(tiles, 1))).astype(np.int64) + 1, 0)
    q = np.where(tiles > heavy_tiles(T, W), 31 - octave, C - 1 - octave)
    q = np.where(named, q, -1)
    counts = np.zeros((C, nb), np.int64)
    for b in range(nb):
        qb = q[b * B:(b + 1) * B]
        counts[:, b] = np.bincount(qb[qb >= 0], minlength=C)
    # sched_scan
    before = np.cumsum(counts, 1) - counts
    total = counts.sum(1)
    heavy = np.where(np.arange(C) < C // 2, total, 0)
    hb = np.cumsum(heavy) - heavy
    taken = np.maximum(0, np.minimum(heavy, team_cap - hb))
    team_all = min(team_cap, int(heavy.sum()))
    team_base = np.where(np.arange(C) < C // 2, np.minimum(hb, team_cap), team_all)
    size = total - taken
    share = np.array([[s * (x + 1) // X - s * x // X for s in size] for x in range(X)])
    xcd_base = np.cumsum(share, 1) - share
    xcd_items = share.sum(1)
    assert xcd_items.max() <= L
    # sched_fill
    sched = np.full(X * L, -99, np.int64)
    team = np.full(TEAM_CAP, -99, np.int64)
    g = np.arange(max(nb * B, X * L))
    tail = (g < X * L) & (g // X >= xcd_items[g % X])
    sched[g[tail]] = -1
    team[team_all:] = -1
    for b in range(nb):
        for t, qq in enumerate(q[b * B:(b + 1) * B]):
            if qq < 0:
                continue
            r = before[qq, b] + int(np.count_nonzero(q[b * B:b * B + t] == qq))
            win = b * B + t
            if r < taken[qq]:
                k = team_base[qq] + r
                assert 0 <= k < TEAM_CAP and team[k] == -99
                team[k] = win
                continue
            sz, r2 = size[qq], r - taken[qq]
            x = (X * r2 + X - 1) // sz
            assert 0 <= x < X and sz * x // X <= r2 < sz * (x + 1) // X
            i = xcd_base[x, qq] + r2 - sz * x // X
            k = i * X + x
            assert 0 <= k < X * L and sched[k] == -99
            sched[k] = win
    assert not (sched == -99).any() and not (team == -99).any()
    return team, sched, q[:W]


def cases():
    r = rng(301)
    out = []
    for k in range(12):
        if k % 3 == 0:                                       # power-law windows, some heavy
            W = int(r.integers(513, 3500))
            tiles = r.zipf(1.6, W).clip(0, 30000)
        elif k % 3 == 1:                                     # no heavy window
            W = int(r.integers(513, 3500))
            tiles = r.integers(0, 400, W)
        else:                                                # more heavy windows than the list
            W = int(r.integers(8000, 10000))
            tiles = r.integers(0, 50, W)
            tiles[r.choice(W, int(r.integers(560, 700)), replace=False)] = r.integers(5000, 9000)
        offs = np.concatenate([[0], np.cumsum(tiles)]).astype(np.int64)
        kind = ("natural", "permutation", "partial")[k % 4 if k % 4 < 3 else 2]
        out.append((k, offs, kind))
    return out


@pytest.mark.parametrize("k,offs,kind", cases())
def test_schedule_places_every_named_window_once(k, offs, kind):
    r = rng(400 + k)
    W = len(offs) - 1
    order = stale = None
    if kind == "permutation":
        order = r.permutation(W)
    elif kind == "partial":
        order = r.integers(-3, W + 3, W)                     # invalid, repeated, missing
    if order is not None:
        stale = r.integers(-5, W + 5, W)                     # whatever the scratch held
    for team_cap in (TEAM_CAP, 0):                           # drop-in launch, plan
        team, sched, q = schedule(offs, order, stale, team_cap)
        placed = np.concatenate([team[team >= 0], sched[sched >= 0]])
        named = set(range(W)) if order is None else {int(v) for v in order if 0 <= v < W}
        assert len(placed) == len(set(placed.tolist())) and set(placed.tolist()) == named
        if team_cap == 0:
            assert (team == -1).all()
        # the team list: the named heavy windows up to its size, heaviest
        # octaves first, index order within an octave
        tiles = np.diff(offs)
        big = [v for v in sorted(named) if tiles[v] > heavy_tiles(int(offs[-1]), W)]
        tl = team[team >= 0]
        assert len(tl) == min(team_cap, len(big)) and all(tiles[tl] > heavy_tiles(int(offs[-1]), W))
        oct_ = np.floor(np.log2(np.maximum(tiles, 1))).astype(int)
        assert all((-oct_[a], a) < (-oct_[b], b) for a, b in zip(tl, tl[1:]))
        rest = np.setdiff1d(np.array(big, np.int64), tl)
        assert len(rest) == 0 or len(tl) == 0 or oct_[rest].max() <= oct_[tl].min()
        assert (q[tl] < C // 2).all() and (q[rest] < C // 2).all()
        assert all((q[a], a) < (q[b], b) for a, b in zip(tl, tl[1:]))
        # each XCD share: classes in order, index order within a class
        L = len(sched) // X
        for x in range(X):
            s = sched[x::X]
            s = s[s >= 0]
            assert all((q[a], a) < (q[b], b) for a, b in zip(s, s[1:]))
        # within a class, share x holds a contiguous range of the class's windows
        for cls in np.unique(q[q >= 0]):
            members = sorted(int(v) for v in sched[sched >= 0] if q[v] == cls)
            if not members:
                continue
            rank = {v: i for i, v in enumerate(members)}
            for x in range(X):
                s = [rank[int(v)] for v in sched[x::X] if v >= 0 and q[v] == cls]
                assert s == list(range(s[0], s[0] + len(s))) if s else True
