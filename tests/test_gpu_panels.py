"""Panels: 16 consecutive row windows that share the K/V rows two or more of
them attend through LDS (community-ordered graphs, masked semantics).

* The compile's staging decision is restated in numpy (`panel_model`): per
  panel, the columns attended by >= 2 of its windows are staged, unless the
  panel has more than 8,192 tiles or more than 6,144 such columns (then every
  column is fetched per window).  The GPU's row-fetch counts must equal the
  model's exactly, which pins which columns each panel stages.
* Outputs meet the CPU oracle at the north-star bar (max abs 2e-3, normwise
  max rel 1e-2), including panels of both fallback kinds and a last, partial
  panel; Q = 0 gives the exact neighbour mean of V, which any column counted
  twice (staged and direct) or dropped would break.
* Repeated passes are bit-identical; O(Q, K, 2V) == 2 O(Q, K, V) bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from conftest import rng

pytestmark = pytest.mark.gpu

ABS_TOL, REL_TOL = 2e-3, 1e-2
PANEL, MAX_TILES, MAX_STAGED = 16, 8192, 6144


def log(msg: str) -> None:
    print(msg, flush=True)


def csr_from_edges(n: int, u: np.ndarray, v: np.ndarray):
    key = np.unique(u.astype(np.int64) * n + v)
    rows, cols = key // n, key % n
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rows + 1, 1)
    return np.cumsum(rp).astype(np.int32), cols.astype(np.int32)


def community_graph(n: int, comm: int, deg: int, p_intra: float, seed: int):
    """Directed graph: each row has `deg` neighbours, a share p_intra inside
    its own community of `comm` consecutive nodes, plus a self-loop."""
    r = rng(seed)
    u = np.repeat(np.arange(n), deg)
    intra = r.random(len(u)) < p_intra
    c0 = (u // comm) * comm
    v = np.where(intra, c0 + r.integers(0, comm, len(u)), r.integers(0, n, len(u)))
    v = np.minimum(v, n - 1)
    return np.concatenate([u, np.arange(n)]), np.concatenate([v, np.arange(n)])


def mixed_graph(seed: int):
    """Community windows, then one panel whose 16 windows hold > 8,192 tiles
    and one whose windows share > 6,144 columns (both fetched per window),
    then a partial panel of community rows."""
    n_comm = 32768
    u1, v1 = community_graph(n_comm, 1024, 24, 0.8, seed)
    r = rng(seed + 1)
    n = n_comm + 2 * 256 + 100
    dense = np.arange(n_comm, n_comm + 256)
    u2 = np.repeat(dense, 700)
    v2 = r.integers(0, n, len(u2))
    shared = np.arange(n_comm + 256, n_comm + 512)
    cols = np.arange(1000, 8000)
    u3 = np.repeat(shared, len(cols))
    v3 = np.tile(cols, len(shared))
    tail = np.arange(n_comm + 512, n)
    u4 = np.repeat(tail, 20)
    v4 = n_comm + 512 + r.integers(0, len(tail), len(u4))
    u = np.concatenate([u1, u2, u3, u4, tail])
    v = np.concatenate([v1, v2, v3, v4, tail])
    return csr_from_edges(n, u, v)


def panel_model(rp: np.ndarray, ci: np.ndarray) -> tuple[int, int]:
    """(window, column) pairs, and K/V row fetches per head with panels."""
    n = len(rp) - 1
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(rp))
    win = rows // 16
    wc = np.unique(win * n + ci)
    w_of, col = wc // n, wc % n
    pan = w_of // PANEL
    gathered = len(wc)
    fetched = 0
    # tiles per panel: distinct (window, block column)
    tiles = np.unique(w_of * ((n + 15) // 16) + col // 16)
    tiles_per_panel = np.bincount(tiles // ((n + 15) // 16) // PANEL, minlength=pan.max() + 1)
    pk, cnt = np.unique(pan * n + col, return_counts=True)
    p_of = pk // n
    for P in range(int(pan.max()) + 1):
        c = cnt[p_of == P]
        staged = int((c >= 2).sum())
        if tiles_per_panel[P] > MAX_TILES or staged > MAX_STAGED:
            fetched += int(c.sum())
        else:
            fetched += staged + int(c[c < 2].sum())
    return gathered, fetched


class Case:
    def __init__(self, f3s, rp, ci, H, seed, Qzero=False, seg=0):
        self.f3s, self.rp, self.ci, self.H = f3s, rp, ci, H
        self.n = n = len(rp) - 1
        r = rng(seed)
        f = lambda: r.standard_normal((n, H, 64)).astype(np.float16)
        self.Q, self.K, self.V = f(), f(), f()
        if Qzero:
            self.Q[:] = 0
        for a in (self.K, self.V):   # no fp16 subnormals: the scaling check is exact
            a[np.abs(a.astype(np.float32)) < 2.0 ** -14] = 0
        self.bsf = f3s.convert_device(f3s.DeviceCSR(rp, ci))
        self.dQ, self.dK, self.dV = (f3s.DeviceArray.from_numpy(x.view(np.uint16))
                                     for x in (self.Q, self.K, self.V))
        self.dO = f3s.DeviceArray((n, H, 64), np.float32)
        self.plan = f3s.Plan(self.bsf, None, H=H, seg_tiles=seg)
        self.plan.compile()

    def run(self, plan=None, V=None, scale=0.125) -> np.ndarray:
        dV = self.dV if V is None else self.f3s.DeviceArray.from_numpy(V.view(np.uint16))
        self.dO.fill_bytes(0xFF)
        (plan or self.plan).forward(self.dQ, self.dK, dV, self.dO, masked=True, scale=scale)
        self.f3s.synchronize()
        return self.dO.numpy()

    def oracle(self, scale=0.125) -> np.ndarray:
        f = lambda x: x.astype(np.float32)
        return orc.masked_attention(self.n, 64, self.H, f(self.Q), f(self.K), f(self.V),
                                    self.rp, self.ci, scale)


def check_close(got, want, what):
    assert np.all(np.isfinite(got)), what
    diff = np.abs(got.astype(np.float64) - want)
    mabs, mrel = float(diff.max()), float(diff.max() / np.abs(want).max())
    log(f"  {what}: max_abs={mabs:.3e} max_rel={mrel:.3e}")
    assert mabs <= ABS_TOL and mrel <= REL_TOL, what


@pytest.mark.parametrize("H", [1, 4])
def test_panels_community_graph(gpu, H):
    n = 20000   # not a multiple of 256: the last panel is partial
    rp, ci = csr_from_edges(n, *community_graph(n, 1024, 24, 0.8, 7))
    c = Case(gpu, rp, ci, H, seed=7)
    npanels, gathered, fetched = c.plan.panel_info()
    assert npanels == (n // 16 + 15) // 16
    assert (gathered, fetched) == panel_model(rp, ci)
    log(f"H={H}: {npanels} panels, row fetches {gathered} -> {fetched} "
        f"({gathered / fetched:.2f}x)")
    got = c.run()
    check_close(got, c.oracle(), f"community H={H}")
    assert np.array_equal(c.run().view(np.uint32), got.view(np.uint32)), "not deterministic"
    # exact V scaling (fp16 doubling and every fp32 step scale exactly)
    two_v = (c.V.astype(np.float32) * 2).astype(np.float16)
    assert np.array_equal(c.run(V=two_v).view(np.uint32), (got * 2).view(np.uint32))
    # against the gathered pass of a plan with a window order (no panels)
    order = gpu.window_order_device(c.bsf)
    gathered_plan = gpu.Plan(c.bsf, order, H=H)
    gathered_plan.compile()
    assert gathered_plan.panel_info()[0] == 0
    check_close(c.run(plan=gathered_plan), got.astype(np.float64), f"gathered vs panels H={H}")


def test_panels_fallbacks_and_mean(gpu):
    rp, ci = mixed_graph(11)
    n = len(rp) - 1
    # no split windows (an automatic plan would split the 2,000-tile ones,
    # and plans with split windows gather per window)
    c = Case(gpu, rp, ci, 1, seed=11, Qzero=True, seg=1 << 30)
    npanels, gathered, fetched = c.plan.panel_info()
    assert npanels > 0
    assert (gathered, fetched) == panel_model(rp, ci)
    log(f"mixed: {npanels} panels, row fetches {gathered} -> {fetched}")
    got = c.run(scale=1.0)[:, 0]
    check_close(got, c.oracle(scale=1.0)[:, 0], "mixed")
    # Q = 0: every row is the plain mean of V over its neighbours
    V = c.V[:, 0].astype(np.float64)
    sums = np.add.reduceat(V[ci], rp[:-1], axis=0)
    want = sums / np.diff(rp)[:, None]
    assert np.abs(got - want).max() <= 1e-3


def test_panels_not_used_when_they_do_not_pay(gpu):
    # a random graph: windows of a panel share almost no columns
    from conftest import random_csr
    rp, ci = random_csr(20000, 16, 3)
    bsf = gpu.convert_device(gpu.DeviceCSR(rp, ci))
    plan = gpu.Plan(bsf, None, H=1)
    plan.compile()
    npanels, gathered, fetched = plan.panel_info()
    assert npanels == 0 and gathered < 1.3 * fetched
    assert (gathered, fetched) == panel_model(rp, ci)
