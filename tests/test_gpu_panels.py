"""Tile-dense panels: 16 consecutive row windows share, through LDS, the K/V
rows of the block columns active in two or more of them; each window's other
tiles run through the gathered pass, which folds the shared part in.

* The compile's staging decision is restated in numpy (`panel_model`): per
  panel, the block columns active in >= 2 of its windows are staged, unless
  the panel has more than 8,192 tiles or their columns (< n) number more than
  6,144 (then nothing is staged).  The GPU's K/V row-fetch counts must equal
  the model's exactly, which pins what each panel stages.
* Outputs meet the CPU oracle (tile-dense semantics, tests/test_fused_3s_v2.cu
  :17-59) at the north-star bar (max abs 2e-3, normwise max rel 1e-2),
  including both fallback kinds and a last, partial panel.  With K = 0 every
  row is the plain mean of V over its window's tile columns < n, which a tile
  counted twice (staged and residual) or dropped would break.
* Repeated passes are bit-identical; O(Q, K, 2V) == 2 O(Q, K, V) bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from conftest import random_csr, rng

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


def community_edges(n: int, comm: int, deg: int, p_intra: float, seed: int):
    """Directed edges: each row has `deg` neighbours, a share p_intra inside
    its own community of `comm` consecutive nodes, plus a self-loop."""
    r = rng(seed)
    u = np.repeat(np.arange(n), deg)
    intra = r.random(len(u)) < p_intra
    c0 = (u // comm) * comm
    v = np.where(intra, c0 + r.integers(0, comm, len(u)), r.integers(0, n, len(u)))
    v = np.minimum(v, n - 1)
    return np.concatenate([u, np.arange(n)]), np.concatenate([v, np.arange(n)])


def mixed_graph(seed: int):
    """Community windows, then one panel whose 16 windows hold > 8,192 tiles,
    one whose shared block columns hold > 6,144 columns (both stage nothing),
    then a partial panel."""
    n_comm = 16384
    u1, v1 = community_edges(n_comm, 512, 16, 0.8, seed)
    r = rng(seed + 1)
    n = n_comm + 2 * 256 + 100
    dense = np.arange(n_comm, n_comm + 256)
    u2 = np.repeat(dense, 700)
    v2 = r.integers(0, n, len(u2))
    shared = np.arange(n_comm + 256, n_comm + 512)
    cols = np.arange(1000, 8000, 2)                  # 438 block columns, 7,000 columns
    u3 = np.repeat(shared, len(cols))
    v3 = np.tile(cols, len(shared))
    tail = np.arange(n_comm + 512, n)
    u4 = np.repeat(tail, 20)
    v4 = n_comm + 512 + r.integers(0, len(tail), len(u4))
    u = np.concatenate([u1, u2, u3, u4, tail])
    v = np.concatenate([v1, v2, v3, v4, tail])
    return csr_from_edges(n, u, v)


def panel_model(rp: np.ndarray, ci: np.ndarray) -> tuple[int, int]:
    """K/V row fetches per head of a tile-dense pass: (without panels, with)."""
    n = len(rp) - 1
    nbc = (n + 15) // 16
    rows = np.repeat(np.arange(n, dtype=np.int64), np.diff(rp))
    tiles = np.unique((rows // 16) * nbc + ci // 16)          # (window, block column)
    w_of, bc = tiles // nbc, tiles % nbc
    width = np.minimum(16, n - 16 * bc)                        # columns < n
    pan = w_of // PANEL
    gathered = int(width.sum())
    key, inv, cnt = np.unique(pan * nbc + bc, return_inverse=True, return_counts=True)
    shared = cnt[inv] >= 2                                     # per tile
    fetched = 0
    for P in range(int(pan.max()) + 1):
        sel = pan == P
        k_sel = (key // nbc == P) & (cnt >= 2)
        S = int(np.minimum(16, n - 16 * (key[k_sel] % nbc)).sum())
        if sel.sum() > MAX_TILES or S > MAX_STAGED:
            fetched += int(width[sel].sum())
        else:
            fetched += S + int(width[sel & ~shared].sum())
    return gathered, fetched


class Case:
    def __init__(self, f3s, rp, ci, H, seed, seg=0, Kzero=False):
        self.f3s, self.rp, self.ci, self.H = f3s, rp, ci, H
        self.n = n = len(rp) - 1
        r = rng(seed)
        f = lambda: r.standard_normal((n, H, 64)).astype(np.float16)
        self.Q, self.K, self.V = f(), f(), f()
        if Kzero:
            self.K[:] = 0
        self.V[np.abs(self.V.astype(np.float32)) < 2.0 ** -14] = 0   # exact scaling check
        self.bsf = f3s.convert_device(f3s.DeviceCSR(rp, ci))
        self.dQ, self.dK, self.dV = (f3s.DeviceArray.from_numpy(x.view(np.uint16))
                                     for x in (self.Q, self.K, self.V))
        self.dO = f3s.DeviceArray((n, H, 64), np.float32)
        self.plan = f3s.Plan(self.bsf, None, H=H, seg_tiles=seg)
        self.plan.compile()

    def run(self, plan=None, V=None, scale=0.125) -> np.ndarray:
        dV = self.dV if V is None else self.f3s.DeviceArray.from_numpy(V.view(np.uint16))
        self.dO.fill_bytes(0xFF)
        (plan or self.plan).forward(self.dQ, self.dK, dV, self.dO, masked=False, scale=scale)
        self.f3s.synchronize()
        return self.dO.numpy()

    def oracle(self, scale=0.125) -> np.ndarray:
        hb = self.bsf.to_host()
        f = lambda x: x.astype(np.float32)
        return orc.tile_dense_attention(self.n, 64, self.H, f(self.Q), f(self.K), f(self.V),
                                        hb.window_offsets, hb.block_col_indices, scale)


def check_close(got, want, what):
    assert np.all(np.isfinite(got)), what
    diff = np.abs(got.astype(np.float64) - want)
    mabs, mrel = float(diff.max()), float(diff.max() / np.abs(want).max())
    log(f"  {what}: max_abs={mabs:.3e} max_rel={mrel:.3e}")
    assert mabs <= ABS_TOL and mrel <= REL_TOL, what


@pytest.mark.parametrize("H", [1, 2])
def test_panels_community_graph(gpu, H):
    # 12,000 nodes: 750 windows, the last panel partial; H = 1 plans teams
    # of 4 waves for masked passes (panels take their windows from them)
    n = 12000
    rp, ci = csr_from_edges(n, *community_edges(n, 512, 16, 0.8, 7))
    c = Case(gpu, rp, ci, H, seed=7)
    npanels, gathered, fetched = c.plan.panel_info()
    assert npanels == ((n + 15) // 16 + 15) // 16
    assert (gathered, fetched) == panel_model(rp, ci)
    log(f"H={H}: {npanels} panels, K/V row fetches {gathered} -> {fetched} "
        f"({gathered / fetched:.2f}x)")
    got = c.run()
    check_close(got, c.oracle(), f"community H={H}")
    assert np.array_equal(c.run().view(np.uint32), got.view(np.uint32)), "not deterministic"
    two_v = (c.V.astype(np.float32) * 2).astype(np.float16)
    assert np.array_equal(c.run(V=two_v).view(np.uint32), (got * 2).view(np.uint32))
    # the gathered pass (a plan with a window order has no panels) agrees
    order = gpu.window_order_device(c.bsf)
    gathered_plan = gpu.Plan(c.bsf, order, H=H)
    gathered_plan.compile()
    assert gathered_plan.panel_info()[0] == 0
    check_close(c.run(plan=gathered_plan), got.astype(np.float64), f"gathered vs panels H={H}")
    # masked passes of the same plan do not use panels and still meet the oracle
    c.dO.fill_bytes(0xFF)
    c.plan.forward(c.dQ, c.dK, c.dV, c.dO, masked=True, scale=0.125)
    gpu.synchronize()
    f = lambda x: x.astype(np.float32)
    want_m = orc.masked_attention(n, 64, H, f(c.Q), f(c.K), f(c.V), rp, ci, 0.125)
    check_close(c.dO.numpy(), want_m, f"masked, same plan H={H}")


def test_panels_fallbacks_and_mean(gpu):
    rp, ci = mixed_graph(11)
    n = len(rp) - 1
    # no split windows (an automatic plan splits the 2,000-tile windows, and
    # plans with split windows take no panels)
    c = Case(gpu, rp, ci, 1, seed=11, seg=1 << 30, Kzero=True)
    npanels, gathered, fetched = c.plan.panel_info()
    assert npanels > 0
    assert (gathered, fetched) == panel_model(rp, ci)
    log(f"mixed: {npanels} panels, K/V row fetches {gathered} -> {fetched}")
    got = c.run(scale=1.0)[:, 0]
    check_close(got, c.oracle(scale=1.0)[:, 0], "mixed")
    # K = 0: each row is the plain mean of V over its window's tile columns
    hb = c.bsf.to_host()
    V = c.V[:, 0].astype(np.float64)
    for w in range(0, (n + 15) // 16, 7):
        b = hb.block_col_indices[hb.window_offsets[w]:hb.window_offsets[w + 1]]
        cols = (b[:, None] * 16 + np.arange(16)).ravel()
        cols = cols[cols < n]
        want = V[cols].mean(axis=0) if len(cols) else np.zeros(64)
        assert np.abs(got[16 * w:min(16 * w + 16, n)] - want).max() <= 1e-3, w


def test_panels_not_used_when_they_do_not_pay(gpu):
    # a random graph: the windows of a panel share almost no block columns
    rp, ci = random_csr(20000, 16, 3)
    bsf = gpu.convert_device(gpu.DeviceCSR(rp, ci))
    plan = gpu.Plan(bsf, None, H=1)
    plan.compile()
    npanels, gathered, fetched = plan.panel_info()
    assert npanels == 0 and gathered < 1.5 * fetched
    assert (gathered, fetched) == panel_model(rp, ci)
