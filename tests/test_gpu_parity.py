"""Parity of the HIP path (through the C-ABI) with the CPU oracle.

Bars: converter tile lists, masks, window order and the fp16 cast are
bit-exact; attention output has max abs error <= 2e-3 and normwise max
relative error max|g - c| / max|c| <= 1e-2 against the fp32 oracle on
identical fp16-rounded inputs.  At the full
sizes of configs 4 and 5 the converter is compared in full and masked
attention on every row; tile-dense attention on every row of config 4 and
on a deterministic sample of row ranges (including the heaviest windows) of
config 5.
"""
from __future__ import annotations

import ctypes as C
import os
import time

import numpy as np
import pytest

import _oracle as orc
from conftest import GOLDEN, random_csr, rng

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3
REL_TOL = 1e-2


def log(msg: str) -> None:
    print(msg, flush=True)


def errors(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    mabs = float(diff.max()) if diff.size else 0.0
    scale = float(np.abs(want).max()) if want.size else 0.0
    return mabs, (mabs / scale if scale > 0 else mabs)


def elem_rel(got: np.ndarray, want: np.ndarray, floor: float = 0.1) -> float:
    """Largest elementwise relative error over the elements with |c| >= floor
    (reported for information; the bars are max_abs and the normwise max_rel)."""
    g, w = got.reshape(-1), want.reshape(-1)
    out = 0.0
    for i in range(0, g.size, 1 << 24):
        wi = w[i:i + (1 << 24)].astype(np.float64)
        big = np.abs(wi) >= floor
        if big.any():
            gi = g[i:i + (1 << 24)].astype(np.float64)
            out = max(out, float((np.abs(gi[big] - wi[big]) / np.abs(wi[big])).max()))
    return out


def assert_close(got, want, what=""):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    mabs, mrel = errors(got, want)
    log(f"  {what}: max_abs={mabs:.3e} max_rel={mrel:.3e} "
        f"(elementwise rel, |c| >= 0.1: {elem_rel(got, want):.3e})")
    assert mabs <= ABS_TOL and mrel <= REL_TOL, f"{what}: max_abs={mabs:.3e} max_rel={mrel:.3e}"


class Problem:
    """A graph plus fp16 features, on host and device."""

    def __init__(self, f3s, rp, ci, H=1, normal=False, seed=0, Qzero=False, f32=False):
        self.f3s = f3s
        self.n = len(rp) - 1
        self.H, self.d = H, 64
        self.rp, self.ci = np.asarray(rp, np.int32), np.asarray(ci, np.int32)
        n = self.n
        r = rng(seed)
        def feat():
            if f32:   # large inputs: U[-1, 1) drawn in float32
                return (r.random((n, H, 64), dtype=np.float32) * 2 - 1).astype(np.float16)
            x = r.standard_normal((n, H, 64)) if normal else r.uniform(-1, 1, (n, H, 64))
            return x.astype(np.float16)
        self.Q, self.K, self.V = feat(), feat(), feat()
        if Qzero:
            self.Q[:] = 0
        self.Qf, self.Kf, self.Vf = (x.astype(np.float32) for x in (self.Q, self.K, self.V))
        self.csr = f3s.DeviceCSR(self.rp, self.ci)
        self.bsf = f3s.convert_device(self.csr)
        self.dQ, self.dK, self.dV = (f3s.DeviceArray.from_numpy(x.view(np.uint16))
                                     for x in (self.Q, self.K, self.V))
        self.dO = f3s.DeviceArray((n, H, 64), np.float32)

    def host_bsf(self):
        return self.bsf.to_host()

    def run(self, masked=True, planned=False, seg=0, order=None, scale=1.0, compiled=False):
        self.dO.fill_bytes(0xFF)    # NaN poison: every real row must be written
        if planned:
            plan = self.f3s.Plan(self.bsf, order, H=self.H, seg_tiles=seg)
            if compiled:
                plan.compile()
            plan.forward(self.dQ, self.dK, self.dV, self.dO, masked=masked, scale=scale)
        else:
            self.f3s.attention_fwd(self.dQ, self.dK, self.dV, self.dO, self.bsf, order,
                                   masked=masked, H=self.H, scale=scale)
        self.f3s.synchronize()
        return self.dO.numpy()

    def oracle(self, masked=True, scale=1.0, rows=None):
        if masked:
            if rows is None:
                return orc.masked_attention(self.n, 64, self.H, self.Qf, self.Kf, self.Vf,
                                            self.rp, self.ci, scale)
            out = {}
            for (a, b) in rows:
                out[(a, b)] = orc.masked_attention(self.n, 64, self.H, self.Qf, self.Kf, self.Vf,
                                                   self.rp, self.ci, scale, a, b)[a:b]
            return out
        hb = self.host_bsf()
        if rows is None:
            return orc.tile_dense_attention(self.n, 64, self.H, self.Qf, self.Kf, self.Vf,
                                            hb.window_offsets, hb.block_col_indices, scale,
                                            fast=True)
        out = {}
        for (a, b) in rows:
            out[(a, b)] = orc.tile_dense_attention(self.n, 64, self.H, self.Qf, self.Kf, self.Vf,
                                                   hb.window_offsets, hb.block_col_indices, scale,
                                                   a, b, fast=True)[a:b]
        return out


def check_converter(f3s, rp, ci, bsf=None):
    n = len(rp) - 1
    if bsf is None:
        bsf = f3s.convert_device(f3s.DeviceCSR(rp, ci))
    hb = bsf.to_host()
    offs, bcol, mask = orc.convert(n, rp, ci)
    assert np.array_equal(hb.window_offsets, offs)
    assert np.array_equal(hb.block_col_indices, bcol)
    assert np.array_equal(hb.tile_masks, mask)
    return bsf


# --------------------------------------------------------------- plumbing

def test_device_visible(gpu):
    log(f"device: {gpu.device_name()}")


def test_cast_f32_to_f16_bit_exact(gpu):
    bits = rng(3).integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    x[np.isnan(x)] = 1.0
    x[:8] = [0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 2.9802322387695312e-08, 1e-30]
    n = len(x) - 3                      # odd tail exercises the scalar path
    dx = gpu.DeviceArray.from_numpy(x[:n])
    dh = gpu.DeviceArray(n, np.uint16)
    gpu.cast_f32_to_f16(dx, dh)
    assert np.array_equal(dh.numpy(), orc.f32_to_f16_bits(x[:n]))


# -------------------------------------------------------------- converter

@pytest.mark.parametrize("name", ["cora", "citeseer"])
def test_converter_fixtures(gpu, name):
    g = gpu.load_csr_graph(str(GOLDEN / name))
    bsf = check_converter(gpu, g.row_ptr, g.col_ind)
    if name == "cora":
        assert bsf.W == 170 and bsf.T == 7355


@pytest.mark.parametrize("cfg", [2, 3])
def test_converter_configs_small(gpu, cfg):
    rp, ci = gpu.CONFIGS[cfg].graph()
    check_converter(gpu, rp, ci)


@pytest.mark.parametrize("n", [0, 37])
def test_graph_without_edges(gpu, n):
    """No node (W = 0) or no edge at all (T = 0): the converter's offsets are
    all zero and T = 0 (converter.cu:15-44 gives the same), the window order
    is the identity, and every pass leaves O = 0 (a node without neighbours
    gets zeros, cpu_baseline.cpp:26-32; an empty window writes zeros)."""
    rp = np.zeros(n + 1, np.int32)
    ci = np.zeros(0, np.int32)
    bsf = check_converter(gpu, rp, ci)
    W = (n + 15) // 16
    assert bsf.W == W and bsf.T == 0
    fmt = gpu.convert_csr_to_block_sparse(n, rp, ci, verbose=False)
    assert fmt.num_row_windows == W and len(fmt.block_col_indices) == 0
    assert fmt.duplicate_entries == 0
    assert np.array_equal(np.sort(gpu.generate_balanced_window_order(fmt)), np.arange(W))
    order = gpu.window_order_device(bsf)
    if W:
        assert np.array_equal(order.numpy(), np.arange(W))
    if n == 0:
        return
    P = Problem(gpu, rp, ci)
    for masked in (True, False):
        assert np.array_equal(P.run(masked=masked), np.zeros((n, 1, 64), np.float32))
        assert np.array_equal(P.run(masked=masked, planned=True, compiled=masked),
                              np.zeros((n, 1, 64), np.float32))


@pytest.mark.parametrize("n,deg,seed", [(1, 0, 0), (2, 1, 1), (17, 3, 2), (100, 5, 3),
                                        (1000, 40, 4), (4099, 7, 5)])
def test_converter_random(gpu, n, deg, seed):
    rp, ci = random_csr(n, deg, seed, self_loops=(seed % 2 == 0))
    check_converter(gpu, rp, ci)


def star_graph(n: int, hubs=(0,)):
    """Hub rows connected to everything: windows far beyond the LDS cap."""
    edges = set()
    for h in hubs:
        for v in range(n):
            if v != h:
                edges.add((h, v))
                edges.add((v, h))
    for v in range(n):
        edges.add((v, v))
    e = np.array(sorted(edges), np.int64)
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, e[:, 0] + 1, 1)
    return np.cumsum(rp).astype(np.int32), e[:, 1].astype(np.int32)


def test_converter_hub_windows(gpu):
    # window 0 holds two hubs (2 x 40000 edges > LDS key capacity) and the
    # block-column range spans several slices of the hub path
    rp, ci = star_graph(40000, hubs=(0, 5))
    check_converter(gpu, rp, ci)


def test_converter_edge_count_boundaries(gpu):
    # Windows at each edge-count boundary of the converter: the persistent
    # kernel takes up to 1,024 edges per window (256 threads x 4), the hub
    # kernel keeps up to 8,192 in registers (1,024 threads x 8) and ORs the
    # masks of heavier windows straight into the output; one window of each
    # of 1,023 / 1,024 / 1,025 / 8,191 / 8,192 / 8,193 edges (row 0 of the
    # window carries the excess, partly repeated columns), beside light ones.
    n = 16 * 64
    r = rng(12)
    rows, cols = [np.arange(n)], [np.arange(n)]                 # self-loops
    for k, E in enumerate((1023, 1024, 1025, 8191, 8192, 8193)):
        u = 16 * (8 * k + 3)
        extra = E - 16                                           # the window's 16 self-loops
        rows.append(np.full(extra, u))
        cols.append(r.integers(0, n, extra))                     # repeats included
    rr, cc = np.concatenate(rows), np.concatenate(cols)
    order = np.lexsort((cc, rr))
    rr, cc = rr[order], cc[order]
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rr + 1, 1)
    rp = np.cumsum(rp).astype(np.int32)
    edges = np.diff(rp[::16])
    assert [int(edges[8 * k + 3]) for k in range(6)] == [1023, 1024, 1025, 8191, 8192, 8193]
    check_converter(gpu, rp, cc.astype(np.int32))


def test_converter_column_slices(gpu):
    # 137,500 block columns: one 4,297-word bitmap in the persistent kernel
    # (more than the per-window kernel's 65,536-column slice), windows with
    # edges at both ends of the column range
    n = 2_200_000
    r = rng(11)
    deg = r.integers(0, 4, n)
    deg[:2000] += 3
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(deg)
    ci = r.integers(0, n, int(rp[-1])).astype(np.int32)
    ci[rp[:2000]] = n - 1 - r.integers(0, 40, 2000)   # far end of the last slice
    ci[rp[:2000] + 1] = r.integers(0, 16 * 131072, 2000)
    check_converter(gpu, rp.astype(np.int32), ci)


@pytest.mark.parametrize("n", [4_194_304, 4_194_320])
def test_converter_bitmap_limit(gpu, n):
    # 4,194,304 nodes = 262,144 block columns: the widest graph whose block
    # columns fit the persistent kernel's LDS bitmap (8,192 words); one more
    # window sends every window through the per-window kernel instead.
    # Hub rows (> 1,024 edges per window) exercise the hub launch as well.
    r = rng(12)
    deg = r.integers(0, 3, n)
    deg[:64] += 200                      # four hub windows
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(deg)
    ci = r.integers(0, n, int(rp[-1])).astype(np.int32)
    ci[rp[:64]] = n - 1                  # last block column
    check_converter(gpu, rp.astype(np.int32), ci)


def test_converter_offsets_past_2m_windows(gpu):
    # 34,000,000 nodes = 2,125,000 windows: more than 1,024 blocks of 2,048
    # window counts, so the count call scans the block sums in a launch of
    # their own before writing the offsets (below that, each block adds up
    # its predecessors' sums itself); a few thousand edges, spread over the
    # whole column range, with repeats and a hub window.
    n = 34_000_000
    r = rng(13)
    rows = np.sort(r.integers(0, n, 6000))
    rows = np.concatenate([rows, np.full(1500, 16 * 1_000_003)])   # one hub window
    rows.sort()
    deg = np.bincount(rows, minlength=n)
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(deg)
    ci = r.integers(0, n, int(rp[-1])).astype(np.int32)
    ci[::7] = ci[0]                                             # repeated columns
    check_converter(gpu, rp.astype(np.int32), ci)


def test_converter_unsorted_and_empty_windows(gpu):
    n = 64
    rows = {0: [63, 1, 17, 1, 63], 5: [0, 0], 48: [47, 3, 62, 16], 63: [63]}
    rp = np.zeros(n + 1, np.int32)
    ci = []
    for u in range(n):
        ci += rows.get(u, [])
        rp[u + 1] = len(ci)
    check_converter(gpu, rp, np.array(ci, np.int32))


def test_converter_rejects_bad_csr(gpu):
    rp = np.array([0, 2, 3], np.int32)
    with pytest.raises(gpu.F3SError) as e:
        gpu.convert_device(gpu.DeviceCSR(rp, np.array([1, 2, 0], np.int32)))   # col 2 >= n
    assert e.value.name == "F3S_EDATA"
    with pytest.raises(gpu.F3SError) as e:
        gpu.convert_device(gpu.DeviceCSR(np.array([0, 3, 2], np.int32),
                                         np.array([0, 1, 1], np.int32)))        # not monotone
    assert e.value.name == "F3S_EDATA"


def test_converter_offsets_mismatch_is_rejected(gpu):
    from fused3s_amd import _lib
    rp, ci = random_csr(100, 5, 1)
    csr = gpu.DeviceCSR(rp, ci)
    W = 7
    offs = gpu.DeviceArray.from_numpy(np.zeros(W + 1, np.int32))   # wrong: all zero
    bcol = gpu.DeviceArray(1000, np.int32)
    T = C.c_int64()
    st = _lib.hip().f3s_convert_csr_to_bsf(csr.row_ptr.ptr, csr.col_idx.ptr, 100, len(ci),
                                           offs.ptr, bcol.ptr, None, C.byref(T), None)
    assert st == 1   # F3S_EINVAL


def test_window_order_device(gpu):
    for rp, ci in (gpu.CONFIGS[2].graph(), random_csr(5000, 9, 3)):
        bsf = gpu.convert_device(gpu.DeviceCSR(rp, ci))
        got = gpu.window_order_device(bsf).numpy()
        want = orc.window_order(bsf.window_offsets.numpy())
        assert np.array_equal(got, want)


def test_bsf_stats(gpu):
    rp, ci = gpu.CONFIGS[3].graph()
    bsf = gpu.convert_device(gpu.DeviceCSR(rp, ci))
    hb = bsf.to_host()
    want_m = orc.bsf_occupancy(bsf.n, hb.block_col_indices, hb.tile_masks, True)
    want_d = orc.bsf_occupancy(bsf.n, hb.block_col_indices, hb.tile_masks, False)
    assert gpu.bsf_stats(bsf, True) == want_m
    assert gpu.bsf_stats(bsf, False)[0] == want_d[0]


# -------------------------------------------------------------- attention

@pytest.mark.parametrize("name", ["cora", "citeseer"])
@pytest.mark.parametrize("masked", [True, False])
def test_attention_fixtures(gpu, name, masked):
    g = gpu.load_csr_graph(str(GOLDEN / name))
    p = Problem(gpu, g.row_ptr, g.col_ind, seed=1)
    want = p.oracle(masked)
    for planned, compiled in ((False, False), (True, False), (True, True)):
        got = p.run(masked, planned=planned, seg=16, compiled=compiled and masked)
        assert_close(got, want, f"{name} masked={masked} planned={planned} compiled={compiled}")


@pytest.mark.parametrize("cfg", [2, 3])
@pytest.mark.parametrize("masked", [True, False])
def test_attention_configs_small(gpu, cfg, masked):
    c = gpu.CONFIGS[cfg]
    rp, ci = c.graph()
    p = Problem(gpu, rp, ci, H=c.H, normal=c.normal, seed=cfg)
    want = p.oracle(masked)
    order = gpu.window_order_device(p.bsf)
    for planned, seg, compiled in ((False, 0, False), (True, 0, False), (True, 8, False),
                                   (True, 0, True), (True, 8, True)):
        got = p.run(masked, planned=planned, seg=seg, order=order, compiled=compiled and masked)
        assert_close(got, want, f"cfg{cfg} masked={masked} planned={planned} seg={seg} "
                                f"compiled={compiled}")


@pytest.mark.parametrize("H", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("n,deg,seed", [(1, 0, 1), (37, 5, 2), (500, 12, 3), (2050, 60, 4)])
def test_attention_random_heads(gpu, H, n, deg, seed):
    rp, ci = random_csr(n, deg, seed, self_loops=(seed % 2 == 0))
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=seed)
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        for planned, compiled in ((False, False), (True, False), (True, True)):
            got = p.run(masked, planned=planned, seg=4, scale=0.125, compiled=compiled and masked)
            assert_close(got, want, f"n={n} H={H} masked={masked} planned={planned} "
                                    f"compiled={compiled}")


@pytest.mark.parametrize("H", [33, 64])
@pytest.mark.parametrize("n,deg,seed", [(37, 5, 5), (500, 12, 6)])
def test_attention_many_heads(gpu, H, n, deg, seed):
    # up to the 64 heads the API accepts (and an odd count past 32), every
    # launch shape, both semantics
    rp, ci = random_csr(n, deg, seed, self_loops=True)
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=seed)
    order = gpu.window_order_device(p.bsf)
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        for planned, compiled in ((False, False), (True, False), (True, True)):
            got = p.run(masked, planned=planned, seg=4, scale=0.125, compiled=compiled and masked)
            assert_close(got, want, f"n={n} H={H} masked={masked} planned={planned} "
                                    f"compiled={compiled}")
        got = p.run(masked, order=order, scale=0.125)
        assert_close(got, want, f"n={n} H={H} masked={masked} ordered")


@pytest.mark.parametrize("case,H,team_m,team_d", [("random", 1, 4, 16), ("random", 4, 4, 4),
                                                 ("random", 8, 1, 4), ("random", 16, 1, 1),
                                                 ("star", 1, 4, 16), ("star", 3, 4, 4)])
def test_attention_teams(gpu, case, H, team_m, team_d):
    # Small graphs run each window on a team of waves that merge in LDS:
    # masked, 4 waves while W*H <= 1024; tile-dense, 16 while W*H <= 512 and
    # 4 up to 2048.  The unplanned launch and an automatic plan make the same
    # items (same bits, with or without compiled lists, in any window order);
    # both meet the oracle.
    rp, ci = random_csr(3000, 10, 41) if case == "random" else star_graph(5000, hubs=(0, 7))
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=41)
    W = (p.n + 15) // 16
    plan = gpu.Plan(p.bsf, None, H=H)
    if team_m > 1:   # plan_info describes the masked item set
        assert plan.num_items == W * team_m and plan.num_split == 0
    else:
        assert plan.num_items < W * 4
    order = gpu.window_order_device(p.bsf)
    for masked in (True, False):
        team = team_m if masked else team_d
        want = p.oracle(masked, scale=0.125)
        base = p.run(masked, scale=0.125)
        assert_close(base, want, f"{case} H={H} team={team} masked={masked}")
        variants = [("planned", dict(planned=True)), ("ordered", dict(order=order)),
                    ("planned+ordered", dict(planned=True, order=order))]
        if masked:
            variants.append(("compiled", dict(planned=True, compiled=True)))
        for what, kw in variants:
            got = p.run(masked, scale=0.125, **kw)
            if team > 1:
                assert np.array_equal(got.view(np.uint32), base.view(np.uint32)), what
            else:
                assert_close(got, want, f"{case} H={H} masked={masked} {what}")


def test_attention_hub_split_merge(gpu):
    rp, ci = star_graph(20000, hubs=(0, 3, 17))
    p = Problem(gpu, rp, ci, H=1, normal=True, seed=9)
    want = p.oracle(True)
    for seg in (0, 64, 1000):
        for compiled in (False, True):
            got = p.run(True, planned=True, seg=seg, compiled=compiled)
            assert_close(got, want, f"star seg={seg} compiled={compiled}")
    # tile-dense passes of an automatic plan run its finer item set
    want_d = p.oracle(False)
    for seg in (0, 64):
        assert_close(p.run(False, planned=True, seg=seg), want_d, f"star tile-dense seg={seg}")
    got = p.run(True, planned=False)
    assert_close(got, want, "star unplanned")


def test_attention_closed_forms(gpu):
    # Q = 0: every row is the mean of V over its neighbours; rows with no
    # edge (no self-loops here) are exactly 0.
    n = 300
    rp, ci = random_csr(n, 4, 5, self_loops=False)
    p = Problem(gpu, rp, ci, seed=2, Qzero=True)
    got = p.run(True)[:, 0]
    deg = np.diff(rp)
    for u in range(n):
        if deg[u] == 0:
            assert np.all(got[u] == 0)
        else:
            assert np.allclose(got[u], p.Vf[ci[rp[u]:rp[u + 1]], 0].mean(axis=0), atol=1e-3)
    # self-loop only: O = V
    rp1 = np.arange(n + 1, dtype=np.int32)
    p1 = Problem(gpu, rp1, np.arange(n, dtype=np.int32), seed=3)
    assert np.array_equal(p1.run(True)[:, 0], p1.Vf[:, 0])
    # Q = K = V with identical rows: equal weights, so every row with a
    # neighbour (masked) or with a tile (tile-dense) is that row
    p2 = Problem(gpu, rp, ci, H=2, seed=4)
    x = p2.Q[0].copy()
    for a in (p2.Q, p2.K, p2.V):
        a[:] = x
    for d, a in zip((p2.dQ, p2.dK, p2.dV), (p2.Q, p2.K, p2.V)):
        d.upload(a.view(np.uint16))
    tiles = np.diff(p2.bsf.window_offsets.numpy())
    for masked in (True, False):
        has = deg > 0 if masked else np.repeat(tiles > 0, 16)[:n]
        for planned in (False, True):
            got = p2.run(masked, planned=planned, seg=4)
            assert np.allclose(got[has], x.astype(np.float32), rtol=1e-6, atol=1e-7)
            assert np.all(got[~has] == 0)
    # tile-dense with K = 0: every row is the mean of V over its window's
    # tile columns < n
    p3 = Problem(gpu, rp, ci, seed=6)
    p3.K[:] = 0
    p3.dK.upload(p3.K.view(np.uint16))
    hb = p3.host_bsf()
    got = p3.run(False)[:, 0]
    for w in range((n + 15) // 16):
        b = hb.block_col_indices[hb.window_offsets[w]:hb.window_offsets[w + 1]]
        cols = (b[:, None] * 16 + np.arange(16)).ravel()
        cols = cols[cols < n]
        want = p3.Vf[cols, 0].mean(axis=0) if len(cols) else np.zeros(64, np.float32)
        assert np.allclose(got[16 * w:16 * w + 16], want, atol=1e-3)


def test_attention_wide_logit_range(gpu):
    # Q and K drawn with standard deviation 4 (logits of standard deviation
    # ~128, most rows' softmax close to one-hot; the running max moves by
    # hundreds between chunks) and a scale of 0 (every weight equal: O is the
    # plain mean of V over the attended columns), against the oracle, every
    # launch shape, both semantics.
    rp, ci = random_csr(2000, 24, 14, self_loops=True)
    p = Problem(gpu, rp, ci, H=2, normal=True, seed=14)
    r = rng(15)
    for a, d in ((p.Q, p.dQ), (p.K, p.dK)):
        a[:] = (r.standard_normal(a.shape) * 4).astype(np.float16)
        d.upload(a.view(np.uint16))
    p.Qf, p.Kf = p.Q.astype(np.float32), p.K.astype(np.float32)
    for scale in (1.0, 0.0):
        for masked in (True, False):
            want = p.oracle(masked, scale=scale)
            for planned, compiled in ((False, False), (True, False), (True, True)):
                got = p.run(masked, planned=planned, seg=4, scale=scale,
                            compiled=compiled and masked)
                assert_close(got, want, f"wide logits scale={scale} masked={masked} "
                                        f"planned={planned} compiled={compiled}")


def test_padded_buffers_with_nan_padding(gpu):
    # The reference's buffers have 16W rows, padded (tests/test_fused_3s_v2.cu:
    # 93-120).  Given such buffers whose padding rows hold NaN, the pass
    # reads none of them (loads past n rows return 0; padded columns are
    # excluded, as on the reference's CPU side) and writes none: rows < n
    # match the oracle, rows >= n keep what they held.
    n = 16 * 50 + 5
    W = (n + 15) // 16
    rp, ci = random_csr(n, 10, 16, self_loops=True)
    p = Problem(gpu, rp, ci, H=2, normal=True, seed=16)
    nan16 = np.full((16 * W - n, 2, 64), 0x7E00, np.uint16)
    pads = [gpu.DeviceArray.from_numpy(np.concatenate([a.view(np.uint16), nan16]))
            for a in (p.Q, p.K, p.V)]
    dO = gpu.DeviceArray((16 * W, 2, 64), np.float32)
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        runs = {
            "drop-in": lambda: gpu.attention_fwd(*pads, dO, p.bsf, None, masked=masked, H=2,
                                                 scale=0.125),
            "plan": lambda: gpu.Plan(p.bsf, None, H=2).forward(*pads, dO, masked=masked,
                                                               scale=0.125),
        }
        for what, fn in runs.items():
            dO.fill_bytes(0xFF)
            fn()
            gpu.synchronize()
            got = dO.numpy()
            assert_close(got[:n], want, f"padded buffers, {what}, masked={masked}")
            assert np.all(got[n:].view(np.uint32) == 0xFFFFFFFF), (what, masked)


@pytest.mark.parametrize("H", [1, 3])
def test_plan_split_merge_state_across_passes(gpu, H):
    # Split windows merge inside the launch: the last segment of a window to
    # finish merges the partials and resets the window's arrival count.  One
    # plan (both item sets share its partials and counts) serves masked and
    # tile-dense passes in turn; every pass must give the first pass's bits
    # on every row (a count left non-zero would leave its window's rows NaN)
    # and meet the oracle.
    rp, ci = star_graph(6000, hubs=(0, 5, 2999))
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=47)
    plan = gpu.Plan(p.bsf, gpu.window_order_device(p.bsf), H=H, seg_tiles=48)
    plan.compile()
    assert plan.num_split > 0
    first = {}
    for rep in range(3):
        for masked in (True, False, True):
            p.dO.fill_bytes(0xFF)
            plan.forward(p.dQ, p.dK, p.dV, p.dO, masked=masked, scale=0.125)
            gpu.synchronize()
            got = p.dO.numpy()
            if masked not in first:
                assert_close(got, p.oracle(masked, scale=0.125),
                             f"split merge, H={H}, masked={masked}")
                first[masked] = got
            assert np.array_equal(got.view(np.uint32), first[masked].view(np.uint32)), \
                (H, rep, masked)


def test_attention_deterministic(gpu):
    rp, ci = star_graph(5000, hubs=(1,))
    p = Problem(gpu, rp, ci, normal=True, seed=4)
    a = p.run(True, planned=True, seg=32)
    b = p.run(True, planned=True, seg=32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    c = p.run(True, planned=True, seg=32, compiled=True)
    d = p.run(True, planned=True, seg=32, compiled=True)
    assert np.array_equal(c.view(np.uint32), d.view(np.uint32))
    # the compiled list visits the columns in the ring's order: same bits
    assert np.array_equal(a.view(np.uint32), c.view(np.uint32))


@pytest.mark.parametrize("H", [4, 8])
def test_padding_slots_read_nothing(gpu, H):
    # Chunk padding must read zeros, never a real row: with V of node 0 set
    # to NaN, only windows that gather node 0 may see it (a gathered column
    # is shared by the window's rows, and 0 * NaN is NaN).  A padding offset
    # plus a large head offset once wrapped around 2^32 onto node 0's row.
    rp, ci = random_csr(700, 7, 31)
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=31)
    p.V[0] = np.float16(np.nan)
    p.Vf = p.V.astype(np.float32)
    p.dV.upload(p.V.view(np.uint16))
    n = p.n
    rows = np.repeat(np.arange(n), np.diff(rp))
    touched = np.zeros((n + 15) // 16, bool)
    touched[rows[ci == 0] // 16] = True               # masked: a row attends node 0
    for masked in (True, False):
        want = p.oracle(masked)
        win = touched if masked else ~np.isfinite(want).reshape(n, -1).all(1)[::16]
        ok = ~np.repeat(win, 16)[:n]
        assert ok.any() and not ok.all()
        for planned, compiled in ((False, False), (True, False), (True, True)):
            got = p.run(masked, planned=planned, compiled=compiled and masked)
            assert np.all(np.isfinite(got[ok])), f"H={H} masked={masked} planned={planned}"
            assert np.all(np.isfinite(want[ok]))
            mabs = float(np.abs(got[ok] - want[ok]).max())
            assert mabs <= ABS_TOL, f"H={H} masked={masked} planned={planned}: {mabs}"


def test_attention_timed_entry(gpu):
    rp, ci = random_csr(3000, 9, 33)
    p = Problem(gpu, rp, ci, H=2, seed=33)
    for masked in (True, False):
        want = p.run(masked)
        p.dO.fill_bytes(0xFF)
        us = gpu.attention_fwd_timed(p.dQ, p.dK, p.dV, p.dO, p.bsf, masked=masked, H=2, reps=5)
        assert us > 0.0
        assert np.array_equal(p.dO.numpy().view(np.uint32), want.view(np.uint32))
        log(f"  timed masked={masked}: {us:.1f} us per pass")


def test_concurrent_streams_and_threads(gpu):
    # Two host threads, each with its own stream, plan and output, run
    # passes at the same time; each result equals a single-threaded run.
    import threading
    rp, ci = star_graph(6000, hubs=(2, 9))
    p = Problem(gpu, rp, ci, H=2, normal=True, seed=35)
    want = p.run(True, planned=True, seg=64, compiled=True)
    outs, errs = {}, []

    def worker(k):
        try:
            st = gpu.Stream()
            plan = gpu.Plan(p.bsf, None, H=2, seg_tiles=64, stream=st)
            plan.compile(st)
            dO = gpu.DeviceArray((p.n, 2, 64), np.float32)
            for _ in range(10):
                plan.forward(p.dQ, p.dK, p.dV, dO, masked=True, stream=st)
            st.synchronize()
            outs[k] = dO.numpy()
        except Exception as e:   # surfaced in the main thread
            errs.append(e)

    th = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not errs, errs
    for k in range(2):
        assert np.array_equal(outs[k].view(np.uint32), want.view(np.uint32))


def test_concurrent_converter_and_natural_order_launch(gpu):
    # Two host threads, each with its own stream, convert their own graph and
    # run unplanned natural-order passes (whose heavy-window list lives in
    # stream-ordered scratch) at the same time; every result equals a
    # single-threaded run, and each thread's tile lists match the oracle.
    import threading
    graphs = [star_graph(20000, hubs=(0, 3, 17, 9000)), star_graph(24000, hubs=(5, 12000))]
    probs = [Problem(gpu, rp, ci, H=1, normal=True, seed=71 + k) for k, (rp, ci) in enumerate(graphs)]
    wants = [p.run(True) for p in probs]
    results, errs = {}, []

    def worker(k):
        try:
            p = probs[k]
            st = gpu.Stream()
            bsf = gpu.convert_device(gpu.DeviceCSR(p.rp, p.ci, st), stream=st)
            dO = gpu.DeviceArray((p.n, 1, 64), np.float32)
            for _ in range(5):
                gpu.attention_fwd(p.dQ, p.dK, p.dV, dO, bsf, None, masked=True, H=1, stream=st)
            st.synchronize()
            results[k] = (bsf.to_host(), dO.numpy())
        except Exception as e:   # surfaced in the main thread
            errs.append(e)

    th = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not errs, errs
    for k, p in enumerate(probs):
        hb, out = results[k]
        offs, bcol, mask = orc.convert(p.n, p.rp, p.ci)
        assert np.array_equal(hb.window_offsets, offs)
        assert np.array_equal(hb.block_col_indices, bcol)
        assert np.array_equal(hb.tile_masks, mask)
        assert np.array_equal(out.view(np.uint32), wants[k].view(np.uint32))


def test_schedule_scratch_outlives_its_launches(gpu):
    # Two natural-order drop-in calls on two streams, back to back with no
    # synchronisation, on two graphs of the same size (so the second call's
    # schedule scratch is the block the first returned to the allocator) but
    # different edges (so their schedules differ): the first call's scratch
    # must go back only after its last launch, or the second call's schedule
    # overwrites the slots the first call's one-wave launch still reads.  The
    # first call is tile-dense (a long launch whose later waves start late),
    # the second masked (short).  Every result equals a call run alone.
    # (A build that returned the scratch before the last launch was enqueued
    # also passed here: the race needs the second stream's schedule kernels
    # to run while the first launch still starts waves, which this run never
    # showed; the ordering itself is shown by reading attention_fwd_impl.)
    n = 200_000
    probs = []
    for k in range(2):
        r = rng(90 + k)
        m = 8 * n
        u, v = r.integers(0, n, m), r.integers(0, n, m)
        if k == 1:
            v = (u + r.integers(0, 4096, m)) % n          # local edges: other tile counts
        key = np.unique(np.concatenate([u, v, np.arange(n)]).astype(np.int64) * n +
                        np.concatenate([v, u, np.arange(n)]))
        rp = np.zeros(n + 1, np.int64)
        np.add.at(rp, key // n + 1, 1)
        probs.append(Problem(gpu, np.cumsum(rp).astype(np.int32), (key % n).astype(np.int32),
                             H=1, seed=92 + k))
    sems = (False, True)
    wants = [p.run(m) for p, m in zip(probs, sems)]
    streams = [gpu.Stream(), gpu.Stream()]
    outs = [gpu.DeviceArray((n, 1, 64), np.float32) for _ in range(2)]
    for rep in range(4):
        for k in range(2):
            outs[k].fill_bytes(0xFF)
        gpu.synchronize()
        for k in range(2):
            p = probs[k]
            gpu.attention_fwd(p.dQ, p.dK, p.dV, outs[k], p.bsf, None, masked=sems[k], H=1,
                              stream=streams[k])
        gpu.synchronize()
        for k in range(2):
            got = outs[k].numpy()
            assert np.array_equal(got.view(np.uint32), wants[k].view(np.uint32)), (rep, k)


def test_unplanned_heavy_windows(gpu):
    # Without a plan, windows of more than max(1024, 8 x mean) tiles run as
    # 16-wave teams in a launch of their own -- in natural order (the
    # library's schedule) the first 512 such windows, heaviest first; given a
    # window order on a launch this size (under 2^18 window-heads), those
    # among its first 512 entries -- and every other window on one wave.
    # Hubs sit in windows 0, 1 and 562 (1,250 tiles each); the orders put
    # them first (sorted) or at positions 700, 5 and 100 (one past 512).
    rp, ci = star_graph(20000, hubs=(0, 3, 17, 9000))
    p = Problem(gpu, rp, ci, H=2, normal=True, seed=61)
    W = p.bsf.W
    offs = p.bsf.window_offsets.numpy()
    tiles = np.diff(offs)
    thr = max(1024, 8 * ((int(offs[-1]) + W - 1) // W))
    heavy = np.nonzero(tiles > thr)[0]
    assert list(heavy) == [0, 1, 562]
    perm = rng(62).permutation(W).astype(np.int32)
    for w, pos in ((0, 700), (1, 5), (562, 100)):      # move the hubs to chosen positions
        j = int(np.nonzero(perm == w)[0][0])
        perm[j], perm[pos] = perm[pos], perm[j]
    orders = {"natural": None, "sorted": gpu.window_order_device(p.bsf),
              "moved": gpu.DeviceArray.from_numpy(perm)}
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        got_by = {}
        for name, order in orders.items():
            got = p.run(masked, order=order, scale=0.125)
            assert_close(got, want, f"unplanned heavy windows masked={masked} order={name}")
            got_by[name] = got
        # natural and sorted orders give all three hubs to teams: same bits
        assert np.array_equal(got_by["natural"].view(np.uint32), got_by["sorted"].view(np.uint32))


@pytest.mark.parametrize("H", [2, 4])
def test_unplanned_schedule_without_heavy_windows(gpu, H):
    # 800 windows: past the 512 from which the drop-in launch runs its
    # schedule, but no window can hold more than 800 tiles (one per block
    # column), under the 1,024 a heavy window needs, so the launch skips the
    # team launch; given an order, one wave per entry.  Every window runs
    # whole on one wave either way: same bits, within the oracle's bar.
    rp, ci = random_csr(16 * 800, 6, 71, self_loops=True)
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=71)
    assert p.bsf.W == 800
    order = gpu.window_order_device(p.bsf)
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        nat = p.run(masked, scale=0.125)
        srt = p.run(masked, order=order, scale=0.125)
        assert_close(nat, want, f"no heavy windows, natural order, H={H} masked={masked}")
        assert np.array_equal(nat.view(np.uint32), srt.view(np.uint32)), (H, masked)


def test_unplanned_schedule_names_windows(gpu):
    # From 2^18 window-heads on (plans and the drop-in launch alike), a window
    # order only names the windows to compute, and the library's schedule
    # runs them: invalid entries are skipped, a repeated
    # window is computed once, windows the order does not name are left
    # untouched, and every order gives the bits of a natural-order call.  4,096 windows x 64 heads; the hub windows 0, 2
    # and 2,062 (rows of 3,000 random neighbours, over 1,024 tiles) take the
    # team launch wherever the order puts them.
    n, H = 65536, 64
    r = rng(66)
    rows = [np.arange(n), np.repeat(np.arange(n), 3)]
    cols = [np.arange(n), r.integers(0, n, 3 * n)]
    for hub in (0, 40, 33000):
        rows.append(np.full(3000, hub))
        cols.append(r.integers(0, n, 3000))
    key = np.unique(np.concatenate(rows).astype(np.int64) * n + np.concatenate(cols))
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, key // n + 1, 1)
    rp, ci = np.cumsum(rp).astype(np.int32), (key % n).astype(np.int32)
    p = Problem(gpu, rp, ci, H=H, seed=64, f32=True)
    W = p.bsf.W
    tiles = np.diff(p.bsf.window_offsets.numpy())
    thr = max(1024, 8 * (-(-int(tiles.sum()) // W)))
    assert W * H >= 1 << 18 and list(np.nonzero(tiles > thr)[0]) == [0, 2, 2062]
    r = rng(65)
    perm = r.permutation(W).astype(np.int32)
    order = perm.copy()
    k = np.arange(0, W, 7)
    order[k] = np.where(k % 3 == 0, -2, np.where(k % 3 == 1, W + 9, order[(k + 1) % W]))
    named = np.zeros(W, bool)
    named[order[(order >= 0) & (order < W)]] = True
    for hub in (0, 2, 2062):     # keep the hub windows named, late in the order
        if not named[hub]:
            order[int(np.nonzero(order == -2)[0][-1])] = hub
            named[hub] = True
    valid = order[(order >= 0) & (order < W)]
    assert (~named).any() and len(set(valid.tolist())) < len(valid)     # some repeat
    rows = np.repeat(named, 16)[:n]
    # oracle windows: every 61st named window, and the hub windows when masked
    sample = sorted(set(np.nonzero(named)[0][::61].tolist()) - {0, 2, 2062})
    dperm, dorder = gpu.DeviceArray.from_numpy(perm), gpu.DeviceArray.from_numpy(order)
    for masked in (True, False):
        full = p.run(masked)
        shuffled = p.run(masked, order=dperm)
        assert np.array_equal(shuffled.view(np.uint32), full.view(np.uint32)), masked
        got = p.run(masked, order=dorder)
        what = f"partial order, scheduled, masked={masked}"
        assert np.all(np.isnan(got[~rows])), what
        assert np.array_equal(got[rows].view(np.uint32), full[rows].view(np.uint32)), what
        # the allocation-free entry point: the order's inverse in its fixed scratch
        from fused3s_amd import _lib
        p.dO.fill_bytes(0xFF)
        bsf = p.bsf
        assert _lib.hip().f3s_attention_fwd_noalloc(
            p.dQ.ptr, p.dK.ptr, p.dV.ptr, p.dO.ptr, bsf.window_offsets.ptr, bsf.block_col.ptr,
            bsf.tile_mask.ptr if masked else None, dorder.ptr, W, n, 64, H, 1.0, None) == 0
        gpu.synchronize()
        assert np.array_equal(p.dO.numpy().view(np.uint32), got.view(np.uint32)), what
        ranges = [(16 * w, 16 * w + 16) for w in (sample + [0, 2, 2062] if masked else sample)]
        want = p.oracle(masked, rows=ranges)
        assert_close(np.concatenate([got[a:b] for a, b in ranges]),
                     np.concatenate([want[r] for r in ranges]), what)
        # plans of a graph this size follow the same schedule (hub windows
        # split into segments instead of teams): any order names the windows
        pfull = p.run(masked, planned=True, compiled=masked)
        pperm = p.run(masked, planned=True, order=dperm, compiled=masked)
        ppart = p.run(masked, planned=True, order=dorder, compiled=masked)
        assert np.array_equal(pperm.view(np.uint32), pfull.view(np.uint32)), what
        assert np.all(np.isnan(ppart[~rows])), what
        assert np.array_equal(ppart[rows].view(np.uint32), pfull[rows].view(np.uint32)), what
        assert_close(np.concatenate([pfull[a:b] for a, b in ranges]),
                     np.concatenate([want[r] for r in ranges]), what + " planned")


def test_unplanned_natural_order_heavy_cap(gpu):
    # The schedule's classes (natural order): 4,200 windows (every 4th of
    # 16,800) hold exactly 600 tiles, a class of their own ([512, 1024)
    # tiles) that the one-wave launch starts first, cut into eight XCD
    # shares; the threshold for teams, max(1024, 8 x mean) = 1,208 tiles,
    # takes none of them.  The class spans all 17 of the schedule's
    # 1,024-window blocks (256 windows in each but the last).  The sorted
    # order runs in its own sequence (no team either).  Results meet the
    # oracle, both orders give the same bits, and repeated runs too.
    W = 16_800
    n = 16 * W
    heavy_w = np.arange(4200) * 4
    rows, cols = [np.arange(n)], [np.arange(n)]            # self-loops
    k = np.arange(600, dtype=np.int64)
    for w in heavy_w:
        rows.append(np.full(600, 16 * w))
        cols.append(16 * ((k * 7919 + w) % W) + (w % 16))   # 600 distinct block columns
    e = np.unique(np.stack([np.concatenate(rows), np.concatenate(cols)], 1), axis=0)
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, e[:, 0] + 1, 1)
    rp = np.cumsum(rp).astype(np.int32)
    ci = e[:, 1].astype(np.int32)
    p = Problem(gpu, rp, ci, H=2, normal=True, seed=63)
    offs = p.bsf.window_offsets.numpy()
    tiles = np.diff(offs)
    mean = (int(offs[-1]) + W - 1) // W
    assert np.array_equal(np.nonzero(tiles > max(512, 2 * mean))[0], heavy_w)
    assert not np.any(tiles > max(1024, 8 * mean))
    sorted_order = gpu.window_order_device(p.bsf)
    for masked in (True, False):
        want = p.oracle(masked)
        a = p.run(masked)
        b = p.run(masked)
        s = p.run(masked, order=sorted_order)
        assert_close(a, want, f"natural order, 4,200 heavy windows, masked={masked}")
        assert_close(s, want, f"sorted order, masked={masked}")
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert np.array_equal(a.view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("H", [1, 16])
def test_window_order_with_invalid_entries(gpu, H):
    # A caller's window order may name invalid windows (< 0 or >= W): they
    # are skipped, the windows it does not name are left unwritten, and the
    # named ones are exact -- with teams (H = 1) and without (H = 16), planned
    # or not.
    rp, ci = random_csr(3000, 8, 51)
    p = Problem(gpu, rp, ci, H=H, normal=True, seed=51)
    W = (p.n + 15) // 16
    order = rng(52).permutation(W).astype(np.int32)
    dropped = order[::5].copy()
    order[::5] = np.where(np.arange(len(dropped)) % 2 == 0, -1, W + 3)
    dorder = gpu.DeviceArray.from_numpy(order)
    named = np.ones(W, bool)
    named[dropped] = False
    rows = np.repeat(named, 16)[:p.n]
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        for planned, compiled in ((False, False), (True, False), (True, True)):
            got = p.run(masked, planned=planned, order=dorder, scale=0.125,
                        compiled=compiled and masked)
            what = f"invalid order H={H} masked={masked} planned={planned} compiled={compiled}"
            assert np.all(np.isnan(got[~rows])), what
            assert_close(got[rows], want[rows], what)


def test_attention_chunk_boundaries(gpu):
    # Masked passes take a window's attended columns 32 at a time, tile-dense
    # ones its tiles two at a time: windows attending exactly 1, 31, 32, 33,
    # 63, 64, 65, 96, 97, 128 and 129 distinct columns (spread over their 16
    # rows), and so holding from 1 to dozens of tiles, odd and even, against
    # the oracle in both semantics and every launch shape.
    sizes = (1, 31, 32, 33, 63, 64, 65, 96, 97, 128, 129)
    W = 2 * len(sizes)
    n = 16 * W
    r = rng(13)
    rows, cols = [], []
    for k, sz in enumerate(sizes):
        w = 2 * k                                        # windows 0, 2, 4, ...; odd ones empty
        c = r.choice(n, sz, replace=False)
        rows.append(16 * w + (np.arange(sz) % 16))
        cols.append(c)
    rr, cc = np.concatenate(rows), np.concatenate(cols)
    o = np.lexsort((cc, rr))
    rr, cc = rr[o], cc[o]
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rr + 1, 1)
    rp = np.cumsum(rp).astype(np.int32)
    p = Problem(gpu, rp, cc.astype(np.int32), H=2, normal=True, seed=13)
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125)
        for planned, compiled in ((False, False), (True, False), (True, True)):
            got = p.run(masked, planned=planned, seg=0, scale=0.125, compiled=compiled and masked)
            assert_close(got, want, f"chunk boundaries masked={masked} planned={planned} "
                                    f"compiled={compiled}")


@pytest.mark.parametrize("n", [0, 37, 16 * 600])
def test_edgeless_graphs(gpu, n):
    # No edges (and, for n = 0, no nodes): no tiles, and every row of O is
    # exactly 0 in both semantics, through every launch shape -- 600 windows
    # take the drop-in launch's schedule with every window in its lightest
    # class.
    from fused3s_amd import _lib
    rp, ci = np.zeros(n + 1, np.int32), np.zeros(0, np.int32)
    p = Problem(gpu, rp, ci, H=2, seed=5)
    bsf = p.bsf
    assert bsf.T == 0 and bsf.W == (n + 15) // 16
    offs, _, _ = orc.convert(n, rp, ci)
    assert np.array_equal(p.host_bsf().window_offsets, offs)
    order = gpu.window_order_device(bsf) if bsf.W else None
    for masked in (True, False):
        runs = {"natural": p.run(masked), "ordered": p.run(masked, order=order)}
        for planned, compiled in ((True, False), (True, True)):
            if compiled and not masked:
                continue
            runs[f"plan compiled={compiled}"] = p.run(masked, planned=True, compiled=compiled)
        p.dO.fill_bytes(0xFF)
        assert _lib.hip().f3s_attention_fwd_noalloc(
            p.dQ.ptr, p.dK.ptr, p.dV.ptr, p.dO.ptr, bsf.window_offsets.ptr, bsf.block_col.ptr,
            bsf.tile_mask.ptr if masked else None, None, bsf.W, n, 64, 2, 1.0, None) == 0
        gpu.synchronize()
        runs["noalloc"] = p.dO.numpy()
        for what, got in runs.items():
            assert got.shape == (n, 2, 64) and not np.any(got), (n, masked, what)


def test_attention_rejects_bad_args(gpu):
    rp, ci = random_csr(40, 3, 1)
    p = Problem(gpu, rp, ci)
    with pytest.raises(gpu.F3SError) as e:
        gpu.attention_fwd(p.dQ, p.dK, p.dV, p.dO, p.bsf, H=1, d=32)
    assert e.value.name == "F3S_EUNSUPPORTED"
    with pytest.raises(gpu.F3SError) as e:
        gpu.attention_fwd(p.dQ, p.dK, p.dV, p.dO, p.bsf, H=65)
    assert e.value.name == "F3S_EUNSUPPORTED"
    # through the C-ABI: W that does not match n, a feature pointer off its
    # 16-byte alignment, a misaligned mask pointer, a NULL block list -- each
    # an F3S_EINVAL before any launch, with the output untouched
    from fused3s_amd import _lib
    lib = _lib.hip()
    b = p.bsf
    args = dict(Q=p.dQ.ptr, K=p.dK.ptr, V=p.dV.ptr, O=p.dO.ptr, offs=b.window_offsets.ptr,
                cols=b.block_col.ptr, mask=b.tile_mask.ptr, order=None, W=b.W, n=p.n)
    bad = [dict(W=b.W + 1), dict(Q=p.dQ.ptr + 2), dict(O=p.dO.ptr + 4),
           dict(mask=b.tile_mask.ptr + 2), dict(cols=None)]
    for change in bad:
        a = {**args, **change}
        p.dO.fill_bytes(0x7F)
        for fn in (lib.f3s_attention_fwd, lib.f3s_attention_fwd_noalloc):
            st = fn(a["Q"], a["K"], a["V"], a["O"], a["offs"], a["cols"], a["mask"], a["order"],
                    a["W"], a["n"], 64, 1, 1.0, None)
            assert st == 1, (change, fn.__name__, st, lib.f3s_last_error())
        gpu.synchronize()
        assert np.all(p.dO.numpy().view(np.uint32) == 0x7F7F7F7F), change


def test_plan_rejects_bad_args(gpu):
    # a plan's pass with another head count or another n, and a compile
    # without masks or with a misaligned mask pointer: F3S_EINVAL, O untouched
    from fused3s_amd import _lib
    lib = _lib.hip()
    rp, ci = random_csr(200, 5, 17)
    p = Problem(gpu, rp, ci, H=2, seed=17)
    plan = gpu.Plan(p.bsf, None, H=2)
    b = p.bsf
    p.dO.fill_bytes(0x7F)
    for H, n in ((1, p.n), (2, p.n + 16)):
        st = lib.f3s_attention_fwd_planned(plan.handle, p.dQ.ptr, p.dK.ptr, p.dV.ptr, p.dO.ptr,
                                           b.block_col.ptr, b.tile_mask.ptr, n, 64, H, 1.0, None)
        assert st == 1, (H, n, lib.f3s_last_error())
    for mask in (None, b.tile_mask.ptr + 2):
        st = lib.f3s_plan_compile(plan.handle, b.block_col.ptr, mask, p.n, None)
        assert st == 1, lib.f3s_last_error()
    gpu.synchronize()
    assert np.all(p.dO.numpy().view(np.uint32) == 0x7F7F7F7F)
    # and the plan still works after the rejected calls
    got = p.run(True, planned=True, compiled=True)
    assert_close(got, p.oracle(True), "plan after rejected calls")


# ------------------------------------------------------ naive comparator

@pytest.mark.parametrize("case", ["cora", "random", "multigraph"])
def test_naive_comparator(gpu, case):
    """The naive edge-exact GPU comparator (baselines/gpu_baseline.cu) against
    the oracle at the reference's 1e-4 (tests/test_baselines.cu:27),
    including zero-degree rows and duplicate CSR entries (counted twice)."""
    if case == "cora":
        g = gpu.load_csr_graph(str(GOLDEN / "cora"))
        rp, ci = g.row_ptr, g.col_ind
    elif case == "random":
        rp, ci = random_csr(700, 9, 3, self_loops=False)
    else:
        rp = np.array([0, 3, 3, 5, 9], np.int32)
        ci = np.array([1, 1, 2, 0, 0, 3, 3, 3, 1], np.int32)
    n, d = len(rp) - 1, 64
    r = rng(7)
    Q, K, V = (r.uniform(-1, 1, (n, d)).astype(np.float32) for _ in range(3))
    csr = gpu.DeviceCSR(rp, ci)
    dQ, dK, dV = (gpu.DeviceArray.from_numpy(x) for x in (Q, K, V))
    dO = gpu.DeviceArray((n, d), np.float32)
    dO.fill_bytes(0xFF)
    gpu.naive_attention_fwd(dQ, dK, dV, dO, csr, d=d)
    gpu.synchronize()
    want = orc.masked_attention(n, d, 1, Q, K, V, rp, ci)[:, 0]
    got = dO.numpy()
    assert np.max(np.abs(got - want)) <= 1e-4


# ------------------------------------------------- repeated CSR entries

def test_repeated_csr_entries(gpu):
    """A CSR that repeats entries (a multigraph).  The reference converter
    accepts it (its std::set drops the repeats, src/converter.cu:20-29), and
    so does the drop-in converter: the tile lists and masks are those of the
    deduplicated CSR, and `duplicate_entries` (= nnz - mask bits, also
    f3s_bsf_stats') counts the repeats.  As documented, the masked pass then
    attends each edge once -- it equals the oracle on the deduplicated CSR --
    whereas cpu_sparse_attention_csr counts every repeat
    (baselines/cpu_baseline.cpp:38-50), so the rows with repeats differ from
    the oracle on the multigraph; the tile-dense pass is unaffected."""
    n = 600
    rp0, ci0 = random_csr(n, 7, 71)
    r = rng(72)
    reps = r.integers(0, len(ci0), 300)            # entries to repeat (some several times)
    rows0 = np.repeat(np.arange(n), np.diff(rp0))
    rows = np.concatenate([rows0, rows0[reps]])
    cols = np.concatenate([ci0, ci0[reps]])
    key = np.argsort(rows.astype(np.int64) * n + cols, kind="stable")
    rows, cols = rows[key], cols[key].astype(np.int32)
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(np.bincount(rows, minlength=n))
    rp = rp.astype(np.int32)
    dup = len(cols) - len(ci0)
    assert dup == 300
    fmt = gpu.convert_csr_to_block_sparse(n, rp, cols, verbose=False)
    offs, bcol, mask = orc.convert(n, rp0, ci0)
    assert fmt.duplicate_entries == dup
    assert np.array_equal(fmt.window_offsets, offs)
    assert np.array_equal(fmt.block_col_indices, bcol)
    assert np.array_equal(fmt.tile_masks, mask)
    # the oracle converter on the multigraph gives the same lists (and masks)
    offs_m, bcol_m, mask_m = orc.convert(n, rp, cols)
    assert np.array_equal(offs_m, offs) and np.array_equal(bcol_m, bcol)
    assert np.array_equal(mask_m, mask)
    csr = gpu.DeviceCSR(rp, cols)
    bsf = gpu.convert_device(csr)
    occ, bits = gpu.bsf_stats(bsf, True)
    assert bits == len(cols) - dup
    Q, K, V = (r.uniform(-1, 1, (n, 1, 64)).astype(np.float16) for _ in range(3))
    Qf, Kf, Vf = (x.astype(np.float32) for x in (Q, K, V))
    dQ, dK, dV = (gpu.DeviceArray.from_numpy(x.view(np.uint16)) for x in (Q, K, V))
    dO = gpu.DeviceArray((n, 1, 64), np.float32)
    for masked in (True, False):
        dO.fill_bytes(0xFF)
        gpu.attention_fwd(dQ, dK, dV, dO, bsf, None, masked=masked)
        gpu.synchronize()
        got = dO.numpy()
        if masked:
            want = orc.masked_attention(n, 64, 1, Qf, Kf, Vf, rp0, ci0)
            counted_twice = orc.masked_attention(n, 64, 1, Qf, Kf, Vf, rp, cols)
            rep_rows = np.unique(rows0[reps])
            assert np.abs(got[rep_rows] - counted_twice[rep_rows]).max() > 10 * ABS_TOL
            other = np.setdiff1d(np.arange(n), rep_rows)
            assert np.array_equal(want[other].view(np.uint32),
                                  counted_twice[other].view(np.uint32))
        else:
            want = orc.tile_dense_attention(n, 64, 1, Qf, Kf, Vf, offs, bcol, fast=True)
        mabs, mrel = errors(got, want)
        assert mabs <= ABS_TOL and mrel <= REL_TOL, (masked, mabs, mrel)


# ------------------------------------------------- full-size configurations

def oracle_threads() -> int:
    """Host threads for whole-graph oracle runs (a one-GPU box's CPU share)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def errors_chunked(got: np.ndarray, want: np.ndarray, chunk: int = 1 << 24) -> tuple[float, float]:
    """errors() over large arrays in bounded memory: max |g - c| (float64)
    and that over max |c|."""
    g, w = got.reshape(-1), want.reshape(-1)
    mabs, scale = 0.0, 0.0
    for i in range(0, g.size, chunk):
        gi = g[i:i + chunk].astype(np.float64)
        wi = w[i:i + chunk].astype(np.float64)
        mabs = max(mabs, float(np.abs(gi - wi).max()))
        scale = max(scale, float(np.abs(wi).max()))
    return mabs, (mabs / scale if scale > 0 else mabs)


def check_whole_graph(what: str, got: np.ndarray, want: np.ndarray) -> None:
    assert np.all(np.isfinite(got)), f"{what}: unwritten or non-finite rows"
    mabs, mrel = errors_chunked(got, want)
    log(f"  {what}: every row, max_abs={mabs:.3e} max_rel={mrel:.3e} "
        f"(elementwise rel, |c| >= 0.1: {elem_rel(got, want):.3e})")
    assert mabs <= ABS_TOL and mrel <= REL_TOL, f"{what}: {mabs} {mrel}"


@pytest.mark.slow
def test_config4_full_size(gpu):
    """Config 4 at full size: the converter in full; masked attention on every
    row (the oracle of baselines/cpu_baseline.cpp:16-91 over the whole graph,
    as tests/test_fused_3s_v2.cu:141-153 compares every row) for the plan,
    the compiled plan and the drop-in launch in the reference's descending
    order and in natural order; tile-dense attention (the reference kernel's
    semantics, tests/test_fused_3s_v2.cu:17-59: about a TFLOP of tile work
    for the CPU oracle) on every row for the plan and the drop-in launch in
    descending order."""
    c = gpu.CONFIGS[4]
    t0 = time.time()
    rp, ci = c.graph()
    log(f"cfg4 graph: n={len(rp)-1} nnz={len(ci)} ({time.time()-t0:.1f}s)")
    csr = gpu.DeviceCSR(rp, ci)
    bsf = gpu.convert_device(csr)
    check_converter(gpu, rp, ci, bsf)
    log(f"cfg4 converter bit-exact: T={bsf.T}")
    n = c.n
    Q, K, V = (c.features(t) for t in range(3))
    Qf, Kf, Vf = (x.astype(np.float32) for x in (Q, K, V))
    dQ, dK, dV = (gpu.DeviceArray.from_numpy(x.view(np.uint16)) for x in (Q, K, V))
    dO = gpu.DeviceArray((n, 1, 64), np.float32)
    order = gpu.window_order_device(bsf)
    hb = bsf.to_host()
    plan = gpu.Plan(bsf, order, H=1)
    log(f"cfg4 plan: items={plan.num_items} split={plan.num_split} seg={plan.seg_tiles}")
    cplan = gpu.Plan(bsf, order, H=1)
    cplan.compile()

    def run(fn):
        dO.fill_bytes(0xFF)   # NaN poison: every row must be written
        fn()
        gpu.synchronize()
        return dO.numpy()

    th = oracle_threads()
    t0 = time.time()
    want = orc.masked_attention(n, 64, 1, Qf, Kf, Vf, rp, ci, 1.0, threads=th)
    log(f"cfg4 masked oracle, whole graph: {time.time()-t0:.2f}s on {th} threads")
    masked_runs = [
        ("plan", lambda: plan.forward(dQ, dK, dV, dO, masked=True)),
        ("compiled plan", lambda: cplan.forward(dQ, dK, dV, dO, masked=True)),
        ("drop-in, descending order",
         lambda: gpu.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=True)),
        ("drop-in, natural order",
         lambda: gpu.attention_fwd(dQ, dK, dV, dO, bsf, None, masked=True)),
    ]
    for what, fn in masked_runs:
        check_whole_graph(f"cfg4 masked {what}", run(fn), want)
    del want
    t0 = time.time()
    want = orc.tile_dense_attention(n, 64, 1, Qf, Kf, Vf, hb.window_offsets,
                                    hb.block_col_indices, 1.0, threads=th, fast=True)
    log(f"cfg4 tile-dense oracle, whole graph: {time.time()-t0:.2f}s on {th} threads")
    for what, fn in (("plan", lambda: plan.forward(dQ, dK, dV, dO, masked=False)),
                     ("drop-in, descending order",
                      lambda: gpu.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=False))):
        check_whole_graph(f"cfg4 tile-dense {what}", run(fn), want)


@pytest.mark.slow
def test_config5_full_size(gpu):
    """Config 5 at full size (121.9 M edges, 4 heads): the converter in full;
    masked attention on every row for the compiled plan and the drop-in
    launch in natural order; tile-dense attention (15.5 TFLOP of tile work
    for the CPU oracle's SIMD form, ~25 s on 16 threads) on every row for the
    plan and for the reference's own launch -- the drop-in f3s_attention_fwd,
    tile-dense, in the descending order (tests/test_fused_3s_v2.cu:124-153)."""
    c = gpu.CONFIGS[5]
    t0 = time.time()
    rp, ci = c.graph()
    log(f"cfg5 graph: n={len(rp)-1} nnz={len(ci)} ({time.time()-t0:.1f}s)")
    bsf = gpu.convert_device(gpu.DeviceCSR(rp, ci))
    check_converter(gpu, rp, ci, bsf)
    log(f"cfg5 converter bit-exact: T={bsf.T}")
    n, H = c.n, c.H
    Q, K, V = (c.features(t) for t in range(3))
    dQ, dK, dV = (gpu.DeviceArray.from_numpy(x.view(np.uint16)) for x in (Q, K, V))
    dO = gpu.DeviceArray((n, H, 64), np.float32)
    hb = bsf.to_host()
    Qf, Kf, Vf = (x.astype(np.float32) for x in (Q, K, V))
    del Q, K, V
    plan = gpu.Plan(bsf, None, H=H)
    plan.compile()

    def run(fn):
        dO.fill_bytes(0xFF)
        fn()
        gpu.synchronize()
        return dO.numpy()

    th = oracle_threads()
    t0 = time.time()
    want = orc.masked_attention(n, 64, H, Qf, Kf, Vf, rp, ci, 1.0, threads=th)
    log(f"cfg5 masked oracle, whole graph: {time.time()-t0:.2f}s on {th} threads")
    for what, fn in (("compiled plan", lambda: plan.forward(dQ, dK, dV, dO, masked=True)),
                     ("drop-in, natural order",
                      lambda: gpu.attention_fwd(dQ, dK, dV, dO, bsf, None, masked=True, H=H))):
        check_whole_graph(f"cfg5 masked {what}", run(fn), want)
    del want
    t0 = time.time()
    want = orc.tile_dense_attention(n, 64, H, Qf, Kf, Vf, hb.window_offsets,
                                    hb.block_col_indices, 1.0, threads=th, fast=True)
    log(f"cfg5 tile-dense oracle, whole graph: {time.time()-t0:.2f}s on {th} threads")
    order = gpu.window_order_device(bsf)
    for what, fn in (("plan", lambda: plan.forward(dQ, dK, dV, dO, masked=False)),
                     ("drop-in, descending order",
                      lambda: gpu.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=False, H=H))):
        check_whole_graph(f"cfg5 tile-dense {what}", run(fn), want)


@pytest.mark.slow
def test_schedule_on_a_graph_of_550_count_blocks(gpu):
    """9,000,000 nodes (562,500 windows; also past the converter's
    one-bitmap limit): the schedule's class counts span 550 blocks, more
    than sched_scan keeps in registers, so it takes its two-pass segment
    loop.  Masked attention on every row for the drop-in launch in natural
    order (three hub windows of ~20,000 tiles on 16-wave teams) and a
    compiled plan (on the same schedule); the drop-in launch in descending
    order (562,500 window-heads: the schedule too) and the allocation-free
    entry point give the natural-order bits, a plan given the order those of
    a plan without it; tile-dense on every row."""
    from fused3s_amd import _lib
    n = 9_000_000
    r = rng(97)
    rows = [np.arange(n), np.repeat(np.arange(n), 2)]
    cols = [np.arange(n), r.integers(0, n, 2 * n)]
    hubs = (5, 4_500_017, 8_999_999)
    for hub in hubs:
        rows.append(np.full(20000, hub))
        cols.append(r.integers(0, n, 20000))
    key = np.unique(np.concatenate(rows).astype(np.int64) * n + np.concatenate(cols))
    del rows, cols
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(np.bincount(key // n, minlength=n))
    rp, ci = rp.astype(np.int32), (key % n).astype(np.int32)
    del key
    p = Problem(gpu, rp, ci, H=1, seed=98, f32=True)
    bsf = p.bsf
    W = bsf.W
    tiles = np.diff(bsf.window_offsets.numpy())
    thr = max(1024, 8 * (-(-int(tiles.sum()) // W)))
    assert -(-W // 1024) == 550 and list(np.nonzero(tiles > thr)[0]) == [h // 16 for h in hubs]
    log(f"550 count blocks: n={n} nnz={len(ci)} W={W} T={int(tiles.sum())}")
    order = gpu.window_order_device(bsf)
    th = oracle_threads()
    t0 = time.time()
    want = orc.masked_attention(n, 64, 1, p.Qf, p.Kf, p.Vf, rp, ci, 1.0, threads=th)
    log(f"  masked oracle, whole graph: {time.time()-t0:.2f}s on {th} threads")
    nat = p.run(True)
    check_whole_graph("drop-in, natural order", nat, want)
    got = p.run(True, order=order)
    assert np.array_equal(got.view(np.uint32), nat.view(np.uint32)), "descending order"
    p.dO.fill_bytes(0xFF)
    assert _lib.hip().f3s_attention_fwd_noalloc(
        p.dQ.ptr, p.dK.ptr, p.dV.ptr, p.dO.ptr, bsf.window_offsets.ptr, bsf.block_col.ptr,
        bsf.tile_mask.ptr, None, W, n, 64, 1, 1.0, None) == 0
    gpu.synchronize()
    assert np.array_equal(p.dO.numpy().view(np.uint32), nat.view(np.uint32)), "noalloc"
    del got, nat
    pl = p.run(True, planned=True, compiled=True)
    check_whole_graph("compiled plan", pl, want)
    got = p.run(True, planned=True, compiled=True, order=order)
    assert np.array_equal(got.view(np.uint32), pl.view(np.uint32)), "plan, descending order"
    del got, pl, want
    hb = p.host_bsf()
    want = orc.tile_dense_attention(n, 64, 1, p.Qf, p.Kf, p.Vf, hb.window_offsets,
                                    hb.block_col_indices, 1.0, threads=th, fast=True)
    nat = p.run(False)
    check_whole_graph("tile-dense drop-in, natural order", nat, want)
    del want
    got = p.run(False, order=order)
    assert np.array_equal(got.view(np.uint32), nat.view(np.uint32)), "tile-dense, descending"
