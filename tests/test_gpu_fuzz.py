"""Randomised parity sweep (deterministic seeds): graphs of random size and
density with optional hub rows and isolated nodes, converted bit-exactly,
then random head counts and scales through every launch shape -- unplanned in natural, sorted and random window
order, automatic plans (teams on small graphs), plans with small forced
segments, compiled lists -- in both semantics, against the CPU oracle at the
north-star bar (max abs 2e-3, normwise max rel 1e-2).  A second sweep draws
sparser graphs of 513 to 2,000 windows, where the unplanned launch in
natural order runs on the library's schedule (classes of tile count, XCD
shares, a team launch for the heavy windows).
"""
from __future__ import annotations

import numpy as np
import pytest

import _oracle as orc
from conftest import rng

pytestmark = pytest.mark.gpu

ABS_TOL, REL_TOL = 2e-3, 1e-2


def random_graph(r: np.random.Generator, n_range=(1, 6000), deg_max: float = 24.0):
    n = int(r.integers(*n_range))
    deg = float(r.uniform(0, deg_max))
    m = int(n * deg / 2)
    u = r.integers(0, n, m)
    v = r.integers(0, n, m)
    if n > 1 and r.random() < 0.4:                       # hub rows
        for h in r.integers(0, n, int(r.integers(1, 4))):
            k = int(r.integers(n // 4, n))
            u = np.concatenate([u, np.full(k, h)])
            v = np.concatenate([v, r.integers(0, n, k)])
    u, v = np.concatenate([u, v]), np.concatenate([v, u])
    if r.random() < 0.7:
        keep = r.random(n) < 0.9                         # some nodes without a self-loop
        u = np.concatenate([u, np.arange(n)[keep]])
        v = np.concatenate([v, np.arange(n)[keep]])
    key = np.unique(u.astype(np.int64) * n + v)
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, key // n + 1, 1)
    return np.cumsum(rp).astype(np.int32), (key % n).astype(np.int32)


@pytest.mark.parametrize("seed", range(64))
def test_random_parity(gpu, seed):
    r = rng(1000 + seed)
    rp, ci = random_graph(r)
    check_parity(gpu, seed, r, rp, ci, int(r.choice([1, 1, 2, 3, 4])))


@pytest.mark.parametrize("seed", range(12))
def test_random_parity_scheduled(gpu, seed):
    r = rng(5000 + seed)
    rp, ci = random_graph(r, (8208, 32000), 6.0)
    assert (len(rp) - 1 + 15) // 16 > 512
    check_parity(gpu, 5000 + seed, r, rp, ci, int(r.choice([1, 2])))


def check_parity(gpu, seed, r, rp, ci, H):
    n = len(rp) - 1
    scale = float(r.choice([1.0, 0.125, 0.5]))
    Q, K, V = (r.standard_normal((n, H, 64)).astype(np.float16) for _ in range(3))
    bsf = gpu.convert_device(gpu.DeviceCSR(rp, ci))
    dQ, dK, dV = (gpu.DeviceArray.from_numpy(x.view(np.uint16)) for x in (Q, K, V))
    dO = gpu.DeviceArray((n, H, 64), np.float32)
    W = bsf.W
    orders = {"natural": None, "sorted": gpu.window_order_device(bsf),
              "random": gpu.DeviceArray.from_numpy(r.permutation(W).astype(np.int32))}
    seg = int(r.integers(2, 64))
    hb = bsf.to_host()
    offs, bcol, mask = orc.convert(n, rp, ci)   # the converter, bit-exact
    assert np.array_equal(hb.window_offsets, offs)
    assert np.array_equal(hb.block_col_indices, bcol)
    assert np.array_equal(hb.tile_masks, mask)
    f = lambda x: x.astype(np.float32)
    print(f"seed {seed}: n={n} nnz={len(ci)} W={W} T={bsf.T} H={H} scale={scale} seg={seg}",
          flush=True)
    for masked in (True, False):
        if masked:
            want = orc.masked_attention(n, 64, H, f(Q), f(K), f(V), rp, ci, scale)
        else:
            want = orc.tile_dense_attention(n, 64, H, f(Q), f(K), f(V), hb.window_offsets,
                                            hb.block_col_indices, scale, fast=True)
        runs = [(f"unplanned/{k}", None, o, False) for k, o in orders.items()]
        runs += [(f"plan/{k}", 0, o, False) for k, o in orders.items()]
        runs += [("plan/seg", seg, None, False), ("plan/seg/sorted", seg, orders["sorted"], False)]
        if masked:
            runs += [("plan/compiled", 0, None, True), ("plan/seg/compiled", seg, None, True)]
        for what, s, order, compiled in runs:
            dO.fill_bytes(0xFF)
            if s is None:
                gpu.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=masked, H=H, scale=scale)
            else:
                plan = gpu.Plan(bsf, order, H=H, seg_tiles=s)
                if compiled:
                    plan.compile()
                plan.forward(dQ, dK, dV, dO, masked=masked, scale=scale)
            gpu.synchronize()
            got = dO.numpy()
            tag = f"seed {seed} masked={masked} {what}"
            assert np.all(np.isfinite(got)), tag
            diff = np.abs(got.astype(np.float64) - want)
            mabs = float(diff.max()) if diff.size else 0.0
            top = float(np.abs(want).max()) if want.size else 0.0
            mrel = mabs / top if top > 0 else mabs
            assert mabs <= ABS_TOL and mrel <= REL_TOL, f"{tag}: {mabs:.3e} {mrel:.3e}"
