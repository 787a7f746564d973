"""f3s_attention_fwd_noalloc (the allocation-free variant of the drop-in
launch, whose schedule scratch is a fixed device array) against
f3s_attention_fwd on the same inputs: bit-identical outputs, both within the
north-star tolerance of the oracle, over two calls in a row on graphs whose
heavy windows take the schedule's team launch -- the second graph smaller,
so stale scratch from the first call would show -- in both semantics, in
natural order and in an order's sequence; the size limit; and replays from
a captured HIP graph, in natural order and -- with 2^18 window-heads, where
the schedule runs an order's windows and keeps the order's inverse in the
same scratch -- in the reference's descending order.  (That scheduled
launch with a partial order is compared in test_gpu_parity.py's
test_unplanned_schedule_names_windows.)"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import rng
from test_gpu_parity import Problem, assert_close

pytestmark = pytest.mark.gpu


def hub_graph(n: int, seed: int, hubs: dict[int, int]) -> tuple[np.ndarray, np.ndarray]:
    """Random graph (about 8 neighbours per row, self-loops) with some rows
    given `deg` random neighbours: hubs[row] = deg."""
    r = rng(seed)
    rows = [np.repeat(np.arange(n), 8), np.arange(n)]
    cols = [r.integers(0, n, 8 * n), np.arange(n)]
    for row, deg in hubs.items():
        rows.append(np.full(deg, row))
        cols.append(r.integers(0, n, deg))
    key = np.unique(np.concatenate(rows).astype(np.int64) * n + np.concatenate(cols))
    rr, cc = key // n, key % n
    rp = np.zeros(n + 1, np.int64)
    np.add.at(rp, rr + 1, 1)
    return np.cumsum(rp).astype(np.int32), cc.astype(np.int32)


def call(lib_fn, p, masked: bool, order=None) -> np.ndarray:
    p.dO.fill_bytes(0xFF)   # NaN poison: every row must be written
    bsf = p.bsf
    st = lib_fn(p.dQ.ptr, p.dK.ptr, p.dV.ptr, p.dO.ptr, bsf.window_offsets.ptr,
                bsf.block_col.ptr, bsf.tile_mask.ptr if masked else None,
                order.ptr if order is not None else None, bsf.W, bsf.n, 64, p.H, 0.125, None)
    assert st == 0, lib_fn.__name__
    p.f3s.synchronize()
    return p.dO.numpy()


def test_noalloc_matches_allocating_entry_point(gpu):
    from fused3s_amd import _lib
    lib = _lib.hip()
    # 40,000 nodes (2,500 windows) then 20,000 (1,250): both above the 512
    # windows from which the drop-in launch runs its schedule, each with
    # heavy windows (more than max(1024, 8 x mean) tiles, for the team
    # launch) and windows of several tile-count classes
    cases = [(40000, 81, {7: 30000, 9000: 30000, 20011: 1000, 33333: 1200, 39999: 800}, 1),
             (20000, 82, {5: 20000, 6000: 900, 11990: 1100}, 2)]
    for n, seed, hubs, H in cases:
        rp, ci = hub_graph(n, seed, hubs)
        p = Problem(gpu, rp, ci, H=H, normal=True, seed=seed)
        tiles = np.diff(p.host_bsf().window_offsets)
        W = len(tiles)
        mean = -(-int(tiles.sum()) // W)
        large = max(1024, 8 * mean)
        octaves = set(np.floor(np.log2(tiles[tiles > 0])).astype(int).tolist())
        assert W > 512 and (tiles > large).any() and len(octaves) >= 4
        order = gpu.window_order_device(p.bsf)
        for masked in (True, False):
            want = p.oracle(masked, scale=0.125)
            for o in (None, order):
                ref = call(lib.f3s_attention_fwd, p, masked, o)
                got = call(lib.f3s_attention_fwd_noalloc, p, masked, o)
                what = f"noalloc n={n} H={H} masked={masked} ordered={o is not None}"
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), what
                assert_close(got, want, what)


def test_noalloc_past_512_count_blocks(gpu):
    """8,500,000 nodes (a self-loop and one more neighbour per row): 531,250
    windows, so the schedule's class counts span 519 blocks of 1,024 windows,
    past the 512 that sched_scan keeps in registers -- it takes its two-pass
    segment loop.  The allocation-free entry point gives f3s_attention_fwd's
    bits in natural and in descending order, in both semantics, and meets the
    oracle on sampled rows; then a second, smaller graph through the same
    scratch gives that entry point's bits too."""
    from fused3s_amd import _lib
    lib = _lib.hip()
    n = 8_500_000
    i = np.arange(n, dtype=np.int64)
    j = (i * 7919 + 13) % n
    two = j != i
    rp = np.zeros(n + 1, np.int64)
    rp[1:] = np.cumsum(1 + two)
    ci = np.empty(int(rp[-1]), np.int32)
    ci[rp[:-1]] = np.minimum(i, j)
    ci[rp[:-1][two] + 1] = np.maximum(i, j)[two]
    p = Problem(gpu, rp.astype(np.int32), ci, H=1, seed=85, f32=True)
    W = p.bsf.W
    assert W == 531_250 and -(-W // 1024) > 512
    order = gpu.window_order_device(p.bsf)
    ranges = [(a, min(n, a + 64)) for a in range(0, n, n // 24)] + [(n - 40, n)]
    for masked in (True, False):
        want = p.oracle(masked, scale=0.125, rows=ranges)
        nat = call(lib.f3s_attention_fwd, p, masked)
        for o in (None, order):
            got = call(lib.f3s_attention_fwd_noalloc, p, masked, o)
            what = f"noalloc W={W} masked={masked} ordered={o is not None}"
            assert np.array_equal(got.view(np.uint32), nat.view(np.uint32)), what
        for (a, b) in ranges:
            assert_close(nat[a:b], want[(a, b)], f"W={W} masked={masked} rows {a}:{b}")
    del p, nat, got
    rp2, ci2 = hub_graph(20000, 86, {5: 20000, 6000: 900})
    p2 = Problem(gpu, rp2, ci2, H=1, normal=True, seed=86)
    for masked in (True, False):
        ref = call(lib.f3s_attention_fwd, p2, masked)
        got = call(lib.f3s_attention_fwd_noalloc, p2, masked)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), ("second call", masked)


def test_noalloc_rejects_graphs_past_its_scratch(gpu):
    from fused3s_amd import _lib
    lib = _lib.hip()
    W = (1 << 21) + 1
    dummy = 256   # never dereferenced: the size check comes first
    st = lib.f3s_attention_fwd_noalloc(dummy, dummy, dummy, dummy, dummy, dummy, None, None,
                                       W, 16 * W, 64, 1, 1.0, None)
    assert st == 5 and b"2097152" in lib.f3s_last_error()


def replay_matches_eager(gpu, torch, lib, p, masked: bool, order=None) -> None:
    """Captures the allocation-free launch into a graph and replays it three
    times, with eager library work and synchronisations between the replays:
    every replay must reproduce the eager result of the allocating entry
    point bit for bit."""
    bsf = p.bsf
    other = gpu.DeviceArray(p.dO.shape, np.float32)
    args = (p.dQ.ptr, p.dK.ptr, p.dV.ptr, p.dO.ptr, bsf.window_offsets.ptr, bsf.block_col.ptr,
            bsf.tile_mask.ptr if masked else None, order.ptr if order is not None else None,
            bsf.W, bsf.n, 64, p.H, 0.125)
    want = call(lib.f3s_attention_fwd, p, masked, order)   # eager, allocating entry point
    st = lib.f3s_attention_fwd_noalloc(*args, None)         # eager warm-up of the variant
    assert st == 0
    gpu.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = lib.f3s_attention_fwd_noalloc(*args, torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.f3s_last_error()
    what = (masked, order is not None)
    for rep in range(3):
        p.dO.fill_bytes(0xFF)
        # eager work between replays: the same pass into another buffer
        assert lib.f3s_attention_fwd(*args[:3], other.ptr, *args[4:], None) == 0
        gpu.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = p.dO.numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (what, rep)
        assert np.array_equal(other.numpy().view(np.uint32), want.view(np.uint32)), (what, rep)
    del g


def test_noalloc_replays_from_a_hip_graph(gpu):
    # The allocation-free launch captured into a graph (no allocation, no
    # host synchronisation and no memset in it): natural order, both
    # semantics, on a graph whose heavy windows take the team launch.
    torch = pytest.importorskip("torch")
    from fused3s_amd import _lib
    lib = _lib.hip()
    rp, ci = hub_graph(40000, 83, {11: 30000, 20000: 1000, 30001: 25000})
    p = Problem(gpu, rp, ci, H=2, normal=True, seed=83)
    for masked in (True, False):
        replay_matches_eager(gpu, torch, lib, p, masked)


def test_noalloc_replays_an_ordered_schedule_from_a_hip_graph(gpu):
    # 4,096 windows x 64 heads = 2^18 window-heads: a window order only names
    # the windows and the schedule runs them, its inverse (sched_inverse)
    # captured with the rest; the reference's descending order, masked.
    torch = pytest.importorskip("torch")
    from fused3s_amd import _lib
    lib = _lib.hip()
    rp, ci = hub_graph(65536, 84, {3: 3000, 40000: 3000})
    p = Problem(gpu, rp, ci, H=64, seed=84, f32=True)
    assert p.bsf.W * p.H >= 1 << 18
    replay_matches_eager(gpu, torch, lib, p, True, gpu.window_order_device(p.bsf))
