"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

How each oracle function is pinned (none is left "parity unpinned"):
  orc_f32_to_f16 / orc_f16_to_f32   numpy's IEEE binary16 conversion (an
                                    independent implementation), exhaustively
                                    over all 2^16 halves, all ties, specials
                                    and random float32 bit patterns
  orc_load_csr                      the fixture files parsed by numpy; the
                                    reference's stated sizes (meta.txt)
  orc_convert_count/fill            W=170 for Cora (README.md:140, the NCU
                                    grid of sc_csvs/v2_cora_ncu_results.csv);
                                    known answers for the reference's input
                                    (T, sums, hashes); and invariants
                                    that characterise the output completely:
                                    every edge's tile is listed with its bit
                                    set, no bit without an edge, ascending
                                    unique lists
  orc_window_order                  stable-sort invariants (permutation,
                                    non-increasing counts, ties ascending)
  orc_masked_attention              the reference's own cpu_sparse_attention_csr
                                    compiled from baselines/cpu_baseline.cpp
                                    (oracle/_ref): bit-identical; float64 dense
                                    brute force; closed forms
  orc_tile_dense_attention          equals the reference's cpu_sparse_attention_csr
                                    run on the tile-expanded CSR (bit-identical);
                                    closed forms
  orc_tile_dense_attention_fast     the same two checks, and bit-identical to
                                    orc_tile_dense_attention on random graphs
                                    (heads, scale, row ranges, empty graphs) and
                                    on config 4's windows, its hub included
  orc_bsf_occupancy                 numpy popcounts
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

from conftest import GOLDEN, random_csr, rng
import _oracle as orc


def load_np(d):
    n, nnz = (int(x) for x in open(d / "meta.txt").read().split())
    rp = np.loadtxt(d / "row_ptr.txt", dtype=np.int64).astype(np.int32)
    ci = np.loadtxt(d / "col_idx.txt", dtype=np.int64).astype(np.int32)
    return n, nnz, rp, ci


# ------------------------------------------------------------------ fp16

def test_f16_to_f32_all_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_roundtrip_and_ties():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    assert np.array_equal(orc.f32_to_f16_bits(f[finite]), h[finite])
    # exact midpoints between consecutive positive finite halves (ties)
    pos = np.arange(0, 0x7bff, dtype=np.uint32).astype(np.uint16)
    lo = pos.view(np.float16).astype(np.float64)
    hi = (pos + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    exact = mid.astype(np.float64) == (lo + hi) / 2
    for sgn in (1.0, -1.0):
        x = (sgn * mid[exact]).astype(np.float32)
        assert np.array_equal(orc.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))


def test_f32_to_f16_random_bits_and_specials():
    bits = rng(1).integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 1e-8, 6e-8,
                         5.960464477539063e-08, 2.9802322387695312e-08, 2.98e-08, 1e30, -1e-30],
                        np.float32)
    for arr in (x, specials):
        with np.errstate(over="ignore"):
            want = arr.astype(np.float16).view(np.uint16)
        assert np.array_equal(orc.f32_to_f16_bits(arr), want)


# ---------------------------------------------------------------- loader

@pytest.mark.parametrize("name,n,nnz", [("cora", 2708, 10556), ("citeseer", 3327, 9104)])
def test_loader_fixtures(name, n, nnz):
    rc, rp, ci = orc.load_csr(str(GOLDEN / name))
    assert rc == 0
    n2, nnz2, rp2, ci2 = load_np(GOLDEN / name)
    assert (len(rp) - 1, len(ci)) == (n, nnz) == (n2, nnz2)
    assert np.array_equal(rp, rp2) and np.array_equal(ci, ci2)


def test_loader_fallback_name_and_errors(tmp_path):
    d = tmp_path / "g"
    d.mkdir()
    (d / "meta.txt").write_text("3 4\n")
    (d / "row_ptr.txt").write_text("0\n1\n3\n4\n")
    (d / "col_ind.txt").write_text("1\n0\n2\n1\n")
    rc, rp, ci = orc.load_csr(str(d))
    assert rc == 0 and list(ci) == [1, 0, 2, 1]
    (d / "col_ind.txt").write_text("1\n0\n")          # short
    assert orc.load_csr(str(d))[0] == 3
    assert orc.load_csr(str(tmp_path / "missing"))[0] == 1


# ------------------------------------------------------------- converter

def check_bsf_invariants(n, rp, ci, offs, bcol, mask):
    """Completeness, soundness and order characterise the converter output."""
    W = (n + 15) // 16
    assert len(offs) == W + 1 and offs[0] == 0 and np.all(np.diff(offs) >= 0)
    assert offs[-1] == len(bcol) == len(mask)
    for w in range(W):
        lst = bcol[offs[w]:offs[w + 1]]
        assert np.all(np.diff(lst) > 0), "ascending unique per window"
    # every edge is present: its tile is listed and its bit set
    rows = np.repeat(np.arange(n), np.diff(rp))
    win = rows // 16
    tiles = {}
    for w in range(W):
        for t in range(offs[w], offs[w + 1]):
            tiles[(w, int(bcol[t]))] = t
    for u, c, w in zip(rows, ci, win):
        t = tiles[(int(w), int(c) // 16)]
        assert (int(mask[t, u - 16 * w]) >> (int(c) % 16)) & 1
    # no bit without an edge (simple graphs): total popcount == nnz
    pop = np.unpackbits(mask.view(np.uint8)).sum()
    assert pop == len(np.unique(rows.astype(np.int64) * n + ci))
    assert np.all(mask.reshape(len(mask), 16).any(axis=1)), "no empty tile is listed"


def sha16(a):
    return hashlib.sha256(np.ascontiguousarray(a, "<i4").tobytes()).hexdigest()[:16]


@pytest.mark.parametrize("name,T,sumbc,h_off,h_col,w0,top", [
    ("cora", 7355, 573490, "06250ff694776912", "1aac9c43d1d26eb9",
     [0, 9, 13, 16, 17, 20, 23, 29, 39, 40, 45, 62], (84, 105)),
    ("citeseer", 7467, 737199, "ac41aa46e652d60d", "99d408ddf8d72ff6",
     [7, 9, 11, 29, 30, 34, 39, 40, 42, 49, 52, 60], (88, 91)),
])
def test_converter_known_answers(name, T, sumbc, h_off, h_col, w0, top):
    n, nnz, rp, ci = load_np(GOLDEN / name)
    offs, bcol, mask = orc.convert(n, rp, ci)
    if name == "cora":
        assert len(offs) - 1 == 170          # README.md:140; 170 workgroups in the NCU grid
    assert len(bcol) == T and int(bcol.sum()) == sumbc
    assert sha16(offs) == h_off and sha16(bcol) == h_col
    assert list(bcol[:12]) == w0
    cnt = np.diff(offs)
    assert (int(cnt.argmax()), int(cnt.max())) == top
    check_bsf_invariants(n, rp, ci, offs, bcol, mask)


def test_converter_reference_loader_bug_shape():
    """With the reference's as-shipped loader every column reads as 0
    (include/utils.cuh:36): one tile per window, T == W."""
    n, nnz, rp, _ = load_np(GOLDEN / "cora")
    offs, bcol, _ = orc.convert(n, rp, np.zeros(nnz, np.int32))
    assert len(bcol) == 170 and np.all(bcol == 0)


@pytest.mark.parametrize("n,deg,seed", [(1, 0, 0), (17, 3, 1), (100, 5, 2), (333, 12, 3),
                                        (1000, 40, 4)])
def test_converter_invariants_random(n, deg, seed):
    rp, ci = random_csr(n, deg, seed)
    offs, bcol, mask = orc.convert(n, rp, ci)
    check_bsf_invariants(n, rp, ci, offs, bcol, mask)


def test_converter_empty_rows_and_unsorted_columns():
    # unsorted columns within rows; windows 1 and 2 are empty
    n = 64
    rows = {0: [63, 1, 17], 5: [0], 48: [47, 3, 62, 16], 63: [63]}
    rp = np.zeros(n + 1, np.int32)
    ci = []
    for u in range(n):
        ci += rows.get(u, [])
        rp[u + 1] = len(ci)
    ci = np.array(ci, np.int32)
    offs, bcol, mask = orc.convert(n, rp, ci)
    assert list(offs) == [0, 3, 3, 3, 7]
    assert list(bcol) == [0, 1, 3, 0, 1, 2, 3]
    check_bsf_invariants(n, rp, ci, offs, bcol, mask)


# ------------------------------------------------------------------ order

def check_order(offs, order):
    W = len(offs) - 1
    cnt = np.diff(offs)
    assert sorted(order.tolist()) == list(range(W))
    c = cnt[order]
    assert np.all(np.diff(c) <= 0)
    same = np.diff(c) == 0
    assert np.all(np.diff(order)[same] > 0), "ties by ascending window index"


def test_window_order_fixtures_and_random():
    n, nnz, rp, ci = load_np(GOLDEN / "cora")
    offs, _, _ = orc.convert(n, rp, ci)
    check_order(offs, orc.window_order(offs))
    r = rng(5)
    for W in (1, 2, 7, 1000):
        cnt = r.integers(0, 5, W)
        offs = np.concatenate([[0], np.cumsum(cnt)]).astype(np.int32)
        check_order(offs, orc.window_order(offs))


# -------------------------------------------------------------- attention

def f16_inputs(shape, seed, normal=False):
    r = rng(seed)
    x = r.standard_normal(shape) if normal else r.uniform(-1, 1, shape)
    return x.astype(np.float16).astype(np.float32)


def dense_masked_f64(n, d, Q, K, V, rp, ci, scale=1.0):
    """float64 dense masked softmax attention (brute force)."""
    A = np.zeros((n, n), bool)
    rows = np.repeat(np.arange(n), np.diff(rp))
    A[rows, ci] = True
    S = (Q.astype(np.float64) @ K.astype(np.float64).T) * scale
    S = np.where(A, S, -np.inf)
    mx = S.max(axis=1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0)
    P = np.exp(S - mx)
    den = P.sum(axis=1, keepdims=True)
    P = np.divide(P, den, out=np.zeros_like(P), where=den > 0)
    return P @ V.astype(np.float64)


needs_ref = pytest.mark.skipif(not orc.ref_available(),
                               reason="oracle/_ref not built (reference tree absent at build time)")


@needs_ref
@pytest.mark.parametrize("name", ["cora", "citeseer"])
def test_masked_oracle_equals_reference_cpu_baseline(name):
    n, nnz, rp, ci = load_np(GOLDEN / name)
    d = 64
    Q, K, V = (f16_inputs((n, d), s) for s in (11, 12, 13))
    ref = orc.ref_masked_attention(n, d, Q, K, V, rp, ci)
    got = orc.masked_attention(n, d, 1, Q, K, V, rp, ci)[:, 0, :]
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


@needs_ref
def test_tile_dense_oracle_equals_reference_on_expanded_csr():
    """TILE_DENSE semantics == MASKED semantics on the graph where each row
    attends every column < n of its window's active tiles."""
    for name in ("cora", "citeseer"):
        n, nnz, rp, ci = load_np(GOLDEN / name)
        offs, bcol, _ = orc.convert(n, rp, ci)
        d = 64
        Q, K, V = (f16_inputs((n, d), s, normal=True) for s in (21, 22, 23))
        cols_w = [np.concatenate([16 * b + np.arange(16) for b in bcol[offs[w]:offs[w + 1]]]
                                 or [np.zeros(0, np.int64)]) for w in range(len(offs) - 1)]
        cols_w = [c[c < n] for c in cols_w]
        erp = np.zeros(n + 1, np.int64)
        eci = []
        for u in range(n):
            eci.append(cols_w[u // 16])
            erp[u + 1] = erp[u] + len(cols_w[u // 16])
        eci = np.concatenate(eci).astype(np.int32)
        ref = orc.ref_masked_attention(n, d, Q, K, V, erp.astype(np.int32), eci)
        got = orc.tile_dense_attention(n, d, 1, Q, K, V, offs, bcol)[:, 0, :]
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
        fast = orc.tile_dense_attention(n, d, 1, Q, K, V, offs, bcol, fast=True)[:, 0, :]
        assert np.array_equal(ref.view(np.uint32), fast.view(np.uint32))


@pytest.mark.parametrize("n,deg,seed,H,scale,r0,r1", [
    (37, 5, 1, 1, 1.0, 0, None),      # n % 16 != 0: padded columns of the last block column
    (200, 9, 2, 2, 0.7, 5, 197),      # a logit scale, partial first and last windows
    (1000, 30, 3, 1, 1.0, 0, None),   # dense windows
    (777, 4, 4, 3, 1.0, 16, 700),     # three heads
    (5000, 12, 5, 4, 1.0, 0, None),
    (300, 0, 6, 1, 1.0, 0, None),     # no edges at all: every window empty, O untouched
])
def test_tile_dense_fast_equals_scalar(n, deg, seed, H, scale, r0, r1):
    """orc_tile_dense_attention_fast (each window's 16 rows in SIMD lanes)
    gives the scalar restatement's bits on every row it computes and leaves
    the others untouched."""
    if deg:
        rp, ci = random_csr(n, deg, seed, self_loops=bool(seed % 2))
    else:
        rp, ci = np.zeros(n + 1, np.int32), np.zeros(0, np.int32)
    offs, bcol, _ = orc.convert(n, rp, ci)
    Q, K, V = (f16_inputs((n, H, 64), seed * 10 + s, normal=bool(seed % 2)) for s in range(3))
    a = orc.tile_dense_attention(n, 64, H, Q, K, V, offs, bcol, scale=scale, r0=r0, r1=r1)
    b = orc.tile_dense_attention(n, 64, H, Q, K, V, offs, bcol, scale=scale, r0=r0, r1=r1,
                                 fast=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_tile_dense_fast_equals_scalar_on_config4_windows():
    """The two forms agree bit for bit on config 4's first 300 windows and on
    its heaviest window (a hub of thousands of tiles), N(0, 1) inputs."""
    import fused3s_amd as f3s
    c = f3s.CONFIGS[4]
    rp, ci = c.graph()
    n = c.n
    offs, bcol, _ = orc.convert(n, rp, ci)
    Q, K, V = (c.features(t).astype(np.float32) for t in range(3))
    hub = int(np.argmax(np.diff(offs)))
    assert offs[hub + 1] - offs[hub] > 1000
    for r0, r1 in ((0, 16 * 300), (16 * hub, min(n, 16 * hub + 16))):
        a = orc.tile_dense_attention(n, 64, 1, Q, K, V, offs, bcol, r0=r0, r1=r1)
        b = orc.tile_dense_attention(n, 64, 1, Q, K, V, offs, bcol, r0=r0, r1=r1, fast=True)
        assert np.array_equal(a[r0:r1].view(np.uint32), b[r0:r1].view(np.uint32))


@pytest.mark.parametrize("n,deg,seed,scale", [(50, 4, 1, 1.0), (200, 9, 2, 0.125), (97, 30, 3, 1.0)])
def test_masked_oracle_vs_dense_brute_force(n, deg, seed, scale):
    rp, ci = random_csr(n, deg, seed, self_loops=(seed % 2 == 1))
    d = 64
    Q, K, V = (f16_inputs((n, d), seed * 10 + s, normal=True) for s in range(3))
    want = dense_masked_f64(n, d, Q, K, V, rp, ci, scale)
    got = orc.masked_attention(n, d, 1, Q, K, V, rp, ci, scale=scale)[:, 0, :]
    assert np.max(np.abs(got - want)) < 2e-5


def test_masked_oracle_closed_forms_and_heads():
    n, d = 40, 64
    rp, ci = random_csr(n, 5, 7, self_loops=False)
    deg = np.diff(rp)
    V = f16_inputs((n, d), 3)
    # Q = 0: each row is the mean of V over its neighbours; degree 0 -> 0
    O = orc.masked_attention(n, d, 1, np.zeros((n, d)), f16_inputs((n, d), 4), V, rp, ci)[:, 0]
    for u in range(n):
        want = V[ci[rp[u]:rp[u + 1]]].mean(axis=0) if deg[u] else np.zeros(d)
        assert np.allclose(O[u], want, atol=1e-6)
    # self-loop only: O[i] = V[i]
    rp1 = np.arange(n + 1, dtype=np.int32)
    O = orc.masked_attention(n, d, 1, f16_inputs((n, d), 5), f16_inputs((n, d), 6), V, rp1,
                             np.arange(n, dtype=np.int32))[:, 0]
    assert np.array_equal(O, V)
    # Q = K = V with identical rows: every row with a neighbour is that row
    x = f16_inputs((1, d), 11)[0]
    same = np.tile(x, (n, 1))
    O = orc.masked_attention(n, d, 1, same, same, same, rp, ci)[:, 0]
    assert np.allclose(O[deg > 0], x, rtol=1e-6, atol=1e-7)
    assert np.all(O[deg == 0] == 0)
    # H heads == H independent single-head problems
    H = 4
    Q, K, V4 = (f16_inputs((n, H, d), s) for s in (8, 9, 10))
    O = orc.masked_attention(n, d, H, Q, K, V4, rp, ci)
    for h in range(H):
        Oh = orc.masked_attention(n, d, 1, Q[:, h], K[:, h], V4[:, h], rp, ci)[:, 0]
        assert np.array_equal(O[:, h], Oh)


def test_tile_dense_closed_form_single_tile():
    """One tile per window, K = 0: each row is the mean of V over the tile's
    columns < n (n % 16 != 0 exercises the padded columns)."""
    n, d = 37, 64
    W = (n + 15) // 16
    offs = np.arange(W + 1, dtype=np.int32)
    bcol = np.array([2, 0, 1], np.int32)
    V = f16_inputs((n, d), 3)
    O = orc.tile_dense_attention(n, d, 1, f16_inputs((n, d), 1), np.zeros((n, d)), V, offs, bcol)
    for u in range(n):
        b = bcol[u // 16]
        cols = [c for c in range(16 * b, 16 * b + 16) if c < n]
        assert np.allclose(O[u, 0], V[cols].mean(axis=0), atol=1e-6)


def test_bsf_occupancy():
    n, nnz, rp, ci = load_np(GOLDEN / "citeseer")
    offs, bcol, mask = orc.convert(n, rp, ci)
    occ, bits = orc.bsf_occupancy(n, bcol, mask, True)
    u = np.bitwise_or.reduce(mask, axis=1)
    assert occ == int(np.unpackbits(u.view(np.uint8)).sum())
    assert bits == nnz
    occ_d, _ = orc.bsf_occupancy(n, bcol, mask, False)
    assert occ_d == int(np.minimum(16, np.maximum(0, n - 16 * bcol.astype(np.int64))).sum())
