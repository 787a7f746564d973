"""The binary graph file of libf3s_host.so (f3s_host_save_graph /
f3s_host_load_graph): exact round trips of the CSR and of the block-sparse
form with its row masks (the latter from the CPU oracle's converter, so the
file carries the same bits the GPU converter is held to), and rejection of
every kind of damaged or inconsistent file.  CPU only."""
from __future__ import annotations

import os

import numpy as np
import pytest

import _oracle as orc
from conftest import GOLDEN, random_csr

import fused3s_amd as f3s


def oracle_bsf(rp, ci) -> f3s.BlockSparseFormat:
    n = len(rp) - 1
    offs, bcol, mask = orc.convert(n, rp, ci)
    return f3s.BlockSparseFormat((n + 15) // 16, offs, bcol, mask)


def same_bsf(a: f3s.BlockSparseFormat, b: f3s.BlockSparseFormat, masks=True) -> bool:
    ok = (a.num_row_windows == b.num_row_windows
          and np.array_equal(a.window_offsets, b.window_offsets)
          and np.array_equal(a.block_col_indices, b.block_col_indices))
    return ok and (not masks or np.array_equal(a.tile_masks, b.tile_masks))


def test_csr_round_trip_cora(tmp_path):
    g = f3s.load_csr_graph(str(GOLDEN / "cora"))
    p = str(tmp_path / "cora.f3sg")
    f3s.save_graph(p, g.row_ptr, g.col_ind)
    g2, bsf = f3s.load_graph(p)
    assert bsf is None
    assert (g2.num_nodes, g2.num_edges) == (2708, 10556)
    assert np.array_equal(g2.row_ptr, g.row_ptr) and np.array_equal(g2.col_ind, g.col_ind)
    assert not os.path.exists(p + ".tmp")
    # header + arrays at 64-byte boundaries
    assert os.path.getsize(p) == 64 + 10880 + 42240


@pytest.mark.parametrize("n,deg,seed", [(1, 0, 0), (17, 3, 1), (1000, 9, 2)])
def test_block_sparse_round_trip(tmp_path, n, deg, seed):
    rp, ci = random_csr(n, deg, seed, self_loops=True)
    bsf = oracle_bsf(rp, ci)
    p = str(tmp_path / "g.f3sg")
    f3s.save_graph(p, rp, ci, bsf)
    g2, b2 = f3s.load_graph(p)
    assert np.array_equal(g2.row_ptr, rp) and np.array_equal(g2.col_ind, ci)
    assert same_bsf(bsf, b2)
    # without masks
    f3s.save_graph(p, rp, ci, f3s.BlockSparseFormat(bsf.num_row_windows, bsf.window_offsets,
                                                    bsf.block_col_indices))
    _, b3 = f3s.load_graph(p)
    assert same_bsf(bsf, b3, masks=False) and len(b3.tile_masks) == 0


def test_repeated_entries_are_counted_on_load(tmp_path):
    """A multigraph's block-sparse form (the oracle converter's: repeats
    dropped from the lists and masks) reloads with duplicate_entries =
    nnz - mask bits."""
    rp0, ci0 = random_csr(200, 5, 9)
    n = len(rp0) - 1
    rows = np.repeat(np.arange(n), np.diff(rp0))
    extra = np.arange(0, len(ci0), 7)
    rows2 = np.concatenate([rows, rows[extra]])
    cols2 = np.concatenate([ci0, ci0[extra]])
    k = np.argsort(rows2.astype(np.int64) * n + cols2, kind="stable")
    rows2, cols2 = rows2[k], cols2[k].astype(np.int32)
    rp = np.zeros(n + 1, np.int32)
    rp[1:] = np.cumsum(np.bincount(rows2, minlength=n))
    p = str(tmp_path / "multi.f3sg")
    f3s.save_graph(p, rp, cols2, oracle_bsf(rp, cols2))
    g, bsf = f3s.load_graph(p)
    assert g.num_edges == len(cols2)
    assert bsf.duplicate_entries == len(extra)
    assert same_bsf(bsf, oracle_bsf(rp0, ci0))


def test_empty_graph(tmp_path):
    p = str(tmp_path / "e.f3sg")
    f3s.save_graph(p, np.zeros(1, np.int32), np.zeros(0, np.int32))
    g, b = f3s.load_graph(p)
    assert g.num_nodes == 0 and g.num_edges == 0 and b is None
    rp = np.zeros(33, np.int32)                       # 32 nodes, no edges
    f3s.save_graph(p, rp, np.zeros(0, np.int32), oracle_bsf(rp, np.zeros(0, np.int32)))
    g, b = f3s.load_graph(p)
    assert g.num_nodes == 32 and b.num_row_windows == 2 and len(b.block_col_indices) == 0


def written(tmp_path):
    rp, ci = random_csr(300, 5, 3)
    p = tmp_path / "g.f3sg"
    f3s.save_graph(str(p), rp, ci, oracle_bsf(rp, ci))
    return p


@pytest.mark.parametrize("offset,what", [(0, "not a graph file"), (20, "header checksum"),
                                         (64 + 8, "payload checksum"),
                                         (-33, "payload checksum")])
def test_damage_is_detected(tmp_path, offset, what):
    p = written(tmp_path)
    b = bytearray(p.read_bytes())
    at = offset if offset >= 0 else len(b) + offset
    # a byte inside an array: the masks (32 B per tile) end at most 32 bytes
    # of zero padding before the end of the file
    b[at] ^= 0x5A
    p.write_bytes(bytes(b))
    with pytest.raises(RuntimeError, match=what):
        f3s.load_graph(str(p))


def test_truncated_and_missing_files(tmp_path):
    p = written(tmp_path)
    b = p.read_bytes()
    p.write_bytes(b[:-64])
    with pytest.raises(RuntimeError, match="does not match the header"):
        f3s.load_graph(str(p))
    p.write_bytes(b[:40])
    with pytest.raises(RuntimeError, match="not a graph file"):
        f3s.load_graph(str(p))
    with pytest.raises(RuntimeError, match="cannot open"):
        f3s.load_graph(str(tmp_path / "absent.f3sg"))


def test_invalid_contents_are_rejected(tmp_path):
    p = str(tmp_path / "bad.f3sg")
    # the writer stores what it is given; the reader checks the invariants
    f3s.save_graph(p, np.array([0, 2, 3], np.int32), np.array([1, 2, 0], np.int32))
    with pytest.raises(RuntimeError, match="outside"):
        f3s.load_graph(p)
    f3s.save_graph(p, np.array([0, 2, 1, 3], np.int32), np.array([0, 1, 2], np.int32))
    with pytest.raises(RuntimeError, match="row_ptr"):
        f3s.load_graph(p)
    rp, ci = random_csr(40, 4, 5)
    bsf = oracle_bsf(rp, ci)
    bc = bsf.block_col_indices.copy()
    lo, hi = bsf.window_offsets[0], bsf.window_offsets[1]
    assert hi - lo >= 2
    bc[lo], bc[lo + 1] = bc[lo + 1], bc[lo]           # not ascending in window 0
    f3s.save_graph(p, rp, ci, f3s.BlockSparseFormat(bsf.num_row_windows, bsf.window_offsets,
                                                    bc, bsf.tile_masks))
    with pytest.raises(RuntimeError, match="ascend"):
        f3s.load_graph(p)


def ascending_tail_graph():
    """32 nodes, two windows: rows 0-15 link to nodes 0 and 16 (window 0
    holds block columns 0 and 1, the last tiles of the list), rows 16-31
    have no edges, so a walk past window 0's end reads ascending columns up
    to the end of block_col and then past it."""
    rp = np.zeros(33, np.int32)
    rp[1:17] = 2 * np.arange(1, 17)
    rp[17:] = 32
    ci = np.tile(np.array([0, 16], np.int32), 16)
    return rp, ci


@pytest.mark.parametrize("graph,k", [("random", 1), ("random", 50), ("random", 100000),
                                     ("tail", 1), ("tail", 7)])
def test_offsets_past_the_tile_count_are_rejected(tmp_path, graph, k):
    # window_offsets = [0, T + k, ..., T]: an entry past T must be rejected
    # before any block column is read through it (the block_col array holds
    # exactly T entries), with a valid checksum in front of it.
    rp, ci = random_csr(64, 4, 7) if graph == "random" else ascending_tail_graph()
    bsf = oracle_bsf(rp, ci)
    T = int(bsf.window_offsets[-1])
    wo = bsf.window_offsets.copy()
    assert len(wo) >= 3
    wo[1] = T + k
    p = str(tmp_path / "o.f3sg")
    f3s.save_graph(p, rp, ci, f3s.BlockSparseFormat(bsf.num_row_windows, wo,
                                                    bsf.block_col_indices, bsf.tile_masks))
    with pytest.raises(RuntimeError, match="not monotone"):
        f3s.load_graph(p)


def test_writer_rejects_wrong_window_count(tmp_path):
    rp, ci = random_csr(40, 4, 6)
    bsf = oracle_bsf(rp, ci)
    with pytest.raises(RuntimeError, match="ceil"):
        f3s.save_graph(str(tmp_path / "w.f3sg"), rp, ci,
                       f3s.BlockSparseFormat(bsf.num_row_windows + 1, bsf.window_offsets,
                                             bsf.block_col_indices))
