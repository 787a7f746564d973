"""Host API of the path, mirroring the reference's include/utils.cuh and
src/converter.cu (same names, argument meaning and error behaviour), plus
the device-resident forms used by the fused pass and the synthetic inputs.
"""
from __future__ import annotations

import ctypes as C
import os
import sys
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .device import DeviceArray, Stream, check


@dataclass
class GraphData:
    """include/utils.cuh:19-24."""
    num_nodes: int
    num_edges: int
    row_ptr: np.ndarray   # int32[n+1]
    col_ind: np.ndarray   # int32[nnz]


@dataclass
class BlockSparseFormat:
    """include/utils.cuh:42-46 plus the intra-tile row masks and the number of
    CSR entries that repeat an earlier (row, column) pair.  With repeats the
    tile lists are those of the deduplicated CSR (as the reference converter
    gives), and the masks -- so the masked pass -- count each edge once, where
    cpu_sparse_attention_csr (baselines/cpu_baseline.cpp:38-50) counts every
    repeat."""
    num_row_windows: int
    window_offsets: np.ndarray        # int32[W+1]
    block_col_indices: np.ndarray     # int32[T]
    tile_masks: np.ndarray = field(default_factory=lambda: np.zeros((0, 16), np.uint16))  # uint16[T,16]
    duplicate_entries: int = 0


def _mask_bits(masks: np.ndarray) -> int:
    """Distinct (row, column) pairs the row masks record."""
    return int(np.bitwise_count(np.ascontiguousarray(masks, np.uint16)).sum(dtype=np.int64))


def _take_i32(ptr, count: int) -> np.ndarray:
    """Copies a library-allocated int32 array into numpy and frees it."""
    try:
        if count == 0:
            return np.zeros(0, np.int32)
        return np.ctypeslib.as_array(ptr, shape=(count,)).copy()
    finally:
        _lib.host().f3s_host_free(C.cast(ptr, C.c_void_p))


def load_csr_graph(dataset_dir: str) -> GraphData:
    """include/utils.cuh:26-40.  Reads meta.txt, row_ptr.txt and col_idx.txt
    (col_ind.txt accepted); raises RuntimeError on a missing/short/invalid
    file rather than returning the reference's silent all-zero columns."""
    n = C.c_int32()
    nnz = C.c_int64()
    rp = C.POINTER(C.c_int32)()
    ci = C.POINTER(C.c_int32)()
    lib = _lib.host()
    if lib.f3s_host_load_csr(os.fsencode(dataset_dir), C.byref(n), C.byref(nnz),
                             C.byref(rp), C.byref(ci)) != 0:
        raise RuntimeError(lib.f3s_host_last_error().decode())
    return GraphData(int(n.value), int(nnz.value), _take_i32(rp, n.value + 1), _take_i32(ci, nnz.value))


def save_graph(path: str, row_ptr, col_ind, bsf: BlockSparseFormat | None = None) -> None:
    """Writes the CSR (and the block-sparse form, with its row masks when it
    holds them) to one checksummed binary file (f3s_host_save_graph)."""
    rp = np.ascontiguousarray(row_ptr, np.int32)
    ci = np.ascontiguousarray(col_ind, np.int32)
    n = len(rp) - 1
    args = [None, None, None]
    W, T = 0, 0
    if bsf is not None:
        wo = np.ascontiguousarray(bsf.window_offsets, np.int32)
        bc = np.ascontiguousarray(bsf.block_col_indices, np.int32)
        W, T = int(bsf.num_row_windows), len(bc)
        tm = (np.ascontiguousarray(bsf.tile_masks, np.uint16)
              if len(bsf.tile_masks) == T and T > 0 else None)
        args = [wo.ctypes.data, bc.ctypes.data, tm.ctypes.data if tm is not None else None]
    lib = _lib.host()
    if lib.f3s_host_save_graph(os.fsencode(path), n, len(ci), rp.ctypes.data, ci.ctypes.data,
                               W, T, *args) != 0:
        raise RuntimeError(lib.f3s_host_last_error().decode())


def load_graph(path: str) -> tuple[GraphData, BlockSparseFormat | None]:
    """Reads a file written by save_graph (f3s_host_load_graph); raises
    RuntimeError on any corruption or invariant violation."""
    n, nnz, W, T = C.c_int32(), C.c_int64(), C.c_int32(), C.c_int64()
    rp, ci, wo, bc = (C.POINTER(C.c_int32)() for _ in range(4))
    tm = C.POINTER(C.c_uint16)()
    lib = _lib.host()
    if lib.f3s_host_load_graph(os.fsencode(path), C.byref(n), C.byref(nnz), C.byref(rp),
                               C.byref(ci), C.byref(W), C.byref(T), C.byref(wo), C.byref(bc),
                               C.byref(tm)) != 0:
        raise RuntimeError(lib.f3s_host_last_error().decode())
    g = GraphData(int(n.value), int(nnz.value), _take_i32(rp, n.value + 1),
                  _take_i32(ci, nnz.value))
    if not wo:
        return g, None
    masks = np.zeros((0, 16), np.uint16)
    if tm:
        try:
            if T.value:
                masks = np.ctypeslib.as_array(tm, shape=(T.value * 16,)).copy().reshape(-1, 16)
        finally:
            lib.f3s_host_free(C.cast(tm, C.c_void_p))
    dup = int(nnz.value) - _mask_bits(masks) if tm else 0
    return g, BlockSparseFormat(int(W.value), _take_i32(wo, W.value + 1),
                                _take_i32(bc, T.value), masks, dup)


class DeviceCSR:
    """A CSR graph resident in device memory."""

    def __init__(self, row_ptr: np.ndarray, col_idx: np.ndarray, stream: Stream | None = None):
        self.n = int(len(row_ptr) - 1)
        self.nnz = int(len(col_idx))
        self.row_ptr = DeviceArray.from_numpy(np.asarray(row_ptr, np.int32), stream)
        self.col_idx = DeviceArray.from_numpy(np.asarray(col_idx, np.int32), stream)


class DeviceBSF:
    """Block-sparse format resident in device memory (converter output)."""

    def __init__(self, n: int, W: int, T: int, window_offsets: DeviceArray,
                 block_col: DeviceArray, tile_mask: DeviceArray | None):
        self.n, self.W, self.T = n, W, T
        self.window_offsets = window_offsets
        self.block_col = block_col
        self.tile_mask = tile_mask

    def to_host(self) -> BlockSparseFormat:
        return BlockSparseFormat(
            self.W, self.window_offsets.numpy(), self.block_col.numpy(),
            self.tile_mask.numpy().reshape(self.T, 16) if self.tile_mask is not None
            else np.zeros((0, 16), np.uint16))


def convert_device(csr: DeviceCSR, masks: bool = True, stream: Stream | None = None) -> DeviceBSF:
    """f3s_convert_csr_to_bsf: counts, then tile lists (and masks)."""
    lib = _lib.hip()
    W = (csr.n + 15) // 16
    offs = DeviceArray(W + 1, np.int32)
    T = C.c_int64(0)
    s = stream.handle if stream else None
    check(lib.f3s_convert_csr_to_bsf(csr.row_ptr.ptr, csr.col_idx.ptr, csr.n, csr.nnz, offs.ptr,
                                     None, None, C.byref(T), s), "f3s_convert_csr_to_bsf(count)")
    bcol = DeviceArray(T.value, np.int32)
    mask = DeviceArray(T.value * 16, np.uint16) if masks else None
    T2 = C.c_int64(0)
    check(lib.f3s_convert_csr_to_bsf(csr.row_ptr.ptr, csr.col_idx.ptr, csr.n, csr.nnz, offs.ptr,
                                     bcol.ptr, mask.ptr if mask else None, C.byref(T2), s),
          "f3s_convert_csr_to_bsf(fill)")
    return DeviceBSF(csr.n, W, int(T.value), offs, bcol, mask)


def convert_csr_to_block_sparse(num_nodes: int, row_ptr, col_ind, verbose: bool = True) -> BlockSparseFormat:
    """src/converter.cu:13-44, computed on the GPU (bit-exact with the
    reference's host converter); prints the reference's two lines (:42-43)."""
    row_ptr = np.asarray(row_ptr, np.int32)
    col_ind = np.asarray(col_ind, np.int32)
    if len(row_ptr) != num_nodes + 1:
        raise ValueError("convert_csr_to_block_sparse: row_ptr must hold n+1 entries")
    dev = convert_device(DeviceCSR(row_ptr, col_ind))
    _, mask_bits = bsf_stats(dev, True)   # the distinct (row, column) pairs, on the device
    bsf = dev.to_host()
    bsf.duplicate_entries = len(col_ind) - mask_bits
    if verbose:
        print(f"Row Windows: {bsf.num_row_windows}")
        print(f"Total Active Blocks: {len(bsf.block_col_indices)}")
    if bsf.duplicate_entries > 0:
        print(f"convert_csr_to_block_sparse: the CSR repeats {bsf.duplicate_entries} entries; "
              "tile lists are unaffected, masked attention counts each edge once "
              "(cpu_sparse_attention_csr counts every repeat)", file=sys.stderr)
    return bsf


def generate_balanced_window_order(fmt: BlockSparseFormat) -> np.ndarray:
    """include/utils.cuh:48-59 (host std::sort, the reference comparator)."""
    W = int(fmt.num_row_windows)
    out = np.empty(W, np.int32)
    offs = np.ascontiguousarray(fmt.window_offsets, np.int32)
    if W:
        if len(offs) != W + 1:
            raise ValueError("window_offsets must hold W+1 entries")
        lib = _lib.host()
        if lib.f3s_host_window_order(offs.ctypes.data, W, out.ctypes.data) != 0:
            raise RuntimeError(lib.f3s_host_last_error().decode())
    return out


def window_order_device(bsf: DeviceBSF, stream: Stream | None = None) -> DeviceArray:
    """f3s_window_order: descending tile count, ties by ascending index."""
    order = DeviceArray(bsf.W, np.int32)
    check(_lib.hip().f3s_window_order(bsf.window_offsets.ptr, bsf.W, order.ptr,
                                      stream.handle if stream else None), "f3s_window_order")
    return order


def bsf_stats(bsf: DeviceBSF, masked: bool, stream: Stream | None = None) -> tuple[int, int]:
    """(occ_sum, mask_bits) of f3s_bsf_stats."""
    occ = C.c_int64()
    bits = C.c_int64()
    check(_lib.hip().f3s_bsf_stats(bsf.block_col.ptr, bsf.tile_mask.ptr if (masked and bsf.tile_mask) else None,
                                   bsf.T, bsf.n, C.byref(occ), C.byref(bits),
                                   stream.handle if stream else None), "f3s_bsf_stats")
    return int(occ.value), int(bits.value)


# ----------------------------------------------------------------- inputs

def powerlaw_graph(n: int, target_edges: int, gamma: float, max_degree: float,
                   permute: bool, self_loops: bool, seed: int) -> tuple[np.ndarray, np.ndarray]:
    rp = C.POINTER(C.c_int32)()
    ci = C.POINTER(C.c_int32)()
    nnz = C.c_int64()
    lib = _lib.host()
    if lib.f3s_gen_powerlaw(n, target_edges, gamma, max_degree, int(permute), int(self_loops),
                            seed, C.byref(rp), C.byref(ci), C.byref(nnz)) != 0:
        raise RuntimeError(lib.f3s_host_last_error().decode())
    return _take_i32(rp, n + 1), _take_i32(ci, nnz.value)


def sbm_graph(n: int, community: int, mean_degree: float, p_intra: float, self_loops: bool,
              seed: int) -> tuple[np.ndarray, np.ndarray]:
    rp = C.POINTER(C.c_int32)()
    ci = C.POINTER(C.c_int32)()
    nnz = C.c_int64()
    lib = _lib.host()
    if lib.f3s_gen_sbm(n, community, mean_degree, p_intra, int(self_loops), seed,
                       C.byref(rp), C.byref(ci), C.byref(nnz)) != 0:
        raise RuntimeError(lib.f3s_host_last_error().decode())
    return _take_i32(rp, n + 1), _take_i32(ci, nnz.value)


def features_f16(seed: int, tensor: int, count: int, normal: bool) -> np.ndarray:
    """binary16 values (as np.float16) of Q (tensor 0), K (1) or V (2)."""
    out = np.empty(count, np.uint16)
    lib = _lib.host()
    if lib.f3s_gen_features_f16(seed, tensor, count, 1 if normal else 0, out.ctypes.data) != 0:
        raise RuntimeError(lib.f3s_host_last_error().decode())
    return out.view(np.float16)
