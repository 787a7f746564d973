"""ctypes view of the CPU oracle (oracle/liboracle.so) and of the
reference's own CPU baseline compiled in place (oracle/_ref/).

Test infrastructure: used only as the checker.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
# F3S_ORACLE_LIB: the sanitizer run's instrumented build (tests/sanitize.sh)
ORACLE_SO = Path(os.environ.get("F3S_ORACLE_LIB") or ROOT / "oracle" / "liboracle.so")
REF_SO = ROOT / "oracle" / "_ref" / "libref_cpu_baseline.so"

_vp, _i32, _i64, _f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float
_API = {
    "orc_f32_to_f16": (C.c_uint16, [_f32]),
    "orc_f16_to_f32": (_f32, [C.c_uint16]),
    "orc_cast_f32_to_f16": (None, [_vp, _vp, _i64]),
    "orc_cast_f16_to_f32": (None, [_vp, _vp, _i64]),
    "orc_load_csr": (C.c_int, [C.c_char_p, C.POINTER(_i32), C.POINTER(_i64),
                               C.POINTER(C.POINTER(_i32)), C.POINTER(C.POINTER(_i32))]),
    "orc_free": (None, [_vp]),
    "orc_convert_count": (_i64, [_i32, _vp, _vp, _vp]),
    "orc_convert_fill": (None, [_i32, _vp, _vp, _vp, _vp, _vp]),
    "orc_window_order": (None, [_vp, _i32, _vp]),
    "orc_masked_attention": (None, [_i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _f32, _i32, _i32,
                                    _vp, _i32]),
    "orc_tile_dense_attention": (None, [_i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _f32, _i32,
                                        _i32, _vp, _i32]),
    "orc_tile_dense_attention_fast": (None, [_i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _f32,
                                             _i32, _i32, _vp, _i32]),
    "orc_bsf_occupancy": (None, [_i32, _i64, _vp, _vp, C.c_int, C.POINTER(_i64), C.POINTER(_i64)]),
}

_lib = None
_ref = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        _lib = C.CDLL(str(ORACLE_SO))
        for name, (res, args) in _API.items():
            fn = getattr(_lib, name)
            fn.restype, fn.argtypes = res, args
    return _lib


def ref_available() -> bool:
    return REF_SO.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        _ref = C.CDLL(str(REF_SO))
        _ref.ref_cpu_sparse_attention_csr.restype = None
        _ref.ref_cpu_sparse_attention_csr.argtypes = [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]
    return _ref


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_cast_f32_to_f16(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_cast_f16_to_f32(_p(h), _p(out), h.size)
    return out


def load_csr(d: str):
    n, nnz = _i32(), _i64()
    rp, ci = C.POINTER(_i32)(), C.POINTER(_i32)()
    rc = lib().orc_load_csr(str(d).encode(), C.byref(n), C.byref(nnz), C.byref(rp), C.byref(ci))
    if rc != 0:
        return rc, None, None
    a = np.ctypeslib.as_array(rp, shape=(n.value + 1,)).copy()
    b = np.ctypeslib.as_array(ci, shape=(max(nnz.value, 1),)).copy()[: nnz.value]
    lib().orc_free(C.cast(rp, _vp))
    lib().orc_free(C.cast(ci, _vp))
    return 0, a, b


def convert(n: int, row_ptr: np.ndarray, col_idx: np.ndarray, masks: bool = True):
    """(window_offsets, block_col, tile_mask[T,16])."""
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    col_idx = np.ascontiguousarray(col_idx, np.int32)
    W = (n + 15) // 16
    offs = np.zeros(W + 1, np.int32)
    T = lib().orc_convert_count(n, _p(row_ptr), _p(col_idx), _p(offs))
    bcol = np.zeros(max(T, 1), np.int32)
    mask = np.zeros((max(T, 1), 16), np.uint16)
    lib().orc_convert_fill(n, _p(row_ptr), _p(col_idx), _p(offs), _p(bcol),
                           _p(mask) if masks else None)
    return offs, bcol[:T], mask[:T]


def window_order(offs: np.ndarray) -> np.ndarray:
    offs = np.ascontiguousarray(offs, np.int32)
    W = len(offs) - 1
    out = np.zeros(max(W, 1), np.int32)
    lib().orc_window_order(_p(offs), W, _p(out))
    return out[:W]


def masked_attention(n, d, H, Q, K, V, row_ptr, col_idx, scale=1.0, r0=0, r1=None, threads=8):
    r1 = n if r1 is None else r1
    Q, K, V = (np.ascontiguousarray(x, np.float32) for x in (Q, K, V))
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    col_idx = np.ascontiguousarray(col_idx, np.int32)
    O = np.zeros((n, H, d), np.float32)
    lib().orc_masked_attention(n, d, H, _p(Q), _p(K), _p(V), _p(row_ptr), _p(col_idx), scale,
                               r0, r1, _p(O), threads)
    return O


def tile_dense_attention(n, d, H, Q, K, V, offs, bcol, scale=1.0, r0=0, r1=None, threads=8,
                         fast=False):
    """TILE_DENSE truth; fast=True runs orc_tile_dense_attention_fast (the
    same bits, each window's rows in SIMD lanes)."""
    r1 = n if r1 is None else r1
    Q, K, V = (np.ascontiguousarray(x, np.float32) for x in (Q, K, V))
    offs = np.ascontiguousarray(offs, np.int32)
    bcol = np.ascontiguousarray(bcol if len(bcol) else np.zeros(1, np.int32), np.int32)
    O = np.zeros((n, H, d), np.float32)
    fn = lib().orc_tile_dense_attention_fast if fast else lib().orc_tile_dense_attention
    fn(n, d, H, _p(Q), _p(K), _p(V), _p(offs), _p(bcol), scale, r0, r1, _p(O), threads)
    return O


def bsf_occupancy(n, bcol, mask, masked: bool):
    bcol = np.ascontiguousarray(bcol, np.int32)
    mask = np.ascontiguousarray(mask, np.uint16)
    occ, bits = _i64(), _i64()
    lib().orc_bsf_occupancy(n, len(bcol), _p(bcol) if len(bcol) else None,
                            _p(mask) if len(mask) else None, int(masked), C.byref(occ), C.byref(bits))
    return occ.value, bits.value


def ref_masked_attention(n, d, Q, K, V, row_ptr, col_idx):
    """The reference's own cpu_sparse_attention_csr (baselines/cpu_baseline.cpp:16)."""
    Q, K, V = (np.ascontiguousarray(x, np.float32) for x in (Q, K, V))
    row_ptr = np.ascontiguousarray(row_ptr, np.int32)
    col_idx = np.ascontiguousarray(col_idx, np.int32)
    O = np.zeros((n, d), np.float32)
    ref().ref_cpu_sparse_attention_csr(n, d, _p(Q), _p(K), _p(V), _p(row_ptr),
                                       _p(col_idx) if len(col_idx) else None, _p(O))
    return O
