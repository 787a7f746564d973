"""The fused SDDMM -> online softmax -> SpMM pass (f3s_1tb1rw_kernel's
counterpart, src/fused3s_v2.cu:81-246), through the C-ABI."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .device import DeviceArray, Stream, check
from .graph import DeviceBSF


def attention_fwd(Q: DeviceArray, K: DeviceArray, V: DeviceArray, O: DeviceArray, bsf: DeviceBSF,
                  window_order: DeviceArray | None = None, masked: bool = True, H: int = 1,
                  d: int = 64, scale: float = 1.0, stream: Stream | None = None) -> None:
    """One fused pass with each window handled whole (the reference's launch,
    tests/test_fused_3s_v2.cu:124-131).  masked=False gives the reference's
    tile-dense semantics."""
    mask = bsf.tile_mask.ptr if (masked and bsf.tile_mask is not None) else None
    if masked and mask is None:
        raise ValueError("masked attention needs a BSF converted with masks")
    check(_lib.hip().f3s_attention_fwd(Q.ptr, K.ptr, V.ptr, O.ptr, bsf.window_offsets.ptr,
                                       bsf.block_col.ptr, mask,
                                       window_order.ptr if window_order is not None else None,
                                       bsf.W, bsf.n, d, H, scale,
                                       stream.handle if stream else None), "f3s_attention_fwd")


def attention_fwd_timed(Q: DeviceArray, K: DeviceArray, V: DeviceArray, O: DeviceArray,
                        bsf: DeviceBSF, window_order: DeviceArray | None = None,
                        masked: bool = True, H: int = 1, d: int = 64, scale: float = 1.0,
                        reps: int = 10, stream: Stream | None = None) -> float:
    """f3s_attention_fwd_timed: `reps` unplanned passes timed with HIP events
    on the launch stream (the reference harness's timed launch,
    tests/test_fused_3s_v2.cu:126-136); mean microseconds per pass."""
    mask = bsf.tile_mask.ptr if (masked and bsf.tile_mask is not None) else None
    if masked and mask is None:
        raise ValueError("masked attention needs a BSF converted with masks")
    us = C.c_float(0.0)
    check(_lib.hip().f3s_attention_fwd_timed(Q.ptr, K.ptr, V.ptr, O.ptr, bsf.window_offsets.ptr,
                                             bsf.block_col.ptr, mask,
                                             window_order.ptr if window_order is not None else None,
                                             bsf.W, bsf.n, d, H, scale,
                                             stream.handle if stream else None, reps,
                                             C.byref(us)), "f3s_attention_fwd_timed")
    return float(us.value)


class Plan:
    """f3s_plan: segments of heavy windows merged inside the launch."""

    def __init__(self, bsf: DeviceBSF, window_order: DeviceArray | None = None, H: int = 1,
                 seg_tiles: int = 0, stream: Stream | None = None):
        h = C.c_void_p()
        check(_lib.hip().f3s_plan_create(bsf.window_offsets.ptr,
                                         window_order.ptr if window_order is not None else None,
                                         bsf.W, H, seg_tiles, stream.handle if stream else None,
                                         C.byref(h)), "f3s_plan_create")
        self.handle = h.value
        self.bsf = bsf
        self.H = H
        ni, ns, T = C.c_int64(), C.c_int64(), C.c_int64()
        seg = C.c_int32()
        check(_lib.hip().f3s_plan_info(self.handle, C.byref(ni), C.byref(ns), C.byref(T),
                                       C.byref(seg)), "f3s_plan_info")
        self.num_items, self.num_split, self.T, self.seg_tiles = ni.value, ns.value, T.value, seg.value

    def compile(self, stream: Stream | None = None) -> None:
        """f3s_plan_compile: list the attended columns once (masked passes)."""
        bsf = self.bsf
        if bsf.tile_mask is None:
            raise ValueError("compiling a plan needs a BSF converted with masks")
        check(_lib.hip().f3s_plan_compile(self.handle, bsf.block_col.ptr, bsf.tile_mask.ptr,
                                          bsf.n, stream.handle if stream else None),
              "f3s_plan_compile")

    def stats(self) -> dict:
        """f3s_plan_stats: compiled chunks and, per item set, items and
        split-window partial slots."""
        v = [C.c_int64() for _ in range(5)]
        check(_lib.hip().f3s_plan_stats(self.handle, *(C.byref(x) for x in v)), "f3s_plan_stats")
        return dict(zip(("num_chunks", "masked_items", "masked_slots", "dense_items",
                         "dense_slots"), (int(x.value) for x in v)))

    def forward(self, Q: DeviceArray, K: DeviceArray, V: DeviceArray, O: DeviceArray,
                masked: bool = True, d: int = 64, scale: float = 1.0,
                stream: Stream | None = None) -> None:
        bsf = self.bsf
        mask = bsf.tile_mask.ptr if (masked and bsf.tile_mask is not None) else None
        if masked and mask is None:
            raise ValueError("masked attention needs a BSF converted with masks")
        check(_lib.hip().f3s_attention_fwd_planned(self.handle, Q.ptr, K.ptr, V.ptr, O.ptr,
                                                   bsf.block_col.ptr, mask, bsf.n, d, self.H,
                                                   scale, stream.handle if stream else None),
              "f3s_attention_fwd_planned")

    def __del__(self):
        try:
            if self.handle:
                _lib.hip().f3s_plan_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def cast_f32_to_f16(x: DeviceArray, out: DeviceArray, stream: Stream | None = None) -> None:
    """float2half_kernel (tests/test_fused_3s_v2.cu:61-64)."""
    count = int(np.prod(x.shape))
    check(_lib.hip().f3s_cast_f32_to_f16(x.ptr, out.ptr, count, stream.handle if stream else None),
          "f3s_cast_f32_to_f16")


def naive_attention_fwd(Q: DeviceArray, K: DeviceArray, V: DeviceArray, O: DeviceArray,
                        csr, d: int = 64, scale: float = 1.0,
                        stream: Stream | None = None) -> None:
    """f3s_naive_attention_fwd: the naive edge-exact comparator
    (baselines/gpu_baseline.cu:28-116), fp32 [n][d] features, CSR as stored."""
    check(_lib.hip().f3s_naive_attention_fwd(Q.ptr, K.ptr, V.ptr, O.ptr, csr.row_ptr.ptr,
                                             csr.col_idx.ptr, csr.n, d, scale,
                                             stream.handle if stream else None),
          "f3s_naive_attention_fwd")


def probe_gather(K: DeviceArray, V: DeviceArray, rows: int, row_stride: int,
                 idx: DeviceArray, out: DeviceArray, cpw: int = 8,
                 stream: Stream | None = None) -> None:
    """f3s_probe_gather (measurement only): loads the 128-byte K and V rows
    named by the int32 ``idx`` (a multiple of 32 entries) in the fused pass's
    load shape and folds them into ``out`` (one uint32 per wave)."""
    count = int(np.prod(idx.shape))
    check(_lib.hip().f3s_probe_gather(K.ptr, V.ptr, rows, row_stride, idx.ptr, count, cpw,
                                      out.ptr, stream.handle if stream else None),
          "f3s_probe_gather")
