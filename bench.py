"""Benchmark of the fused sparse graph-attention pass on one MI355X.

Workload (config 4): 1,000,000-node power-law graph (mean degree 16,
exponent 2.2, random node order, self-loops), d = 64, one head, Q/K/V
~ N(0, 1) in fp16, edge-exact (masked) semantics, windows in descending
workload order with heavy windows split by the plan.  A step is one fused
pass over the whole graph with inputs already resident in HBM.

Prints one JSON line: whole-job edges/s over K timed steps and the roofline
of the fused pass.  `roofline.achieved` is the pass's compulsory HBM bytes
(Q read once, O written once, every K/V row the pass needs read once, its
metadata read once) over the mean pass time from HIP events recorded on the
launch stream, so `frac` cannot exceed 1 for a real measurement.  Beside it:
the survey's gather model (every gathered K/V row counted), the traffic the
L2 sends below itself as measured by rocprofv3 on this workload (HBM or the
256 MB Infinity Cache: no gfx950 counter tells them apart), the matrix-core
work, the reference's own semantics and launch shape timed on the same
inputs after the timed region, the reference's CPU baseline
(baselines/cpu_baseline.cpp compiled under oracle/_ref, one thread as in the
reference) and the CPU restatement of it on all available host cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA
ROW_BYTES = 128                # one fp16 row of one head at d = 64
PARTIAL_BYTES = 4224           # (m, l, O) of one split-window segment and head


def gather_model_bytes(n: int, W: int, T: int, occ_sum: int, H: int, d: int,
                       masked: bool) -> int:
    """The survey's byte model: Q fp16 and O fp32 per row, window offsets +
    order, per tile a column index (+ 32 B of row masks when masked) and one
    K and one V fp16 row per attended (tile, column).  Counts every gather,
    including those the caches serve."""
    return (n * H * d * (2 + 4) + (W + 1) * 4 + W * 4 + T * (4 + (32 if masked else 0))
            + occ_sum * H * d * 2 * 2)


def kv_rows_needed(n: int, ci: np.ndarray, block_col: np.ndarray | None, masked: bool) -> int:
    """Distinct K/V rows the pass reads: the columns with at least one edge
    (masked), or every node < n of every active block column (tile-dense)."""
    if masked:
        return int(np.count_nonzero(np.bincount(ci, minlength=n)))
    W = (n + 15) // 16
    act = np.flatnonzero(np.bincount(block_col, minlength=W))
    return int(np.minimum(16, n - 16 * act).sum())


def compulsory_bytes(n: int, H: int, W: int, T: int, kv_rows: int, masked: bool,
                     launch: str, ps: dict | None) -> int:
    """HBM bytes one pass cannot avoid: Q once (fp16), O once (fp32), each
    needed K and V row once, and the metadata the launch reads once --
    compiled chunk records (256 B), items (16 B) and chunk bases, or the
    tile lists (4 B per tile, + 32 B of masks when masked) with the window
    offsets and order -- plus split-window partials written and read back."""
    b = n * H * ROW_BYTES * 3 + kv_rows * H * ROW_BYTES * 2
    if launch == "plan":
        items = ps["masked_items"] if masked else ps["dense_items"]
        slots = ps["masked_slots"] if masked else ps["dense_slots"]
        b += items * 16 + slots * H * PARTIAL_BYTES * 2
        if masked and ps["num_chunks"]:
            b += ps["num_chunks"] * 256 + (items + 1) * 4
        else:
            b += T * (4 + (32 if masked else 0))
    else:
        b += T * (4 + (32 if masked else 0)) + (W + 1) * 4 + W * 4
    return int(b)


LOCALITY_ORDERS = ("sorted-xcd", "lowest-block-column", "top-hub", "random")


def locality_order(kind: str, rp, ci, offs, bcol) -> np.ndarray:
    """A window order for the locality experiments: descending workload,
    windows by their lowest block column, windows grouped by their attended
    column of highest degree, or random; all but random laid out so that each
    eighth of the sequence runs on one XCD (given an order, workgroup b of 4
    windows runs on XCD b mod 8)."""
    cnt = np.diff(offs)
    W = len(cnt)
    if kind == "random":
        return np.random.default_rng(1).permutation(W).astype(np.int32)
    if kind == "sorted-xcd":
        seq = np.argsort(-cnt, kind="stable")
    elif kind == "lowest-block-column":
        first = np.where(cnt > 0, bcol[np.minimum(offs[:-1], max(len(bcol) - 1, 0))], 1 << 30)
        seq = np.argsort(first, kind="stable")
    else:
        n = len(rp) - 1
        deg = np.diff(rp)
        rows = np.repeat(np.arange(n), deg)
        top = np.full(W, -1, np.int64)
        best = np.full(W, -1, np.int64)
        # per window, the attended column of highest degree (ties: lowest id)
        key = deg[ci].astype(np.int64) * (n + 1) + (n - ci)
        np.maximum.at(best, rows // 16, key)
        has = best >= 0
        top[has] = n - best[has] % (n + 1)
        seq = np.lexsort((-cnt, top))
    # XCD x owns the positions of workgroups b = x, x + 8, ...; it takes the
    # x-th contiguous part of the sequence, in order (every window once)
    pos = np.arange(W)
    xcd = (pos // 4) % 8
    out = np.empty(W, np.int32)
    start = 0
    for x in range(8):
        p = pos[xcd == x]
        out[p] = seq[start:start + len(p)]
        start += len(p)
    return out


def read_profile(path: Path, key: str) -> float | None:
    """`key value` line of a committed rocprofv3 summary."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split()
        if len(parts) == 2 and parts[0] == key:
            return float(parts[1])
    return None


def convert_phases_ms(csr, bsf, stream, reps: int = 5) -> float:
    """GPU time of f3s_convert_csr_to_bsf's count call plus its fill call into
    the outputs of an earlier conversion of the same CSR (HIP events on the
    launch stream around each call); the median of `reps` conversions."""
    import fused3s_amd as f3s
    from fused3s_amd import _lib
    from fused3s_amd.device import check
    lib = _lib.hip()
    T = C.c_int64(0)
    times = []
    for _ in range(reps):
        e = [f3s.Event() for _ in range(4)]
        e[0].record(stream)
        check(lib.f3s_convert_csr_to_bsf(csr.row_ptr.ptr, csr.col_idx.ptr, csr.n, csr.nnz,
                                         bsf.window_offsets.ptr, None, None, C.byref(T),
                                         stream.handle), "convert(count)")
        e[1].record(stream)
        e[2].record(stream)
        check(lib.f3s_convert_csr_to_bsf(csr.row_ptr.ptr, csr.col_idx.ptr, csr.n, csr.nnz,
                                         bsf.window_offsets.ptr, bsf.block_col.ptr,
                                         bsf.tile_mask.ptr, C.byref(T), stream.handle),
              "convert(fill)")
        e[3].record(stream)
        f3s.synchronize()
        times.append(e[0].elapsed_ms(e[1]) + e[2].elapsed_ms(e[3]))
    return float(np.median(times))


def time_passes(f3s, one_pass, stream, reps: int) -> np.ndarray:
    """Per-pass milliseconds from HIP events on the launch stream, after one
    untimed pass."""
    return time_passes_cold(f3s, one_pass, stream, reps)[0]


def time_passes_cold(f3s, one_pass, stream, reps: int):
    """(per-pass milliseconds of `reps` passes, milliseconds of the first
    pass before them), all from HIP events on the launch stream."""
    c0, c1 = f3s.Event(), f3s.Event()
    c0.record(stream)
    one_pass()
    c1.record(stream)
    evs = [(f3s.Event(), f3s.Event()) for _ in range(reps)]
    for a, b in evs:
        a.record(stream)
        one_pass()
        b.record(stream)
    stream.synchronize()
    return np.array([a.elapsed_ms(b) for a, b in evs]), c0.elapsed_ms(c1)


def pass_times(t: np.ndarray, cold_ms: float) -> dict:
    """The per-pass statistics every timed leg reports (microseconds)."""
    return {"kernel_us": float(t.mean()) * 1e3, "kernel_us_median": float(np.median(t)) * 1e3,
            "kernel_us_min": float(t.min()) * 1e3, "cold_first_launch_us": cold_ms * 1e3,
            "passes": int(len(t))}


def gather_ceiling(f3s, dK, dV, rows: int, H: int, count: int, stream, reps: int = 10,
                   seed: int = 11, pattern: str = "uniform") -> dict:
    """The device's random-gather ceiling for the pass's load shape
    (f3s_probe_gather): `count` columns (rounded down to 32) of rows < `rows`,
    the K and V row of head 0 of each, on the workload's own tensors; mean of
    `reps` launches timed with events on `stream`.  Rows: uniformly random
    ("uniform", a masked pass's columns), runs of 16 consecutive rows from
    random multiples of 16 ("tile16", a tile-dense pass's tiles) or in order
    ("stream")."""
    count = max(32, count // 32 * 32)
    g = np.random.default_rng(seed)
    if pattern == "uniform":
        idx = g.integers(0, rows, count, dtype=np.int64)
    elif pattern == "tile16":
        runs = g.integers(0, rows // 16, (count + 15) // 16, dtype=np.int64)
        idx = (runs[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)[:count]
    elif pattern == "stream":
        idx = np.arange(count, dtype=np.int64) % rows
    else:
        raise ValueError(pattern)
    idx = idx.astype(np.int32)
    didx = f3s.DeviceArray.from_numpy(idx, stream)
    cpw = 8
    out = f3s.DeviceArray(((count // 32 + cpw - 1) // cpw,), np.uint32)
    stride = H * 128
    t = time_passes(f3s, lambda: f3s.probe_gather(dK, dV, rows, stride, didx, out, cpw, stream),
                    stream, reps)
    mean = float(t.mean())
    return {"rows_per_s": 2 * count / (mean * 1e-3), "GBps": 2 * count * 128 / (mean * 1e-3) / 1e9,
            "probe_us": mean * 1e3, "columns": count, "table_rows": rows,
            "table_bytes_each": rows * stride, "pattern": pattern}


def host_handover(f3s, rp, ci, Q, K, V, n: int, H: int, d: int, masked: bool,
                  reps: int = 3) -> dict:
    """The reference harness's flow from host memory, PCIe copies included
    (tests/test_fused_3s_v2.cu:66-137): the drop-in converter
    (convert_csr_to_block_sparse: host CSR in, host tile lists and masks
    out), the host window order (generate_balanced_window_order), then one
    pass from host buffers -- tile lists, order and Q/K/V uploaded, the
    drop-in launch in that order, O downloaded.  Host wall time of each step,
    the best of `reps`; pageable host memory, as the harness uses."""
    conv, ordt, pas = [], [], []
    for _ in range(reps):
        f3s.synchronize()
        t0 = time.perf_counter()
        fmt = f3s.convert_csr_to_block_sparse(n, rp, ci, verbose=False)
        t1 = time.perf_counter()
        host_order = f3s.generate_balanced_window_order(fmt)
        t2 = time.perf_counter()
        offs = f3s.DeviceArray.from_numpy(np.ascontiguousarray(fmt.window_offsets, np.int32))
        cols = f3s.DeviceArray.from_numpy(np.ascontiguousarray(fmt.block_col_indices, np.int32))
        mask = (f3s.DeviceArray.from_numpy(np.ascontiguousarray(fmt.tile_masks, np.uint16))
                if masked else None)
        dord = f3s.DeviceArray.from_numpy(host_order)
        dbsf = f3s.DeviceBSF(n, int(fmt.num_row_windows), len(fmt.block_col_indices), offs, cols,
                             mask)
        dq, dk, dv = (f3s.DeviceArray.from_numpy(x.view(np.uint16)) for x in (Q, K, V))
        do = f3s.DeviceArray((n, H, d), np.float32)
        f3s.attention_fwd(dq, dk, dv, do, dbsf, dord, masked=masked, H=H, d=d)
        out = do.numpy()
        t3 = time.perf_counter()
        conv.append(t1 - t0)
        ordt.append(t2 - t1)
        pas.append(t3 - t2)
        del fmt, host_order, offs, cols, mask, dord, dbsf, dq, dk, dv, do, out
    edges = int(rp[n])
    total = min(conv) + min(ordt) + min(pas)
    return {"convert_us": min(conv) * 1e6, "order_us": min(ordt) * 1e6,
            "pass_us": min(pas) * 1e6, "total_us": total * 1e6, "edges_per_s": edges / total,
            "note": "host buffers in and out (PCIe copies included): convert_csr_to_block_sparse, "
                    "generate_balanced_window_order, then upload of tile lists, order and Q/K/V, "
                    "the drop-in launch and O back; never the headline value"}


def host_cpu_model() -> str:
    """The host CPU's model name (first processor of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


ABS_TOL, REL_TOL = 2e-3, 1e-2   # the north star's bounds against the fp32 CPU truth

# Sources each profiled kernel is compiled from: a committed profile records
# their digest, and the bench flags a profile whose digest differs from the
# sources it runs.
KERNEL_SOURCES = {
    "fused_attention": ["fused3s_amd/csrc/attention.hip", "fused3s_amd/csrc/attn_common.hpp",
                        "fused3s_amd/csrc/attn_plan.hpp", "fused3s_amd/csrc/f3s_common.hpp",
                        "fused3s_amd/csrc/f3s_device.hpp"],
    "converter": ["fused3s_amd/csrc/convert.hip", "fused3s_amd/csrc/f3s_common.hpp",
                  "fused3s_amd/csrc/f3s_device.hpp"],
}


def source_digest(kernel: str) -> str:
    """First 16 hex digits of the SHA-256 over the named kernel's source
    files (path and bytes, in list order)."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES[kernel]:
        h.update(rel.encode() + b"\0")
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def read_profile_field(path: Path, key: str) -> str | None:
    """`key value` line of a committed profile, the value as text."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        parts = line.split(None, 1)
        if len(parts) == 2 and parts[0] == key:
            return parts[1].strip()
    return None


def oracle_module():
    """The CPU oracle's ctypes view (tests/_oracle.py over oracle/liboracle.so):
    the checker of the CPU leg, never what is timed as the GPU path."""
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle
    return _oracle


def check_threads() -> int:
    """Host threads the checker and the all-core baseline use: the cores this
    process may run on, at most 16 (a one-GPU box's CPU share)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def compare_rows(got: np.ndarray, want: np.ndarray) -> dict:
    """Every element of a pass's output against the fp32 truth: max abs error,
    normwise max rel error (max abs / max |truth|), the largest elementwise
    relative error over |truth| >= 0.1 (for information), and whether the
    output is within the north star's bounds with no NaN or inf."""
    g = got.reshape(-1)
    w = want.reshape(-1)
    assert g.size == w.size, (got.shape, want.shape)
    max_abs = 0.0
    max_ref = 0.0
    rel_elem = 0.0
    bad = 0
    step = 1 << 22
    for i in range(0, g.size, step):
        gi, wi = g[i:i + step], w[i:i + step]
        fin = np.isfinite(gi)
        bad += int(gi.size - np.count_nonzero(fin))
        diff = np.abs(gi - wi)
        if diff.size:
            max_abs = max(max_abs, float(np.max(diff, where=fin, initial=0.0)))
            aw = np.abs(wi)
            max_ref = max(max_ref, float(aw.max()))
            big = aw >= 0.1
            if np.any(big):
                rel_elem = max(rel_elem, float((diff[big] / aw[big]).max()))
    max_rel = max_abs / max_ref if max_ref > 0 else (0.0 if max_abs == 0 else float("inf"))
    return {"max_abs": max_abs, "max_rel": max_rel, "max_rel_elem_ge_0.1": rel_elem,
            "non_finite": bad, "elements": int(g.size), "rows": "every row",
            "ok": bool(bad == 0 and max_abs <= ABS_TOL and max_rel <= REL_TOL)}


def converter_exact(orc, bsf, n: int, rp, ci) -> dict:
    """The GPU converter's offsets, block columns and row masks against the
    oracle converter (src/converter.cu:13-44 restated, plus masks), bit for
    bit; the oracle's wall time on the checker threads beside it."""
    t0 = time.perf_counter()
    offs, bcol, mask = orc.convert(n, rp, ci)
    dt = time.perf_counter() - t0
    hb = bsf.to_host()
    same = (np.array_equal(hb.window_offsets, offs) and np.array_equal(hb.block_col_indices, bcol)
            and np.array_equal(hb.tile_masks, mask))
    return {"tile_lists_bit_exact": bool(same), "row_windows": int(len(offs) - 1),
            "active_tiles": int(len(bcol)), "oracle_converter_s": dt,
            "compared": "window_offsets, block_col_indices and tile_masks, every entry"}


def reference_single_thread(rp, ci, Q, K, V, n: int, d: int, min_s: float = 0.5) -> dict | None:
    """The reference's cpu_sparse_attention_csr (baselines/cpu_baseline.cpp,
    compiled in place under oracle/_ref), one thread, over the whole graph and
    head 0 (the reference is single-head); repeated until `min_s` seconds
    have passed on small graphs, mean time per call."""
    ref = ROOT / "oracle" / "_ref" / "libref_cpu_baseline.so"
    if not ref.exists():
        return None
    lib = C.CDLL(str(ref))
    fn = lib.ref_cpu_sparse_attention_csr
    fn.restype = None
    fn.argtypes = [C.c_int32, C.c_int32] + [C.c_void_p] * 6
    Qf, Kf, Vf = (np.ascontiguousarray(x.reshape(n, -1, d)[:, 0, :], np.float32)
                  for x in (Q, K, V))
    rp32 = np.ascontiguousarray(rp, np.int32)
    ci32 = np.ascontiguousarray(ci, np.int32)
    O = np.zeros((n, d), np.float32)
    calls = 0
    t0 = time.perf_counter()
    while True:
        fn(n, d, Qf.ctypes.data, Kf.ctypes.data, Vf.ctypes.data, rp32.ctypes.data,
           ci32.ctypes.data, O.ctypes.data)
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            break
    edges = int(rp[n])
    per = dt / calls
    return {"value": edges / per, "unit": "edges/s", "cores": 1, "kind": "reference",
            "sample": f"all {n} rows / {edges} edges, head 0 (the reference is single-head), "
                      f"{calls} call(s), {per:.4f} s per call on 1 thread",
            "threads_used": 1, "cores_available": len(os.sched_getaffinity(0)),
            "cpu_model": host_cpu_model()}


def config_legs(f3s, orc, cfgnum: int, stream, reps_masked: int = 20,
                reps_dense: int = 20) -> dict:
    """One configuration end to end on the GPU, then checked on the host:
    converter (GPU time of its two phases; output bit-exact against the
    oracle converter), the planned masked and tile-dense passes and the
    drop-in launch f3s_attention_fwd in the reference's descending order in
    both semantics (mean of HIP events per pass on the launch stream), each
    output compared on every row with the fp32 oracle after all GPU timing;
    the reference's single-thread CPU baseline (head 0) and the CPU
    restatement on all checker threads (every head) beside them."""
    c = f3s.CONFIGS[cfgnum]
    t0 = time.time()
    rp, ci = c.graph()
    n, H, d = c.n, c.H, c.d
    nnz = int(len(ci))
    Q, K, V = (c.features(t) for t in range(3))
    print(f"[bench] leg cfg{cfgnum} {c.name}: n={n} nnz={nnz} H={H} inputs "
          f"{time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    csr = f3s.DeviceCSR(rp, ci, stream)
    bsf = f3s.convert_device(csr, masks=True, stream=stream)
    f3s.synchronize()
    conv_ms = convert_phases_ms(csr, bsf, stream)
    order = f3s.window_order_device(bsf, stream)
    plan = f3s.Plan(bsf, order, H=H, stream=stream)
    plan.compile(stream)
    ps = plan.stats()
    occ_sum, mask_bits = f3s.bsf_stats(bsf, True, stream)
    dQ, dK, dV = (f3s.DeviceArray.from_numpy(x.view(np.uint16), stream) for x in (Q, K, V))
    dO = f3s.DeviceArray((n, H, d), np.float32)
    kv_rows = {True: kv_rows_needed(n, ci, None, True),
               False: kv_rows_needed(n, ci, bsf.block_col.numpy(), False)}
    runs = [
        ("masked_planned", lambda: plan.forward(dQ, dK, dV, dO, masked=True, stream=stream),
         True, "plan", reps_masked),
        ("tile_dense_planned", lambda: plan.forward(dQ, dK, dV, dO, masked=False, stream=stream),
         False, "plan", reps_dense),
        ("dropin_descending_masked",
         lambda: f3s.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=True, H=H, d=d,
                                   stream=stream), True, "unplanned", reps_masked),
        ("dropin_descending_tile_dense",
         lambda: f3s.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=False, H=H, d=d,
                                   stream=stream), False, "unplanned", reps_dense),
    ]
    legs, outs = {}, {}
    for name, fn, sem, lnch, reps in runs:
        dO.fill_bytes(0xFF, stream)   # NaN: a row the pass does not write cannot match
        t, cold = time_passes_cold(f3s, fn, stream, reps)
        mean = float(t.mean())
        b = compulsory_bytes(n, H, bsf.W, bsf.T, kv_rows[sem], sem, lnch, ps)
        chunks = (ps["num_chunks"] if (sem and lnch == "plan") else
                  (occ_sum + 31) // 32 if sem else (bsf.T + 1) // 2)
        issued = chunks * H * 8 * (2 * 16 * 16 * 32)
        tile_model = bsf.T * 4 * 16 * 16 * d * H
        legs[name] = {"semantics": "masked" if sem else "tile_dense", "launch": lnch,
                      **pass_times(t, cold), "edges_per_s": nnz / (mean * 1e-3),
                      "compulsory_bytes": b,
                      "roofline_frac": b / (mean * 1e-3) / 1e9 / HBM_PEAK_GBS,
                      "mfma_issued_frac": issued / (mean * 1e-3) / (MFMA_F16_PEAK_TFLOPS * 1e12),
                      # the tile model's flops are the work of the tile-dense
                      # semantics only (a masked pass computes attended columns)
                      "mfma_tile_model_frac": (None if sem else tile_model / (mean * 1e-3)
                                               / (MFMA_F16_PEAK_TFLOPS * 1e12))}
        outs[name] = dO.numpy()
    del dQ, dK, dV, dO, plan, order, csr
    # ---- host side, after every GPU timing: checker and CPU baselines
    print(f"[bench] leg cfg{cfgnum}: checking every row on the host ...", file=sys.stderr,
          flush=True)
    res = {"workload": f"cfg{c.cfg}: {c.name}", "nodes": n, "edges": nnz, "heads": H,
           "head_dim": d, "row_windows": bsf.W, "active_tiles": bsf.T,
           "attended_tile_columns": occ_sum, "mask_bits": mask_bits,
           "converter_us": conv_ms * 1e3}
    res["converter_check"] = converter_exact(orc, bsf, n, rp, ci)
    # measured traffic below the L2, where a committed rocprofv3 profile of
    # this configuration's planned masked pass exists (config 5; the small
    # graphs fit in the L2 and are not profiled), with its provenance
    prof = ROOT / "profiles" / f"pmc_traffic_cfg{cfgnum}.txt"
    below = read_profile(prof, "bytes_per_launch") if cfgnum != 4 else None
    if below and "masked_planned" in legs:
        mean_ms = legs["masked_planned"]["kernel_us"] * 1e-3
        digest = read_profile_field(prof, "sources_fused_attention")
        legs["masked_planned"]["below_l2"] = {
            "bytes_per_launch": below, "GBps": below / (mean_ms * 1e-3) / 1e9,
            "frac_of_hbm_peak": below / (mean_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "l2_read_hit_rate": read_profile(prof, "l2_read_hit_rate"),
            "profiled_kernel_avg_us": read_profile(prof, "kernel_avg_us"),
            "kind": "HBM + Infinity Cache (rocprofv3 FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, "
                    "copy-calibrated)",
            "source": str(prof.relative_to(ROOT)),
            "commit": read_profile_field(prof, "commit"),
            "sources_current": digest == source_digest("fused_attention")}
    offs = bsf.window_offsets.numpy()
    bcol = bsf.block_col.numpy()
    del bsf
    Qf, Kf, Vf = (x.astype(np.float32) for x in (Q, K, V))
    thr = check_threads()
    # the masked oracle, repeated on small graphs until 0.5 s have passed (its
    # mean time is the all-core baseline)
    calls = 0
    t1 = time.perf_counter()
    while True:
        want_m = orc.masked_attention(n, d, H, Qf, Kf, Vf, rp, ci, threads=thr)
        calls += 1
        if time.perf_counter() - t1 >= 0.5:
            break
    masked_s = (time.perf_counter() - t1) / calls
    t1 = time.perf_counter()
    want_d = orc.tile_dense_attention(n, d, H, Qf, Kf, Vf, offs, bcol, threads=thr, fast=True)
    dense_s = time.perf_counter() - t1
    for name, leg in legs.items():
        leg["check"] = compare_rows(outs.pop(name),
                                    want_m if leg["semantics"] == "masked" else want_d)
    del want_m, want_d
    res["legs"] = legs
    res["verified"] = bool(res["converter_check"]["tile_lists_bit_exact"]
                           and all(l["check"]["ok"] for l in legs.values()))
    res["oracle_s"] = {"masked_all_rows": masked_s, "tile_dense_all_rows": dense_s,
                       "threads": thr}
    res["cpu_baseline"] = reference_single_thread(rp, ci, Qf, Kf, Vf, n, d)
    res["cpu_baseline_all_cores"] = {
        "value": nnz / masked_s, "unit": "edges/s", "cores": thr, "kind": "port",
        "sample": f"all {n} rows / {nnz} edges x {H} head(s): the masked oracle run that "
                  f"checked the legs, {calls} call(s), {masked_s:.4f} s per call on {thr} "
                  "threads (OpenMP)",
        "cpu_model": host_cpu_model()}
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=4)
    ap.add_argument("--semantics", choices=["masked", "tile_dense"], default="masked")
    ap.add_argument("--order", choices=["auto", "sorted", "natural"] + list(LOCALITY_ORDERS),
                    default="auto",
                    help="window order: descending workload (the reference's sort) or natural; "
                         "auto = sorted (launches from 2^18 window-heads on run the library's "
                         "schedule whatever the order; smaller ones the order's sequence); "
                         "the others are locality experiments, laid out so that each eighth "
                         "of the sequence runs on one XCD")
    ap.add_argument("--seg", type=int, default=0,
                    help="plan segment size in tiles (0 = automatic)")
    ap.add_argument("--no-compile", action="store_true",
                    help="masked passes expand tiles on every pass instead of using the "
                         "plan's compiled column lists")
    ap.add_argument("--heads", type=int, default=0,
                    help="override the configuration's head count (1 to 64); the line is "
                         "then not the configuration's own workload")
    ap.add_argument("--unplanned", action="store_true",
                    help="time the drop-in launch f3s_attention_fwd (each window whole, in "
                         "the given order; the reference's launch) instead of a plan")
    ap.add_argument("--no-reference-launches", action="store_true",
                    help="skip timing the reference's semantics and launch shape, and the "
                         "flow from host memory, after the timed region")
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU leg: CPU baselines, the checker of every timed output, "
                         "and the other configurations")
    ap.add_argument("--configs", default="2,3,5",
                    help="comma-separated configurations measured and checked after the "
                         "headline, each in both semantics, planned and through the drop-in "
                         "launch (empty: none)")
    ap.add_argument("--gather-probe", action="store_true",
                    help="only measure the random-gather ceiling (f3s_probe_gather) over "
                         "tables of several sizes and exit")
    ap.add_argument("--print-source-digests", action="store_true",
                    help="print the digests of the profiled kernels' sources (the lines a "
                         "profile under profiles/ records) and exit")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run device-to-device copies of this size (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters against known bytes) and exit")
    args = ap.parse_args()
    if args.print_source_digests:
        print("\n".join(f"sources_{k} {source_digest(k)}" for k in KERNEL_SOURCES))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the path shards "
              "by row-window range with a K/V all-gather, which is not built here.",
              file=sys.stderr)
        return 2

    import fused3s_amd as f3s

    if f3s.device_count() < 1:
        print("no GPU visible", file=sys.stderr)
        return 1
    if args.copy_probe_mib:
        nb = args.copy_probe_mib << 20
        src = f3s.DeviceArray(nb, np.uint8, zero=True)
        dst = f3s.DeviceArray(nb, np.uint8)
        from fused3s_amd import _lib
        e0, e1 = f3s.Event(), f3s.Event()
        times = []
        for _ in range(args.steps):
            e0.record()
            _lib.hip().f3s_memcpy_d2d(dst.ptr, src.ptr, nb, None)
            e1.record()
            f3s.synchronize()
            times.append(e0.elapsed_ms(e1))
        best = min(times)
        # and a plain fill of the same buffer (f3s_memset): the write-only rate
        fills = []
        for _ in range(args.steps):
            e0.record()
            dst.fill_bytes(0x5A)
            e1.record()
            f3s.synchronize()
            fills.append(e0.elapsed_ms(e1))
        # read + write bytes over the fastest copy: the practical HBM rate
        print(json.dumps({"copy_probe_bytes": nb, "launches": args.steps,
                          "copy_ms": times, "copy_GBps_rw": 2 * nb / best / 1e6,
                          "fill_ms": fills, "fill_GBps_w": nb / min(fills) / 1e6}), flush=True)
        return 0
    if args.gather_probe:
        # uniformly random 128-byte K and V rows, the config-4 pass's column
        # count, tables from L2-resident (1 MB each) to past the Infinity
        # Cache (512 MB each); on the 1,000,000-row tables also 16-row runs
        # (a tile-dense pass's tiles) and rows in order
        f3s.init()
        stream = f3s.Stream()
        for rows in (8192, 1_000_000, 4_000_000):
            tk = f3s.DeviceArray((rows, 64), np.uint16, zero=True)
            tv = f3s.DeviceArray((rows, 64), np.uint16, zero=True)
            for pattern in ("uniform", "tile16", "stream") if rows == 1_000_000 else ("uniform",):
                r = gather_ceiling(f3s, tk, tv, rows, 1, 16_907_486, stream,
                                   reps=max(3, args.steps), pattern=pattern)
                print(json.dumps({"gather_probe": r}), flush=True)
            del tk, tv
        return 0
    f3s.init()
    c = f3s.CONFIGS[args.config]
    if args.heads:
        import dataclasses
        c = dataclasses.replace(c, H=args.heads)
    masked = args.semantics == "masked"
    t0 = time.time()
    rp, ci = c.graph()
    n, H, d = c.n, c.H, c.d
    nnz = int(len(ci))
    Q, K, V = (c.features(t) for t in range(3))
    print(f"[bench] cfg{c.cfg} {c.name}: n={n} nnz={nnz} H={H} inputs in {time.time()-t0:.1f}s",
          file=sys.stderr, flush=True)

    stream = f3s.Stream()
    csr = f3s.DeviceCSR(rp, ci, stream)
    ev0, ev1 = f3s.Event(), f3s.Event()
    # converter (timed separately; not part of a step): end to end through
    # the Python wrapper (output allocation included; host wall time to
    # completion), the first call of the process and the median of four
    # later ones (the allocator then reuses the freed outputs), and the two
    # C-ABI phases alone into already allocated outputs
    conv_e2e = []
    bsf = None
    for _ in range(5):
        bsf = None
        f3s.synchronize()
        t_conv = time.perf_counter()
        bsf = f3s.convert_device(csr, masks=True, stream=stream)
        f3s.synchronize()
        conv_e2e.append((time.perf_counter() - t_conv) * 1e3)
    conv_e2e_first_ms, conv_e2e_ms = conv_e2e[0], float(np.median(conv_e2e[1:]))
    conv_ms = convert_phases_ms(csr, bsf, stream)
    use_sorted = args.order in ("sorted", "auto")
    order = f3s.window_order_device(bsf, stream) if use_sorted else None
    if args.order in LOCALITY_ORDERS:
        hb = bsf.to_host()
        order = f3s.DeviceArray.from_numpy(
            locality_order(args.order, rp, ci, hb.window_offsets, hb.block_col_indices), stream)
        del hb
    plan = None
    plan_ms = None
    compiled = masked and not args.no_compile and not args.unplanned

    def make_plan():
        p = f3s.Plan(bsf, order, H=H, seg_tiles=args.seg, stream=stream)
        if masked and not args.no_compile:
            p.compile(stream)
        return p

    plan_first_ms = None
    if not args.unplanned:
        # plan creation (+ compile) through the Python wrapper, host wall
        # time to completion: the first of the process and the median of
        # four later ones, as for the converter
        times = []
        for _ in range(5):
            plan = None
            f3s.synchronize()
            t_plan = time.perf_counter()
            plan = make_plan()
            f3s.synchronize()
            times.append((time.perf_counter() - t_plan) * 1e3)
        plan_first_ms, plan_ms = times[0], float(np.median(times[1:]))
    occ_sum, mask_bits = f3s.bsf_stats(bsf, masked, stream)
    dQ, dK, dV = (f3s.DeviceArray.from_numpy(x.view(np.uint16), stream) for x in (Q, K, V))
    dO = f3s.DeviceArray((n, H, d), np.float32)
    ps = plan.stats() if plan is not None else None
    if plan is not None:
        print(f"[bench] W={bsf.W} T={bsf.T} occ={occ_sum} items={plan.num_items} "
              f"split={plan.num_split} seg={plan.seg_tiles} convert={conv_ms:.2f}ms "
              f"plan={plan_ms:.2f}ms",
              file=sys.stderr, flush=True)

        def one_pass():
            plan.forward(dQ, dK, dV, dO, masked=masked, stream=stream)
    else:
        print(f"[bench] W={bsf.W} T={bsf.T} occ={occ_sum} unplanned convert={conv_ms:.2f}ms",
              file=sys.stderr, flush=True)

        def one_pass():
            f3s.attention_fwd(dQ, dK, dV, dO, bsf, order, masked=masked, H=H, d=d, stream=stream)

    # cold first launch (the reference times exactly this, tests/test_fused_3s_v2.cu:126-137)
    ev0.record(stream)
    one_pass()
    ev1.record(stream)
    cold_ms = ev0.elapsed_ms(ev1)
    for _ in range(args.warmup):
        one_pass()
    stream.synchronize()

    # timed region: K steps bracketed by synchronisation; one event pair per
    # launch on the launch stream gives the pass's own duration
    evs = [(f3s.Event(), f3s.Event()) for _ in range(args.steps)]
    f3s.synchronize()
    t_start = time.perf_counter()
    for a, b in evs:
        a.record(stream)
        one_pass()
        b.record(stream)
    stream.synchronize()
    f3s.synchronize()
    wall = time.perf_counter() - t_start
    kern_ms = np.array([a.elapsed_ms(b) for a, b in evs])
    ms_per_step = wall * 1e3 / args.steps
    kavg = float(kern_ms.mean())
    # the last timed pass's output, checked on every row in the CPU leg
    head_out = dO.numpy(stream)

    launch = "unplanned" if args.unplanned else "plan"
    kv_rows = {True: kv_rows_needed(n, ci, None, True)}
    hb_bcol = None
    if not masked or not args.no_reference_launches:
        hb_bcol = bsf.block_col.numpy()
        kv_rows[False] = kv_rows_needed(n, ci, hb_bcol, False)
    need = compulsory_bytes(n, H, bsf.W, bsf.T, kv_rows[masked], masked, launch, ps)
    achieved = need / (kavg * 1e-3) / 1e9
    gbytes = gather_model_bytes(n, bsf.W, bsf.T, occ_sum, H, d, masked)
    # matrix-core work: what the pass issues -- 8 MFMA 16x16x32 per chunk of
    # 32 gathered columns (masked: the attended columns, at least occ_sum / 32
    # chunks; tile-dense: two tiles per chunk) -- and the reference's tile
    # model (per active tile and head, S = Q K^T and O += P V, two products of
    # 16x16x64 at 2 flops per multiply-add), a work figure, not a rate
    flops_tile = bsf.T * 4 * 16 * 16 * d * H
    chunks = (occ_sum + 31) // 32 if masked else (bsf.T + 1) // 2
    flops_issued = chunks * H * 8 * (2 * 16 * 16 * 32)
    default_pass = (compiled and args.order == "auto" and args.seg == 0 and not args.heads)
    prof = ROOT / "profiles" / f"pmc_traffic_cfg{c.cfg}.txt"
    below = read_profile(prof, "bytes_per_launch") if default_pass else None
    below_us = read_profile(prof, "kernel_avg_us") if default_pass else None
    # provenance of the traffic figure: the commit and the digest of the
    # kernel's sources the profile measured, against the sources run here
    prof_digest = read_profile_field(prof, "sources_fused_attention") if below else None
    prof_commit = read_profile_field(prof, "commit") if below else None
    digest_now = source_digest("fused_attention")
    res = {
        "metric": "fused attention edges/s + kernel us; achieved HBM GB/s (% of peak) on 1 MI355X",
        "value": nnz * args.steps / wall,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 in, f32 accumulate/softmax/out",
        "data": "synthetic (seeded generator; no dataset download)",
        "config": {"workload": f"cfg{c.cfg}: {c.name}" + (f" with H={H}" if args.heads else ""), "nodes": n, "edges": nnz, "heads": H,
                   "head_dim": d, "semantics": args.semantics,
                   "window_order": ("descending workload" if use_sorted else
                                    args.order if args.order in LOCALITY_ORDERS else "natural"),
                   "launch": "f3s_attention_fwd (unplanned)" if args.unplanned else "plan",
                   "row_windows": bsf.W,
                   "active_tiles": bsf.T, "attended_tile_columns": occ_sum},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": below,
                     "bytes_per_launch": need,
                     "bytes_model": "compulsory: Q fp16 + O fp32 once per row, each needed K and "
                                    "V row once, launch metadata once (compiled chunk records "
                                    "256 B, items 16 B), split-window partials written and "
                                    "read back",
                     "traffic_kind": "rocprofv3 FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 per launch "
                                     "(copy-calibrated): traffic below the L2, HBM or the 256 MB "
                                     "Infinity Cache (no gfx950 counter separates them); read "
                                     "from the committed profile of this workload",
                     "traffic_source": str(prof.relative_to(ROOT)) if below else None,
                     "traffic_commit": prof_commit,
                     "traffic_sources_digest": prof_digest,
                     "sources_digest_now": digest_now,
                     "traffic_sources_current": (prof_digest == digest_now) if below else None},
        "gather_model": {"bytes_per_launch": gbytes, "GBps": gbytes / (kavg * 1e-3) / 1e9,
                         "note": "every gathered K/V row counted once per attending tile "
                                 "(the survey's model); L2 and the Infinity Cache serve part "
                                 "of it, so this rate can exceed the HBM peak"},
        "below_l2": ({"bytes_per_launch": below, "GBps": below / (kavg * 1e-3) / 1e9,
                      "frac_of_hbm_peak": below / (kavg * 1e-3) / 1e9 / HBM_PEAK_GBS,
                      "profiled_kernel_avg_us": below_us, "kind": "HBM + Infinity Cache",
                      "source": str(prof.relative_to(ROOT))} if below else None),
        "mfma": {"issued_tflop_per_pass": flops_issued / 1e12,
                 "issued_frac_of_peak": flops_issued / (kavg * 1e-3) / (MFMA_F16_PEAK_TFLOPS * 1e12),
                 "tile_model_tflop_per_pass": flops_tile / 1e12},
        "cpu_baseline": None,
        "cpu_baseline_all_cores": None,
        "kernel_us": {"mean": kavg * 1e3, "min": float(kern_ms.min()) * 1e3,
                      "median": float(np.median(kern_ms)) * 1e3, "cold_first_launch": cold_ms * 1e3},
        "converter_us": conv_ms * 1e3,
        "converter_end_to_end_us": conv_e2e_ms * 1e3,
        "converter_end_to_end_first_us": conv_e2e_first_ms * 1e3,
        "plan_us": plan_ms * 1e3 if plan_ms is not None else None,
        "plan_first_us": plan_first_ms * 1e3 if plan_first_ms is not None else None,
        "plan_compiled": compiled,
        "device": f3s.device_name(),
    }

    # the device's random-gather ceiling for this workload's tensors and column
    # count, beside the rate at which the pass gathers rows
    rows_pass = 2 * H * (occ_sum if masked else bsf.T * 16)
    gc = gather_ceiling(f3s, dK, dV, n, H, occ_sum, stream)
    gc["tile16_rows_per_s"] = gather_ceiling(f3s, dK, dV, n, H, occ_sum, stream,
                                             pattern="tile16")["rows_per_s"]
    gc["stream_rows_per_s"] = gather_ceiling(f3s, dK, dV, n, H, occ_sum, stream,
                                             pattern="stream")["rows_per_s"]

    def ceiling(sem_masked: bool) -> float:
        return gc["rows_per_s"] if sem_masked else gc["tile16_rows_per_s"]

    gc["pass_rows_per_s"] = rows_pass / (kavg * 1e-3)
    gc["pass_over_ceiling"] = gc["pass_rows_per_s"] / ceiling(masked)
    if res.get("below_l2") and H == 1:
        # the traffic below the L2 (reads and writes, from the committed
        # profile) against the rate at which the same loads read rows in
        # order (with one head the rows are contiguous)
        stream_gbs = gc["stream_rows_per_s"] * 128 / 1e9
        res["below_l2"]["frac_of_in_order_read_rate"] = res["below_l2"]["GBps"] / stream_gbs
    gc["note"] = ("f3s_probe_gather, the pass's load shape (K and V rows of 128 B, head 0) on the "
                  "workload's tensors: rows_per_s over uniformly random rows (a masked pass's "
                  "columns), tile16_rows_per_s over runs of 16 consecutive rows (a tile-dense "
                  "pass's tiles), stream_rows_per_s over rows in order; pass_over_ceiling divides "
                  "the pass's gathered K and V rows per head (masked: attended columns; "
                  "tile-dense: 16 per tile) per second by the ceiling of its semantics")
    res["gather_ceiling"] = gc

    legs, leg_outs = {}, {}
    if not args.no_reference_launches:
        # The reference's own semantics (tile-dense, src/fused3s_v2.cu:145-228)
        # and launch shape (every window whole, descending order, one launch:
        # tests/test_fused_3s_v2.cu:124-137) on the same inputs, after the
        # timed region; per-pass times from events on the launch stream.
        print("[bench] timing the reference's semantics and launch shapes ...", file=sys.stderr,
              flush=True)
        sorted_order = order if use_sorted else f3s.window_order_device(bsf, stream)
        occ_masked = occ_sum if masked else f3s.bsf_stats(bsf, True, stream)[0]
        ref_plan = plan if plan is not None else make_plan()
        rps = ref_plan.stats()
        reps_m = max(3, min(20, args.steps))
        reps_d = max(3, min(20, args.steps))

        def leg(name, fn, sem_masked, lnch, reps):
            dO.fill_bytes(0xFF, stream)   # NaN: a row the pass does not write cannot match
            t, cold = time_passes_cold(f3s, fn, stream, reps)
            mean = float(t.mean())
            leg_outs[name] = dO.numpy(stream)
            b = compulsory_bytes(n, H, bsf.W, bsf.T, kv_rows[sem_masked], sem_masked, lnch, rps)
            rows = 2 * H * (occ_masked if sem_masked else bsf.T * 16)
            legs[name] = {"semantics": "masked" if sem_masked else "tile_dense",
                          **pass_times(t, cold), "edges_per_s": nnz / (mean * 1e-3),
                          "compulsory_bytes": b,
                          "roofline_frac": b / (mean * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "gathered_rows_per_s": rows / (mean * 1e-3),
                          "over_gather_ceiling": rows / (mean * 1e-3) / ceiling(sem_masked)}

        leg("tile_dense_planned",
            lambda: ref_plan.forward(dQ, dK, dV, dO, masked=False, stream=stream),
            False, "plan", reps_d)
        for nm, sem in (("masked", True), ("tile_dense", False)):
            leg(f"dropin_descending_{nm}",
                lambda sem=sem: f3s.attention_fwd(dQ, dK, dV, dO, bsf, sorted_order, masked=sem,
                                                  H=H, d=d, stream=stream),
                sem, "unplanned", reps_m if sem else reps_d)
        leg("dropin_natural_masked",
            lambda: f3s.attention_fwd(dQ, dK, dV, dO, bsf, None, masked=True, H=H, d=d,
                                      stream=stream),
            True, "unplanned", reps_m)
        res["reference_launches"] = legs

    if not args.no_reference_launches:
        print("[bench] timing the flow from host memory ...", file=sys.stderr, flush=True)
        res["host_handover"] = host_handover(f3s, rp, ci, Q, K, V, n, H, d, masked)

    if not args.no_cpu_baseline:
        # The CPU leg, after every GPU timing: the reference's CPU baseline,
        # its restatement on all checker threads, and the checker -- the GPU
        # converter's output bit for bit and every timed pass's output on
        # every row, against the oracle (tests/test_fused_3s_v2.cu:137-155
        # checks the launch it timed the same way).
        orc = oracle_module()
        thr = check_threads()
        print("[bench] timing the reference CPU baseline ...", file=sys.stderr, flush=True)
        Qf, Kf, Vf = (x.astype(np.float32) for x in (Q, K, V))
        res["cpu_baseline"] = reference_single_thread(rp, ci, Qf, Kf, Vf, n, d)
        print("[bench] checking the converter and every timed output ...", file=sys.stderr,
              flush=True)
        ver = {"converter": converter_exact(orc, bsf, n, rp, ci)}
        t1 = time.perf_counter()
        want_m = orc.masked_attention(n, d, H, Qf, Kf, Vf, rp, ci, threads=thr)
        masked_s = time.perf_counter() - t1
        res["cpu_baseline_all_cores"] = {
            "value": nnz / masked_s, "unit": "edges/s", "cores": thr, "kind": "port",
            "sample": f"all {n} rows / {nnz} edges x {H} head(s): the masked oracle run that "
                      f"checks the timed passes, {masked_s:.2f} s on {thr} threads (OpenMP) of "
                      f"{len(os.sched_getaffinity(0))} available cores",
            "threads_used": thr, "cores_available": len(os.sched_getaffinity(0)),
            "cpu_model": host_cpu_model()}
        want_d = None
        if not masked or any(l["semantics"] == "tile_dense" for l in legs.values()):
            t1 = time.perf_counter()
            want_d = orc.tile_dense_attention(n, d, H, Qf, Kf, Vf, bsf.window_offsets.numpy(),
                                              bsf.block_col.numpy(), threads=thr, fast=True)
            dense_s = time.perf_counter() - t1
            res["tile_dense_oracle"] = {
                "tiles_per_s": bsf.T * H / dense_s, "threads": thr, "cpu_model": host_cpu_model(),
                "sample": f"every row: {bsf.T} tiles x {H} head(s), {dense_s:.2f} s on {thr} "
                          "threads (each window's 16 rows in AVX2 lanes, bit-identical to the "
                          "scalar restatement)"}
        ver["headline"] = compare_rows(head_out, want_m if masked else want_d)
        for name, out in leg_outs.items():
            legs[name]["check"] = compare_rows(out, want_m if legs[name]["semantics"] == "masked"
                                               else want_d)
        res["verification"] = ver
        del head_out, leg_outs, want_m, want_d, Qf, Kf, Vf
        cfgs = [int(x) for x in args.configs.split(",") if x.strip()] if args.configs else []
        if cfgs:
            res["configs"] = {}
        for k in cfgs:
            if k == c.cfg and not args.heads:
                continue
            res["configs"][f"cfg{k}"] = config_legs(f3s, orc, k, stream)
        res["verified"] = bool(
            ver["converter"]["tile_lists_bit_exact"] and ver["headline"]["ok"]
            and all(l["check"]["ok"] for l in legs.values())
            and all(v["verified"] for v in res.get("configs", {}).values()))
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
