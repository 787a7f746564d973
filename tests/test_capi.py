"""Host-side checks that need no GPU: the C-ABI libraries load and export
every declared entry point, argument validation and no-device behaviour,
the host loader / window order / generators, and the harness and bench
entry behaviour."""
from __future__ import annotations

import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import GOLDEN, ROOT

import fused3s_amd as f3s
from fused3s_amd import _lib


def declared(header: Path) -> list[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(f3s_[a-z0-9_]+)\s*\(", text)
    return sorted(set(n for n in names if n not in ("f3s_status",)))


@pytest.mark.parametrize("header,lib", [("f3s_capi.h", "libf3s_hip.so"),
                                        ("f3s_host.h", "libf3s_host.so")])
def test_library_exports_every_declared_symbol(header, lib):
    names = declared(ROOT / "include" / header)
    assert len(names) >= 8
    so = C.CDLL(str(ROOT / "fused3s_amd" / lib))
    missing = [n for n in names if not hasattr(so, n)]
    assert not missing, f"{lib} lacks {missing}"
    # and the Python binding declares each of them
    api = _lib.HIP_API if lib == "libf3s_hip.so" else _lib.HOST_API
    assert set(names) <= set(api), set(names) - set(api)


def test_status_strings_and_abi():
    h = _lib.hip()
    assert h.f3s_abi_version() == 1
    for s in range(7):
        assert h.f3s_status_string(s).startswith(b"F3S")


def test_validation_happens_before_device_access():
    h = _lib.hip()
    # d != 64 and bad H are rejected with F3S_EUNSUPPORTED on any host
    assert h.f3s_attention_fwd(None, None, None, None, None, None, None, None,
                               1, 16, 32, 1, 1.0, None) == 5
    for bad_h in (0, 65):
        assert h.f3s_attention_fwd(None, None, None, None, None, None, None, None,
                                   1, 16, 64, bad_h, 1.0, None) == 5
    # misaligned pointers are F3S_EINVAL
    assert h.f3s_attention_fwd(8, 16, 16, 16, 16, 16, None, None, 1, 16, 64, 1, 1.0, None) == 1
    us = C.c_float()
    assert h.f3s_attention_fwd_timed(None, None, None, None, None, None, None, None,
                                     1, 16, 64, 1, 1.0, None, 0, C.byref(us)) == 1   # reps < 1
    assert h.f3s_attention_fwd_timed(None, None, None, None, None, None, None, None,
                                     1, 16, 64, 1, 1.0, None, 3, None) == 1          # no us_out
    T = C.c_int64()
    assert h.f3s_convert_csr_to_bsf(None, None, -1, 0, None, None, None, C.byref(T), None) == 1
    assert h.f3s_cast_f32_to_f16(None, None, -1, None) == 1


def test_no_device_is_reported_not_faked():
    # decided at run time, not at collection: no HIP call while collecting
    if f3s.device_count() > 0:
        pytest.skip("checks the no-GPU behaviour")
    h = _lib.hip()
    p = C.c_void_p()
    assert h.f3s_malloc(C.byref(p), 16) == 4      # F3S_ENODEV
    assert b"no HIP device" in h.f3s_last_error()
    with pytest.raises(f3s.F3SError) as e:
        f3s.DeviceArray(4, np.float32)
    assert e.value.name == "F3S_ENODEV"


@pytest.mark.parametrize("name,n,nnz", [("cora", 2708, 10556), ("citeseer", 3327, 9104)])
def test_load_csr_graph(name, n, nnz):
    g = f3s.load_csr_graph(str(GOLDEN / name))
    assert (g.num_nodes, g.num_edges) == (n, nnz)
    assert np.array_equal(g.row_ptr, np.loadtxt(GOLDEN / name / "row_ptr.txt", dtype=np.int32))
    assert np.array_equal(g.col_ind, np.loadtxt(GOLDEN / name / "col_idx.txt", dtype=np.int32))


def test_load_csr_graph_errors_are_loud(tmp_path):
    with pytest.raises(RuntimeError, match="meta.txt"):
        f3s.load_csr_graph(str(tmp_path / "nope"))
    d = tmp_path / "g"
    d.mkdir()
    (d / "meta.txt").write_text("3 4\n")
    (d / "row_ptr.txt").write_text("0\n1\n3\n4\n")
    with pytest.raises(RuntimeError, match="col_idx"):
        f3s.load_csr_graph(str(d))
    (d / "col_ind.txt").write_text("1 0 2 1\n")          # the reference's file name
    assert list(f3s.load_csr_graph(str(d)).col_ind) == [1, 0, 2, 1]
    (d / "col_ind.txt").write_text("1 0 7 1\n")          # column >= n
    with pytest.raises(RuntimeError, match="column"):
        f3s.load_csr_graph(str(d))


def test_host_window_order_is_reference_sort():
    offs = np.array([0, 3, 3, 7, 8, 11, 11, 15], np.int32)
    fmt = f3s.BlockSparseFormat(7, offs, np.zeros(15, np.int32))
    order = f3s.generate_balanced_window_order(fmt)
    cnt = np.diff(offs)
    assert sorted(order.tolist()) == list(range(7))
    assert np.all(np.diff(cnt[order]) <= 0)


def test_generators_deterministic_and_well_formed():
    a = f3s.CONFIGS[3].graph()
    b = f3s.CONFIGS[3].graph()
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    for cfg in (2, 3):
        rp, ci = f3s.CONFIGS[cfg].graph()
        n = len(rp) - 1
        assert rp[0] == 0 and np.all(np.diff(rp) >= 1)            # self-loop on every row
        rows = np.repeat(np.arange(n), np.diff(rp))
        for u in range(0, n, 97):
            r = ci[rp[u]:rp[u + 1]]
            assert np.all(np.diff(r) > 0) and u in r              # sorted unique, self-loop
        key = set(zip(rows.tolist(), ci.tolist()))
        assert all((v, u) in key for (u, v) in list(key)[:2000])  # symmetric
    rp, ci = f3s.CONFIGS[2].graph()
    e = len(ci) - 2708
    assert 10000 <= e <= 11000, e                                  # ~10,556 directed edges
    rp, ci = f3s.CONFIGS[3].graph()
    deg = np.diff(rp)
    assert 8500 <= len(ci) - 3327 <= 9700 and (deg == 1).sum() > 300   # many isolated


def test_sbm_generator_small():
    rp, ci = f3s.graph.sbm_graph(20000, 4096, 50.0, 0.8, True, 5)
    n = 20000
    rows = np.repeat(np.arange(n), np.diff(rp))
    intra = (rows // 4096) == (ci // 4096)
    frac = intra[rows != ci].mean()
    assert 0.78 < frac < 0.86          # 80 % intra + random hits in the own community
    assert 45 < (len(ci) - n) / n < 52


def test_feature_generator():
    q = f3s.graph.features_f16(1, 0, 100000, normal=True).astype(np.float64)
    assert abs(q.mean()) < 0.02 and abs(q.std() - 1) < 0.02
    u = f3s.graph.features_f16(1, 1, 100000, normal=False).astype(np.float64)
    assert u.min() >= -1 and u.max() <= 1 and abs(u.mean()) < 0.01
    assert np.array_equal(f3s.graph.features_f16(1, 2, 1000, False),
                          f3s.graph.features_f16(1, 2, 1000, False))
    assert not np.array_equal(f3s.graph.features_f16(1, 1, 1000, False),
                              f3s.graph.features_f16(1, 2, 1000, False))


def test_harness_needs_gpu():
    exe = ROOT / "tests" / "cpp" / "bin" / "test_fused_3s"
    if not exe.exists():
        pytest.skip("harness not built")
    if f3s.device_count() > 0:
        pytest.skip("checks the no-GPU behaviour")
    r = subprocess.run([str(exe), str(GOLDEN / "cora")], capture_output=True, text=True)
    assert r.returncode == 2 and "no GPU" in r.stderr


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def _bench():
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_checker_flags_errors_and_unwritten_rows():
    """bench.py's row checker: the north star's bounds (2e-3 abs, 1e-2
    normwise rel), a NaN (an unwritten row) always fails, an exact copy
    passes with zero error."""
    b = _bench()
    want = np.random.default_rng(3).standard_normal((1000, 2, 64)).astype(np.float32)
    ok = b.compare_rows(want.copy(), want)
    assert ok["ok"] and ok["max_abs"] == 0.0 and ok["rows"] == "every row"
    near = want.copy()
    near[7, 1, 3] += 1.5e-3
    assert b.compare_rows(near, want)["ok"]
    far = want.copy()
    far[999, 0, 63] += 3e-3
    r = b.compare_rows(far, want)
    assert not r["ok"] and abs(r["max_abs"] - 3e-3) < 1e-6
    nan = want.copy()
    nan[500] = np.nan
    r = b.compare_rows(nan, want)
    assert not r["ok"] and r["non_finite"] == 128


def test_profiles_record_their_sources():
    """Every committed profile names the commit it measured and the digests
    of the kernel sources; bench.py reads them, and --print-source-digests
    prints the current ones in the same form."""
    b = _bench()
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--print-source-digests"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0
    now = dict(line.split() for line in r.stdout.splitlines())
    assert set(now) == {f"sources_{k}" for k in b.KERNEL_SOURCES}
    for prof in sorted((ROOT / "profiles").glob("*.txt")):
        commit = b.read_profile_field(prof, "commit")
        assert commit and len(commit) >= 7, prof.name
        for k in b.KERNEL_SOURCES:
            d = b.read_profile_field(prof, f"sources_{k}")
            assert d and len(d) == 16, (prof.name, k)
