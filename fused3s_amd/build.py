"""Builds the native libraries in-tree.

* ``fused3s_amd/libf3s_hip.so``  -- HIP kernels + C-ABI (hipcc, gfx950 only)
* ``fused3s_amd/libf3s_host.so`` -- host C++ (loader, order, generators,
  drop-in C++ API); links libf3s_hip.so
* ``tests/cpp/bin/test_fused_3s`` -- the C++ launch/verify harness (the
  counterpart of the reference's tests/test_fused_3s_v2.cu), when the
  oracle library is present
* ``oracle/`` via ``make -C oracle`` (test infrastructure)
* ``tests/cpp/bin/libl2model.so`` -- the L2 cache model of tests/test_l2_bound.py

Run ``python -m fused3s_amd.build``.  Objects go to ``fused3s_amd/_build``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
HIP_SOURCES = ["runtime.hip", "convert.hip", "attention.hip", "bsf_util.hip", "naive.hip",
               "probe.hip"]
HOST_SOURCES = ["host/gen.cpp", "host/graph.cpp", "host/graph_file.cpp"]
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed FP32 VALU forms are kept out of the code objects.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fopenmp", "-Wall", "-Wextra"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build_hip(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        for src in HIP_SOURCES:
            obj = OBJ / (Path(src).stem + ".o")
            objs.append(obj)
            cmd = [HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
            jobs.append(ex.submit(_run, cmd, verbose))
        for j in jobs:
            j.result()
    out = PKG / "libf3s_hip.so"
    tmp = PKG / "libf3s_hip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def build_host(verbose: bool = True) -> Path:
    out = PKG / "libf3s_host.so"
    tmp = PKG / "libf3s_host.so.tmp"
    cmd = ["g++", *HOST_FLAGS, "-shared", *(str(CSRC / s) for s in HOST_SOURCES),
           "-L", str(PKG), "-lf3s_hip", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


SAN_DIR = OBJ / "san"
SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=undefined"]


def build_host_sanitized(verbose: bool = True) -> Path:
    """ASan + UBSan build of libf3s_host.so in fused3s_amd/_build/san/, beside
    a link to the normal libf3s_hip.so (the HIP library is not instrumented),
    for the CPU suite's sanitizer run (tests/sanitize.sh, which loads the
    libraries from that directory through F3S_LIB_DIR)."""
    SAN_DIR.mkdir(parents=True, exist_ok=True)
    hip = SAN_DIR / "libf3s_hip.so"
    if hip.is_symlink() or hip.exists():
        hip.unlink()
    hip.symlink_to(PKG / "libf3s_hip.so")
    out = SAN_DIR / "libf3s_host.so"
    flags = [f for f in HOST_FLAGS if f != "-O3"] + SAN_FLAGS
    cmd = ["g++", *flags, "-shared", *(str(CSRC / s) for s in HOST_SOURCES),
           "-L", str(SAN_DIR), "-lf3s_hip", "-Wl,-rpath,$ORIGIN", "-o", str(out)]
    _run(cmd, verbose)
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], verbose)
    return out


def build_oracle(verbose: bool = True) -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle")], verbose)


HARNESSES = ["test_fused_3s", "test_baselines"]


def build_harness(verbose: bool = True) -> list[Path]:
    """The C++ harness binaries (tests/cpp/*.cpp); they link the oracle."""
    outs = []
    for name in HARNESSES:
        out = _build_one_harness(name, verbose)
        if out:
            outs.append(out)
    return outs


def _build_one_harness(name: str, verbose: bool) -> Path | None:
    src = ROOT / "tests" / "cpp" / f"{name}.cpp"
    if not src.exists() or not (ROOT / "oracle" / "liboracle.so").exists():
        return None
    bindir = ROOT / "tests" / "cpp" / "bin"
    bindir.mkdir(parents=True, exist_ok=True)
    out = bindir / name
    cmd = ["g++", "-O2", "-std=c++17", "-fopenmp", "-Wall", str(src),
           "-I", str(ROOT / "include"), "-I", str(ROOT / "oracle"),
           "-L", str(PKG), "-lf3s_host", "-lf3s_hip",
           "-L", str(ROOT / "oracle"), "-loracle",
           f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{ROOT / 'oracle'}",
           "-Wl,-rpath,$ORIGIN/../../../fused3s_amd", "-Wl,-rpath,$ORIGIN/../../../oracle",
           "-o", str(out)]
    _run(cmd, verbose)
    return out


def build_l2_model(verbose: bool = True) -> Path:
    """The test-side L2 cache model (tests/cpp/l2_model.cpp), a plain shared
    library for tests/test_l2_bound.py."""
    bindir = ROOT / "tests" / "cpp" / "bin"
    bindir.mkdir(parents=True, exist_ok=True)
    out = bindir / "libl2model.so"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          str(ROOT / "tests" / "cpp" / "l2_model.cpp"), "-o", str(out)], verbose)
    return out


def build_all(verbose: bool = True) -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_hip(verbose)
    build_host(verbose)
    build_oracle(verbose)
    build_harness(verbose)
    build_l2_model(verbose)


if __name__ == "__main__":
    if "--sanitize" in sys.argv:
        build_host_sanitized(verbose="-q" not in sys.argv)
    else:
        build_all(verbose="-q" not in sys.argv)
