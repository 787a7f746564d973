"""ctypes bindings of the two native libraries (include/f3s_capi.h,
include/f3s_host.h).

The libraries are loaded from this package directory (or, for the CPU
suite's sanitizer run, from the directory F3S_LIB_DIR names, which holds the
instrumented build); if one is missing the import of the binding fails loudly
(there is no Python or CPU fallback for any function of the path).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(os.environ.get("F3S_LIB_DIR") or Path(__file__).resolve().parent)

c_i32, c_i64, c_u64, c_f32, c_dbl = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_double
c_vp = C.c_void_p
P_i32 = C.POINTER(C.c_int32)
P_i64 = C.POINTER(C.c_int64)
P_f32 = C.POINTER(C.c_float)
P_vp = C.POINTER(C.c_void_p)

# name -> (restype, argtypes) for libf3s_hip.so
HIP_API = {
    "f3s_status_string": (C.c_char_p, [c_i32]),
    "f3s_last_error": (C.c_char_p, []),
    "f3s_abi_version": (c_i32, []),
    "f3s_init": (c_i32, []),
    "f3s_device_count": (c_i32, [P_i32]),
    "f3s_set_device": (c_i32, [c_i32]),
    "f3s_device_name": (c_i32, [C.c_char_p, c_i32]),
    "f3s_malloc": (c_i32, [P_vp, c_u64]),
    "f3s_free": (c_i32, [c_vp]),
    "f3s_release_cached_memory": (c_i32, []),
    "f3s_memcpy_h2d": (c_i32, [c_vp, c_vp, c_u64, c_vp]),
    "f3s_memcpy_d2h": (c_i32, [c_vp, c_vp, c_u64, c_vp]),
    "f3s_memcpy_d2d": (c_i32, [c_vp, c_vp, c_u64, c_vp]),
    "f3s_memset": (c_i32, [c_vp, c_i32, c_u64, c_vp]),
    "f3s_synchronize": (c_i32, [c_vp]),
    "f3s_stream_create": (c_i32, [P_vp]),
    "f3s_stream_destroy": (c_i32, [c_vp]),
    "f3s_event_create": (c_i32, [P_vp]),
    "f3s_event_destroy": (c_i32, [c_vp]),
    "f3s_event_record": (c_i32, [c_vp, c_vp]),
    "f3s_event_elapsed_ms": (c_i32, [c_vp, c_vp, P_f32]),
    "f3s_cast_f32_to_f16": (c_i32, [c_vp, c_vp, c_i64, c_vp]),
    "f3s_convert_csr_to_bsf": (c_i32, [c_vp, c_vp, c_i32, c_i64, c_vp, c_vp, c_vp, P_i64, c_vp]),
    "f3s_window_order": (c_i32, [c_vp, c_i32, c_vp, c_vp]),
    "f3s_bsf_stats": (c_i32, [c_vp, c_vp, c_i64, c_i32, P_i64, P_i64, c_vp]),
    "f3s_attention_fwd": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                  c_i32, c_i32, c_i32, c_i32, c_f32, c_vp]),
    "f3s_attention_fwd_noalloc": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                          c_i32, c_i32, c_i32, c_i32, c_f32, c_vp]),
    "f3s_attention_fwd_timed": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                        c_i32, c_i32, c_i32, c_i32, c_f32, c_vp, c_i32,
                                        C.POINTER(c_f32)]),
    "f3s_naive_attention_fwd": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_f32,
                                        c_vp]),
    "f3s_plan_create": (c_i32, [c_vp, c_vp, c_i32, c_i32, c_i32, c_vp, P_vp]),
    "f3s_plan_destroy": (c_i32, [c_vp]),
    "f3s_plan_compile": (c_i32, [c_vp, c_vp, c_vp, c_i32, c_vp]),
    "f3s_plan_info": (c_i32, [c_vp, P_i64, P_i64, P_i64, P_i32]),
    "f3s_plan_stats": (c_i32, [c_vp, P_i64, P_i64, P_i64, P_i64, P_i64]),
    "f3s_attention_fwd_planned": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                          c_i32, c_i32, c_i32, c_f32, c_vp]),
    "f3s_probe_gather": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_vp, c_i64, c_i32, c_vp, c_vp]),
}

# name -> (restype, argtypes) for libf3s_host.so
HOST_API = {
    "f3s_host_free": (None, [c_vp]),
    "f3s_host_last_error": (C.c_char_p, []),
    "f3s_host_load_csr": (c_i32, [C.c_char_p, P_i32, P_i64, C.POINTER(P_i32), C.POINTER(P_i32)]),
    "f3s_host_window_order": (c_i32, [c_vp, c_i32, c_vp]),
    "f3s_gen_powerlaw": (c_i32, [c_i32, c_i64, c_dbl, c_dbl, c_i32, c_i32, c_u64,
                                 C.POINTER(P_i32), C.POINTER(P_i32), P_i64]),
    "f3s_gen_sbm": (c_i32, [c_i32, c_i32, c_dbl, c_dbl, c_i32, c_u64,
                            C.POINTER(P_i32), C.POINTER(P_i32), P_i64]),
    "f3s_gen_features_f16": (c_i32, [c_u64, c_i32, c_i64, c_i32, c_vp]),
    "f3s_host_f16_to_f32": (None, [c_vp, c_vp, c_i64]),
    "f3s_host_save_graph": (c_i32, [C.c_char_p, c_i32, c_i64, c_vp, c_vp, c_i32, c_i64,
                                    c_vp, c_vp, c_vp]),
    "f3s_host_load_graph": (c_i32, [C.c_char_p, P_i32, P_i64, C.POINTER(P_i32),
                                    C.POINTER(P_i32), P_i32, P_i64, C.POINTER(P_i32),
                                    C.POINTER(P_i32), C.POINTER(C.POINTER(C.c_uint16))]),
}


def _bind(lib: C.CDLL, api: dict) -> C.CDLL:
    for name, (res, args) in api.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_hip = None
_host = None


def hip() -> C.CDLL:
    """libf3s_hip.so, loaded once.  Raises if it was not built."""
    global _hip
    if _hip is None:
        path = PKG / "libf3s_hip.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run `python -m fused3s_amd.build` "
                               "(the HIP path has no fallback)")
        _hip = _bind(C.CDLL(str(path)), HIP_API)
    return _hip


def host() -> C.CDLL:
    """libf3s_host.so, loaded once (after libf3s_hip.so, which it links)."""
    global _host
    if _host is None:
        hip()
        path = PKG / "libf3s_host.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run `python -m fused3s_amd.build`")
        _host = _bind(C.CDLL(str(path)), HOST_API)
    return _host
