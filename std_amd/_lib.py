"""ctypes binding of libstdhip.so (the C ABI in include/std_hip.h).

The library is loaded from ``std_amd/_lib/libstdhip.so`` (built in-tree by
``std_amd.build``). There is no fallback: if the library is missing every op
raises, so a run can never silently compute on another path.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import c_double, c_float, c_int, c_int32, c_longlong, c_size_t, c_void_p, POINTER
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libstdhip.so"

STD_F32 = 0
STD_BF16 = 1
STD_F16 = 2

STD_STATUS_CACHE_OVERFLOW = 1    # device status word bit: a row or length past the cache capacity

STATUS_NAMES = {
    -1: "STD_E_NULL",
    -2: "STD_E_DTYPE",
    -3: "STD_E_SHAPE",
    -4: "STD_E_WORKSPACE",
    -5: "STD_E_ALIGN",
    -6: "STD_E_RANGE",
}

# name -> (restype, argtypes); mirrors include/std_hip.h
SIGNATURES = {
    "std_status_string": (ctypes.c_char_p, [c_int]),
    "std_version": (c_int, []),
    "std_gqa_decode_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "std_attn_split_count": (c_int, [c_int, c_int, c_int, c_int]),
    "std_gqa_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                               c_longlong, c_longlong, c_float, c_int, c_void_p, c_size_t, c_void_p]),
    "std_gqa_decode_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                       c_longlong, c_longlong, c_float, c_int, c_void_p]),
    "std_gqa_decode_batched_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "std_gqa_decode_batched": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                       c_longlong, c_longlong, c_longlong, c_longlong, c_longlong, c_longlong,
                                       c_float, c_int, c_void_p, c_size_t, c_void_p]),
    "std_gqa_decode_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                      c_int, c_int, c_longlong, c_longlong, c_longlong, c_float, c_int, c_void_p,
                                      c_size_t, c_void_p]),
    "std_verify_attn_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "std_verify_attn_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                       c_int, c_int, c_int, c_longlong, c_longlong, c_longlong, c_longlong, c_float,
                                       c_int, c_void_p, c_size_t, c_void_p]),
    "std_verify_attn": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                c_longlong, c_longlong, c_float, c_int, c_void_p, c_size_t, c_void_p]),
    "std_verify_attn_collect_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "std_verify_attn_collect": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                        c_int, c_int, c_int, c_longlong, c_longlong, c_longlong, c_longlong, c_float,
                                        c_int, c_int, c_int, c_void_p, c_longlong, c_void_p, c_size_t, c_void_p]),
    "std_verify_attn_collect_ex": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                           c_int, c_int, c_void_p, c_int, c_longlong, c_longlong, c_longlong,
                                           c_longlong, c_float, c_int, c_int, c_int, c_void_p, c_void_p, c_int,
                                           c_void_p, c_longlong, c_void_p, c_size_t, c_void_p, c_void_p]),
    "std_select_topk_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "std_select_topk": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_longlong, c_int,
                                c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "std_select_topk_probs_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "std_select_topk_probs": (c_int, [c_void_p, c_longlong, c_longlong, c_int, c_int, c_int, c_int, c_int, c_void_p,
                                      c_int, c_int, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "std_build_compact_index": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "std_compact_kv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                               c_longlong, c_int, c_longlong, c_int, c_int, c_void_p]),
    "std_kv_append": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_longlong,
                              c_longlong, c_longlong, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "std_len_add": (c_int, [c_void_p, c_int, c_int, c_void_p]),
    "std_gqa_decode_indexed": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_longlong, c_longlong, c_void_p,
                                       c_longlong, c_int, c_void_p, c_void_p, c_longlong, c_longlong, c_void_p,
                                       c_int, c_int, c_int, c_void_p, c_int, c_float, c_int, c_void_p, c_size_t,
                                       c_void_p, c_void_p]),
    "std_gemv_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "std_gemv": (c_int, [c_void_p, c_longlong, c_void_p, c_longlong, c_void_p, c_void_p, c_longlong, c_int, c_int,
                         c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "std_gemv_ex": (c_int, [c_void_p, c_longlong, c_void_p, c_longlong, c_void_p, c_void_p, c_longlong, c_void_p,
                            c_longlong, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "std_gemv_norm": (c_int, [c_void_p, c_void_p, c_float, c_void_p, c_longlong, c_void_p, c_void_p, c_void_p, c_int,
                              c_int, c_int, c_int, c_void_p]),
    "std_qkv_rope_append": (c_int, [c_void_p, c_longlong, c_int, c_int, c_void_p, c_longlong, c_void_p, c_int, c_int,
                                    c_int, c_void_p, c_void_p, c_void_p, c_longlong, c_int, c_void_p, c_void_p, c_int,
                                    c_void_p, c_void_p, c_float, c_int, c_void_p, c_void_p]),
    "std_argmax_rows": (c_int, [c_void_p, c_longlong, c_int, c_int, c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "std_rms_norm": (c_int, [c_void_p, c_longlong, c_void_p, c_void_p, c_longlong, c_int, c_int, c_float, c_int,
                             c_void_p]),
    "std_rope_append": (c_int, [c_void_p, c_longlong, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                c_longlong, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "std_attn_devlen": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_int,
                                c_longlong, c_longlong, c_float, c_int, c_void_p, c_size_t, c_void_p, c_void_p]),
    "std_greedy_accept_workspace_bytes": (c_size_t, [c_int, c_int]),
    "std_stream_read": (c_int, [c_void_p, c_size_t, c_int, c_int, c_void_p, c_void_p]),
    "std_greedy_accept": (c_int, [c_void_p, c_longlong, c_int, c_int, c_int, c_void_p, c_int, c_int, c_void_p,
                                  c_void_p, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
}

_lock = threading.Lock()
_lib = None


class StdHipError(RuntimeError):
    """A nonzero status from libstdhip.so."""

    def __init__(self, fn: str, status: int, text: str):
        self.fn = fn
        self.status = status
        name = STATUS_NAMES.get(status, "hipError" if status > 0 else "unknown")
        super().__init__(f"{fn} failed with status {status} ({name}): {text}")


def library_path() -> Path:
    return LIB_PATH


def load_library():
    """Load and bind libstdhip.so; raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m std_amd.build` "
                "(the HIP path has no fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols():
    return sorted(SIGNATURES)


def check(fn_name: str, status: int) -> None:
    if status != 0:
        text = load_library().std_status_string(status).decode()
        raise StdHipError(fn_name, status, text)


def call(fn_name: str, *args) -> None:
    """Call an int-returning entry point and raise StdHipError on failure."""
    check(fn_name, getattr(load_library(), fn_name)(*args))
