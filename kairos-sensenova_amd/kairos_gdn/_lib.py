"""ctypes binding of libkairos_gdn.so (the C ABI declared in include/kairos_gdn.h).

The library is the only compute path: if it is missing or cannot be loaded,
every entry point raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libkairos_gdn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

F32, BF16, F8E4M3 = 0, 1, 2
ACT_SWISH, ACT_SIGMOID = 0, 1
OK, EINVAL, EUNSUPPORTED, EWORKSPACE, EHIP = 0, 1, 2, 3, 4
ABI_VERSION = 2

# every symbol the header declares, with (restype, argtypes)
_p = ctypes.c_void_p
_fp = ctypes.c_void_p          # float* passed as a raw address
_i64 = ctypes.c_int64
_i = ctypes.c_int
_sz = ctypes.c_size_t
_f = ctypes.c_float

SIGNATURES = {
    "kairos_gdn_abi_version": (_i, []),
    "kairos_gdn_last_error": (ctypes.c_char_p, []),
    "kairos_gdn_num_chunks_bound": (_i64, [_i64, _i64, _i64]),
    "kairos_gdn_chunk_fwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _i]),
    "kairos_gdn_chunk_fwd_gated_norm_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _i]),
    "kairos_gdn_chunk_fwd": (_i, [_p, _p, _p, _p, _p, _fp, _fp, _p, _p, _fp, _p, _i64,
                                  _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _i, _f, _i, _p, _sz, _p]),
    "kairos_gdn_chunk_fwd_gated_norm": (_i, [_p, _p, _p, _p, _p, _fp, _fp, _p, _p, _p, _p, _p, _fp, _p, _i64,
                                             _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _i, _i, _i, _f, _i,
                                             _f, _i, _p, _sz, _p]),
    "kairos_gdn_chunk_fwd_noalloc": (_i, [_p, _p, _p, _p, _p, _fp, _fp, _p, _p, _fp, _p, _i64,
                                         _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _i, _f, _i, _p]),
    "kairos_gdn_chunk_fwd_noalloc_max_bytes": (_sz, []),
    "kairos_gdn_chunk_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _i]),
    "kairos_gdn_chunk_bwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _fp, _p, _p, _p, _fp, _p, _fp, _p, _i64, _i64,
                                  _i64, _i64, _i64, _i64, _i, _i, _i, _i, _i, _f, _i, _p, _sz, _p]),
    "kairos_gdn_stage_workspace_size": (_sz, [_i64]),
    "kairos_gdn_chunk_local_cumsum": (_i, [_p, _i, _fp, _p, _i64, _i64, _i64, _i64, _p, _sz, _p]),
    "kairos_gdn_prepare_wy": (_i, [_p, _p, _p, _p, _fp, _fp, _p, _p, _fp, _p, _p, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _p, _sz, _p]),
    "kairos_gdn_fwd_h": (_i, [_p, _fp, _p, _p, _fp, _p, _p, _p, _fp, _p, _i64,
                              _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _p, _sz, _p]),
    "kairos_gdn_fwd_o": (_i, [_p, _p, _fp, _fp, _p, _p, _fp, _p, _f, _p, _i64,
                              _i64, _i64, _i64, _i64, _i64, _i, _i, _p, _sz, _p]),
    "kairos_gdn_stage_tokens_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i]),
    "kairos_gdn_prepare_wy_tokens": (_i, [_p, _p, _p, _p, _fp, _fp, _p, _p, _fp, _p, _p, _i64,
                                          _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _p, _sz, _p]),
    "kairos_gdn_fwd_h_tokens": (_i, [_p, _fp, _p, _p, _fp, _p, _p, _p, _fp, _p, _i64,
                                     _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _p, _sz, _p]),
    "kairos_gdn_fwd_o_tokens": (_i, [_p, _p, _fp, _fp, _p, _p, _fp, _p, _f, _p, _i64,
                                     _i64, _i64, _i64, _i64, _i64, _i, _i, _p, _sz, _p]),
    "kairos_gdn_l2norm_fwd": (_i, [_p, _p, _p, _i, _i64, _i64, _p]),
    "kairos_gdn_rms_norm_gated": (_i, [_p, _p, _p, _p, _p, _fp, _i, _i, _i, _i64, _i64, _f, _i, _p]),
    "kairos_gdn_fused_recurrent_fwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _fp, _p, _i64, _i64, _i64, _i64,
                                            _i64, _i64, _i64, _i, _i, _i, _i, _i, _i, _i, _i, _f, _i, _p]),
    "kairos_gdn_causal_conv1d_fwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i, _i, _i, _i,
                                          _p]),
    "kairos_gdn_chunk_fwd_conv_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64, _i]),
    "kairos_gdn_chunk_fwd_conv": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i,
                                       _p, _p, _p, _p, _fp, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _i,
                                       _f, _i, _p, _sz, _p]),
    "kairos_gdn_gates_fwd": (_i, [_p, _p, _p, _p, _fp, _p, _i64, _i64, _i, _i, _i, _i, _p]),
    "kairos_gdn_segment_chunks": (_i, [_i64, _i64, _i64, _i64]),
    "kairos_gdn_varlen_maps": (_i, [_p, _i64, _i64, _p, _p, _p]),
    "kairos_gdn_profile_begin": (_i, []),
    "kairos_gdn_profile_end": (_i, [ctypes.POINTER(ctypes.c_double), _i]),
}

_lock = threading.Lock()
_lib = None


class KairosGdnError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


def load(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and return the native library with typed entry points."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        # torch ships its own HIP runtime (libamdhip64.so.7, libhsa-runtime64.so.1); importing it
        # first makes this library bind to that same copy by soname, so the process has one runtime.
        import torch  # noqa: F401
        if not os.path.exists(p):
            raise RuntimeError(
                f"{LIB_NAME} is not built ({p} missing): run `python kairos-sensenova_amd/kairos_gdn/build.py` "
                "(or __graft_entry__.build()); there is no fallback path")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.kairos_gdn_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI version {lib.kairos_gdn_abi_version()} != {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def check(fn_name: str, rc: int) -> None:
    if rc != OK:
        msg = load().kairos_gdn_last_error()
        raise KairosGdnError(fn_name, rc, msg.decode() if msg else "")


def call(fn_name: str, *args) -> None:
    lib = load()
    check(fn_name, getattr(lib, fn_name)(*args))
