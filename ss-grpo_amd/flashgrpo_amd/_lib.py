"""ctypes binding of libflashgrpo_amd.so (the C ABI declared in include/flashgrpo_amd.h).

The library is loaded after torch so that both share torch's HIP runtime (the
bundled libamdhip64.so.7 satisfies the library's dependency by soname). A
missing library raises immediately: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

from ._build import LIB_PATH

_P = C.c_void_p
_I = C.c_int
_I64 = C.c_int64
_SZ = C.c_size_t
_F = C.c_float
_U32 = C.c_uint32
_U64 = C.c_uint64

# name -> (restype, argtypes); mirrors include/flashgrpo_amd.h
SIGNATURES = {
    "fg_last_error": (C.c_char_p, []),
    "fg_version": (_I, []),
    "fg_medusa_heads_workspace": (_SZ, [_I, _I, _I, _I]),
    "fg_medusa_heads": (_I, [_P, _I, _I, _I, _I64, _I, _P, _P, _F, _P, _P, _P, _I, _P, _SZ, _P]),
    "fg_lm_head": (_I, [_P, _I, _I, _I, _I64, _P, _P, _P, _I64, _I, _P, _I, _I64, _P]),
    "fg_lm_head_topk_workspace": (_SZ, [_I, _I, _I]),
    "fg_lm_head_topk_parts": (_I, [_I]),
    "fg_lm_head_topk": (_I, [_P, _I, _I, _I64, _P, _P, _P, _I64, _I, _P, _I, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _SZ,
                             _P]),
    "fg_medusa_topk_workspace": (_SZ, [_I, _I, _I]),
    "fg_medusa_topk": (_I, [_P, _I, _I64, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P]),
    "fg_tree_layout": (_I, [_P, _P, _I, _I, _P, _P, _P, _I, _P, _P, _I, _P]),
    "fg_sparse_tree_layout": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _F, C.c_double, _I, _P, _P, _P, _P, _P,
                                   _P, _P, _P, _P]),
    "fg_rope_kv_write": (_I, [_P, _I, _I64, _I, _I, _I, _I, _I, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I, _P,
                              _P, _P]),
    "fg_tree_attention_workspace": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "fg_tree_attention": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I64, _I64, _I, _P, _P, _P, _I64, _F, _P,
                               _SZ, _P]),
    "fg_rmsnorm": (_I, [_P, _P, _P, _P, _I, _I, _I, _F, _P]),
    "fg_swiglu": (_I, [_P, _P, _I, _I, _I, _P]),
    "fg_chain_cell_norm": (_I, [_P, _I64, _P, _I64, _I, _I, _I, _P, _P, _P, _P, _F, _P, _P]),
    "fg_gate_up_swiglu": (_I, [_P, _I64, _P, _I64, _P, _I64, _I, _I, _I, _I, _P]),
    "fg_linear_parts": (_I, [_P, _I64, _P, _I64, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "fg_residual_rmsnorm_parts": (_I, [_P, _I, _I, _I, _P, _I64, _P, _F, _P, _I64, _P]),
    "fg_rope_kv_write_parts": (_I, [_P, _I, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I,
                                    _P, _P, _P]),
    "fg_rope_cos_sin": (_I, [_P, _P, _I64, _P, _I, _I, _I, _P, _P]),
    "fg_linear_rope_kv_write": (_I, [_P, _I64, _P, _I64, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P,
                                    _P, _P, _P, _I64, _I64, _I, _P, _P, _P]),
    "fg_sample_workspace": (_SZ, [_I]),
    "fg_sample_tokens": (_I, [_P, _I, _I64, _I, _I, _P, _P, _P, _I, _I, _U64, _U64, _P, _I, _F, _I, _I, _U32, _P,
                              _P, _SZ, _P]),
    "fg_sample_tokens_noalloc_max_rows": (_SZ, []),
    "fg_sample_tokens_noalloc": (_I, [_P, _I, _I64, _I, _I, _P, _P, _P, _I, _I, _U64, _U64, _P, _I, _F, _I, _I, _U32,
                                      _P, _P]),
    "fg_accept_walk": (_I, [_P, _I, _I64, _I, _P, _P, _P, _P, _I, _I, _I, _P, _I, _I, _U64, _U64, _P, _I, _F, _I, _I,
                            _U32, _P, _P, _I, _P, _P, _P, _P, _P, _P]),
    "fg_walk_begin": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _P, _P, _P, _P, _P]),
    "fg_walk_rows": (_I, [_P, _I, _I, _P, _P, _P]),
    "fg_walk_step": (_I, [_P, _I, _I64, _I, _P, _P, _P, _I, _I, _I, _P, _I, _I, _U64, _U64, _P, _I, _F, _I, _I, _U32,
                          _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _SZ, _P]),
    "fg_accept_finalize": (_I, [_P, _P, _I, _P, _P, _P, _P, _I, _I, _P, _P, _I, _P]),
    "fg_kv_path_gather": (_I, [_P, _I, _I, _I, _I, _I, _I64, _I64, _I64, _I, _P, _P, _P, _I, _P, _I, _P, _P]),
}

_lock = threading.Lock()
_lib = None


class NativeError(RuntimeError):
    """A C-ABI call returned an error code."""


def library_path() -> str:
    return LIB_PATH


def load() -> C.CDLL:
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            import torch  # noqa: F401  -- HIP runtime first

            if not os.path.exists(LIB_PATH):
                raise NativeError(f"flashgrpo_amd native library missing at {LIB_PATH}; "
                                  "build it with `python __graft_entry__.py build` (hipcc, gfx950)")
            lib = C.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> int:
    lib = load()
    rc = getattr(lib, name)(*args)
    if SIGNATURES[name][0] is _I and rc != 0:
        msg = lib.fg_last_error().decode(errors="replace")
        if "null pointer" in msg or "bad" in msg or "must" in msg or "shape" in msg:
            raise ValueError(msg)
        raise NativeError(msg)
    return rc


def exported_symbols() -> list:
    return sorted(SIGNATURES)
