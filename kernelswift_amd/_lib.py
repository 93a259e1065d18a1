"""ctypes binding of libkswift_amd.so (the C ABI declared in include/kswift.h).

The library must have been built (python -m kernelswift_amd.build, or
__graft_entry__.build()).  There is no fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkswift_amd.so")
TORCH_LIB_PATH = os.path.join(HERE, "libkswift_torch.so")

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_p = ctypes.c_void_p
_c_f = ctypes.c_float
_c_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/kswift.h one to one
SIGNATURES = {
    "ks_last_error": (ctypes.c_char_p, []),
    "ks_version": (ctypes.c_int, []),
    "ks_sinkhorn": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i32, _c_f, _c_p]),
    "ks_rope_inplace": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _c_p]),
    "ks_indexer_scores": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_i32, _c_p]),
    "ks_indexer_row_stats": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "ks_indexer_workspace_size": (_c_sz, [_c_i64] * 5),
    "ks_indexer": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i32, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_i32,
                                  _c_i64, _c_i32, _c_i64, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                  _c_i64, _c_p, _c_sz, _c_p]),
    "ks_indexer_scaled": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i32, _c_f, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64,
                                         _c_i32, _c_i64, _c_i32, _c_i64, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_p, _c_sz, _c_p]),
    "ks_fp8_quant_rows": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_p]),
    "ks_indexer_fp8": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i32, _c_i64,
                                      _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_sz,
                                      _c_p]),
    "ks_indexer_topk": (ctypes.c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_i32, _c_i64,
                                       _c_p, _c_i32, _c_p]),
    "ks_sparse_attn_workspace_size": (_c_sz, [_c_i64] * 6),
    "ks_sparse_attn": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                      _c_i64, _c_f, _c_p, _c_sz, _c_p]),
    "ks_mhc_pre": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_p]),
    "ks_mhc_post": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_f, _c_p]),
    "ks_sparse_attn_noalloc_max_scratch": (_c_sz, []),
    "ks_sparse_attn_noalloc": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                              _c_i64, _c_i64, _c_f, _c_p]),
    "ks_copy_bytes": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_p]),
}

# diagnostic exports (not in include/kswift.h)
DEBUG_SIGNATURES = {
    "ks_dbg_indexer_scores_bounded": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                                     _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_p]),
    "ks_dbg_indexer_topk_bounded": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                                   _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_p, _c_p,
                                                   _c_p, _c_i64]),
    "ks_dbg_topk_bounded_slots": (ctypes.c_int64, [_c_i64, _c_i64]),
    "ks_dbg_sparse_attn_count": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                                _c_f, _c_p, _c_sz, _c_p]),
    "ks_dbg_indexer": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i32, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_i32,
                                      _c_i64, _c_i32, _c_i64, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                      _c_i64, _c_p, _c_sz, _c_p, _c_f, _c_p, _c_i32]),
    "ks_dbg_indexer_scores": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64,
                                             _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i64, _c_i32, _c_f, _c_p,
                                             _c_p]),
    "ks_dbg_indexer_fp8": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i64, _c_i32, _c_i64, _c_i32,
                                          _c_i64, _c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p,
                                          _c_sz, _c_p, _c_p, _c_i32]),
    "ks_dbg_mfma_bf16_chain": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_p]),
    "ks_dbg_mfma_fp8_chain": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_p]),
    "ks_dbg_mfma_fp8_plain_chain": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_p]),
    "ks_dbg_fp8_cvt": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i32, _c_p, _c_p]),
    "ks_dbg_exact_dot_wide": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_p]),
    "ks_dbg_score_bound_c": (ctypes.c_float, []),
    "ks_dbg_score_bound_c_d": (ctypes.c_float, [_c_i64]),
}

_lib = None
_lock = threading.Lock()


class KsError(RuntimeError):
    """Raised when a C-ABI call returns non-zero (argument or HIP error)."""


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise KsError(f"{LIB_PATH} is missing: build it with `python -m kernelswift_amd.build` "
                              "(there is no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in list(SIGNATURES.items()) + list(DEBUG_SIGNATURES.items()):
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


_torch_ops = None


def torch_ops():
    """torch.ops.ks_mi355x, the TORCH_LIBRARY registration of libkswift_torch.so (loaded on first use).
    Raises KsError when the library has not been built (there is no fallback)."""
    global _torch_ops
    if _torch_ops is not None:
        return _torch_ops
    with _lock:
        if _torch_ops is None:
            import torch
            if not os.path.exists(TORCH_LIB_PATH):
                raise KsError(f"{TORCH_LIB_PATH} is missing: build it with `python -m kernelswift_amd.build`")
            torch.ops.load_library(TORCH_LIB_PATH)
            _torch_ops = torch.ops.ks_mi355x
    return _torch_ops


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().ks_last_error().decode(errors="replace")
        raise KsError(f"{what}: {msg} (code {rc})")
