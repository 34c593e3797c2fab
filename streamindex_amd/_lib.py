"""ctypes binding of ``libstreamindex.so`` (the C ABI declared in
``include/streamindex.h``).

There is exactly one implementation of every operator: the HIP kernels in this
library.  If the library has not been built, every operator raises; nothing
falls back to a CPU or torch implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

from .build import LIB_PATH

SI_OK = 0
SI_ERR_INVALID = 1
SI_ERR_UNSUPPORTED = 2
SI_ERR_LAUNCH = 3

_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_I64P = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must match include/streamindex.h
SIGNATURES = {
    "si_abi_version": (_I32, []),
    "si_last_error": (ctypes.c_char_p, []),
    "si_indexer_topk_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "si_indexer_set_topk_kernel": (_I32, [_I32]),
    "si_indexer_topk_plan": (_I32, [_I64, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "si_indexer_topk": (_I32, [_P, _I64P, _P, _I64P, _P, _I32, _I64P, _P, _I64P,
                               _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "si_indexer_score": (_I32, [_P, _I64P, _P, _I64P, _P, _I32, _I64P,
                                _I64, _I64, _I64, _I64, _I64, _P, _I64P, _P]),
    "si_csa_indexer_topk": (_I32, [_P, _I64P, _P, _I64P, _P, _I32, _I64P, _I64, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _P, _I64P, _P, _P]),
    "si_csa_scores_topk": (_I32, [_P, _I64P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64P, _P]),
    "si_hca_topk_idxs": (_I32, [_I64, _I64, _I64, _I64, _I64, _I64, _P, _I64P, _P]),
    "si_sparse_attn_fwd": (_I32, [_P, _I64P, _P, _I64P, _P, _P, _I32, _I64P,
                                  _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I32,
                                  _P, _I64P, _P, _I64P, _P]),
    "si_sparse_attn_fwd_ragged": (_I32, [_P, _I64P, _P, _I64P, _P, _P, _I32, _I64P,
                                         _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I32,
                                         _P, _I64P, _P, _I64P, _P, _I64P, _P]),
    "si_sparse_attn_fwd_kv2": (_I32, [_P, _I64P, _P, _I64P, _I64, _P, _I64P, _I64, _P, _P, _I64P,
                                      _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I32,
                                      _P, _I64P, _P, _I64P, _P, _I64P, _P]),
    "si_indexer_topk_q": (_I32, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I32, _I64P, _P, _I64P,
                                 _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "si_csa_indexer_topk_q": (_I32, [_P, _I64P, _P, _I64P, _P, _I64P, _P, _I64P, _P, _I32, _I64P,
                                     _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64P, _P, _P]),
    "si_build_inverted_topk_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "si_build_inverted_topk": (_I32, [_P, _I32, _I64P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P]),
    "si_quant_simulate": (_I32, [_P, _P, _I32, _I64, _I64, _I32, _P]),
    "si_quant_pack": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I32, _I32, _P]),
    "si_token_compress": (_I32, [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _I32, _P, _P]),
    "si_gated_pool": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _P]),
    "si_sparse_attn_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64, _I64]),
    "si_sparse_attn_bwd": (_I32, [_P, _I64P, _P, _I64P, _P, _P, _I32, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                  _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I32,
                                  _P, _I64P, _P, _I64P, _P, _P, _I64, _P]),
    "si_sparse_attn_bwd_ragged": (_I32, [_P, _I64P, _P, _I64P, _P, _P, _I32, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                         _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I32,
                                         _P, _I64P, _P, _I64P, _P, _P, _I64, _P, _I64P, _P]),
    "si_fill_normal": (_I32, [_P, _I32, _I64, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float, _P]),
    "si_sparse_attn_bwd_noalloc_scratch_bytes": (_I64, []),
    "si_sparse_attn_bwd_noalloc": (_I32, [_P, _I64P, _P, _I64P, _P, _P, _I32, _I64P, _P, _I64P, _P, _I64P, _P, _I64P,
                                          _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I32,
                                          _P, _I64P, _P, _I64P, _P, _P, _I64P, _P]),
}


class ExtensionNotBuilt(RuntimeError):
    pass


def lib_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Loads the HIP library once; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ExtensionNotBuilt(
                    f"StreamIndex HIP library not found at {LIB_PATH}; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def strides(t: torch.Tensor):
    arr = (ctypes.c_int64 * t.dim())(*t.stride())
    return arr


def int64s(*vals):
    return (ctypes.c_int64 * len(vals))(*vals)


SI_DTYPE_BF16 = 0
SI_DTYPE_F16 = 1


def qkv_dtype(t: torch.Tensor) -> int:
    """C-ABI element-type code of a sparse-attention operand (bf16 or fp16)."""
    if t.dtype == torch.bfloat16:
        return SI_DTYPE_BF16
    if t.dtype == torch.float16:
        return SI_DTYPE_F16
    raise ValueError(f"sparse attention operands must be bfloat16 or float16, got {t.dtype}")


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def check(rc: int) -> None:
    """Maps a C-ABI status to the exception types the reference raises."""
    if rc == SI_OK:
        return
    msg = load().si_last_error().decode("utf-8", "replace")
    if rc in (SI_ERR_INVALID, SI_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)
