"""Token compressor and softmax-gated pooling on MI355X (gfx950 HIP kernels).

Mirrors ``flash_sparse/reference.py:176-272`` (``reference_token_compressor``:
eq. 11-12 for CSA with two overlapping streams, eq. 22-23 for HCA) and
``flash_sparse/utils/compression.py:13-24`` (``softmax_gated_pool``).  The
kernels compute in fp32 and round the result to the input dtype once (the
reference's torch ops round after each step in bf16).  The mounted reference
builds the overlap path only inside its bias-shape error branch (its body is
indented one level too deep, ``flash_sparse/reference.py:230-270``); the
function-level behaviour its docstring states is implemented.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .quant import _dtype_code


def token_compressor(
    c_a: torch.Tensor,
    z_a: torch.Tensor,
    b_a: torch.Tensor,
    m: int,
    *,
    c_b: Optional[torch.Tensor] = None,
    z_b: Optional[torch.Tensor] = None,
    b_b: Optional[torch.Tensor] = None,
    overlap: bool,
) -> torch.Tensor:
    """Compress ``m`` consecutive tokens into one entry by softmax-gated pooling.

    ``c_a, z_a [B, S, c]``; ``b_a [m, c]``; with ``overlap=True`` also
    ``c_b, z_b [B, S, c]`` and ``b_b [m, c]`` (block i's b half is block i-1 of
    the b stream; block 0's is empty).  Returns ``[B, S // m, c]``.
    """
    if c_a.dim() != 3:
        raise ValueError("c_a must be [B, S, c]")
    B, S, c = c_a.shape
    if z_a.shape != c_a.shape:
        raise ValueError("z_a must match c_a shape")
    n_blocks = S // m
    if n_blocks == 0:
        return c_a.new_zeros(B, 0, c)
    if not overlap:
        if tuple(b_a.shape) != (m, c):
            raise ValueError(f"b_a must be [m={m}, c={c}] when overlap=False, got {tuple(b_a.shape)}")
    else:
        if c_b is None or z_b is None or b_b is None:
            raise ValueError("overlap=True requires c_b, z_b, b_b")
        if tuple(b_a.shape) != (m, c) or tuple(b_b.shape) != (m, c):
            raise ValueError(f"with overlap=True, b_a and b_b must each be [m={m}, c={c}], "
                             f"got b_a={tuple(b_a.shape)}, b_b={tuple(b_b.shape)}")
        if c_b.shape != c_a.shape or z_b.shape != c_a.shape:
            raise ValueError("c_b and z_b must match c_a shape")
    assert c_a.is_cuda, "inputs must be on the GPU"
    dt = _dtype_code(c_a)
    for t in (z_a, c_b, z_b):
        if t is not None and t.dtype != c_a.dtype:
            raise ValueError("c and z streams must share one dtype")
    ca, za = c_a.contiguous(), z_a.contiguous()
    cb = c_b.contiguous() if overlap else None
    zb = z_b.contiguous() if overlap else None
    ba = b_a.to(torch.float32).contiguous()
    bb = b_b.to(torch.float32).contiguous() if overlap else None
    out = torch.empty((B, n_blocks, c), dtype=c_a.dtype, device=c_a.device)
    L = _lib.load()
    with torch.cuda.device(c_a.device):
        rc = L.si_token_compress(ca.data_ptr(), za.data_ptr(), ba.data_ptr(),
                                 None if cb is None else cb.data_ptr(), None if zb is None else zb.data_ptr(),
                                 None if bb is None else bb.data_ptr(), dt, B, S, c, m, int(overlap),
                                 out.data_ptr(), _lib.stream_ptr(c_a.device))
    _lib.check(rc)
    return out


def softmax_gated_pool(kv: torch.Tensor, score: torch.Tensor, *, dim: int = -2) -> torch.Tensor:
    """``(kv * score.softmax(dim)).sum(dim)`` (``compression.py:13-24``)."""
    assert kv.is_cuda, "inputs must be on the GPU"
    if kv.shape != score.shape or kv.dtype != score.dtype:
        raise ValueError("kv and score must share shape and dtype")
    dt = _dtype_code(kv)
    d = dim % kv.dim()
    outer = 1
    for s in kv.shape[:d]:
        outer *= s
    inner = 1
    for s in kv.shape[d + 1:]:
        inner *= s
    Lk = kv.shape[d]
    out = torch.empty(kv.shape[:d] + kv.shape[d + 1:], dtype=kv.dtype, device=kv.device)
    if Lk == 0:
        return out.zero_()
    kc, sc = kv.contiguous(), score.contiguous()
    L = _lib.load()
    with torch.cuda.device(kv.device):
        rc = L.si_gated_pool(kc.data_ptr(), sc.data_ptr(), out.data_ptr(), dt, outer, Lk, inner,
                             _lib.stream_ptr(kv.device))
    _lib.check(rc)
    return out


__all__ = ["token_compressor", "softmax_gated_pool"]
