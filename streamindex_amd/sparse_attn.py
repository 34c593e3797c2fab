"""Sparse attention on MI355X (gfx950 HIP kernels via the C ABI).

Mirrors ``flash_sparse/triton/sparse_attn_fwd.py:180-292`` (``sparse_attn_fwd``),
``flash_sparse/triton/sparse_attn_bwd.py:286-416`` (``sparse_attn_bwd``) and
``flash_sparse/triton/__init__.py:19-60`` (``sparse_attn`` with autograd).
Same argument names, shapes, dtypes and return values.

Differences, all deliberate:

* ``D`` may be any of 32, 64, 128, 256, 512 or 576 — including the V4 head dim
  576 that the reference kernel rejects (``sparse_attn_fwd.py:217-218``).
* ``block_h`` / ``block_n`` are accepted and ignored: the kernel gathers each
  query's KV rows once for all heads, so there is no head-block knob.
* An index ``>= N_kv`` is treated like ``-1`` (masked) instead of reading out
  of bounds.
* The backward reduces dkv deterministically (per-(query, slot) rows
  reduced key by key in a fixed order) instead of with fp32 atomics, so
  repeated calls give bit-identical gradients; each row is rounded to the
  operand type (bf16 or fp16) before the fp32 sum.  Its workspace comes from the torch caching allocator
  and long sequences are processed in chunks of query rows that fit it.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

SUPPORTED_D = (32, 64, 128, 256, 512, 576)


def _check_device(dev: torch.device, **tensors) -> None:
    """Every tensor argument the kernels dereference must live on ``dev``
    (the reference asserts ``is_cuda`` on its inputs; a host pointer handed to
    a kernel would fault instead of raising)."""
    for name, t in tensors.items():
        if t is None:
            continue
        assert t.is_cuda and t.device == dev, f"{name} must be a CUDA tensor on {dev}, got {t.device}"


def sparse_attn_fwd(
    q: torch.Tensor,
    kv: torch.Tensor,
    attn_sink: torch.Tensor,
    topk_idxs: torch.Tensor,
    softmax_scale: Optional[float] = None,
    *,
    block_h: Optional[int] = None,
    block_n: int = 64,
    row_len: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """MQA sparse attention with attention sink.

    Args:
      q: ``[B, S, H, D]`` bf16 or fp16.  kv: ``[B, N_kv, D]`` of q's type (one shared head).
      attn_sink: ``[H]`` fp32.  topk_idxs: ``[B, S, K]`` int32/int64, ``-1`` = masked.
      softmax_scale: defaults to ``D ** -0.5``.
      row_len: optional ``[B, S]`` int32 (an extension, not in the reference):
        columns ``j >= row_len[b, s]`` are masked and their 32-key tiles are
        never gathered or computed.  For rows whose tail is already ``-1``
        (HCA, short CSA rows) the result is unchanged and the tail costs nothing.
    Returns:
      ``(o [B,S,H,D] in q's type, lse [B,S,H] fp32)``.  A row with no valid index
      gets ``o = 0`` and ``lse = sink`` (or ``-1e30`` if the sink is ``-inf``).
    """
    del block_h, block_n
    assert q.is_cuda and kv.is_cuda
    _check_device(q.device, kv=kv, attn_sink=attn_sink, topk_idxs=topk_idxs, row_len=row_len)
    assert q.dim() == 4 and kv.dim() == 3
    assert q.dtype in (torch.bfloat16, torch.float16), f"Q must be bf16 or fp16, got {q.dtype}"
    assert kv.dtype == q.dtype
    assert attn_sink.dtype == torch.float32
    B, S, H, D = q.shape
    B2, N_kv, D2 = kv.shape
    assert B2 == B and D2 == D, "q and kv shape mismatch"
    assert attn_sink.shape == (H,)
    assert topk_idxs.shape[:2] == (B, S)
    assert topk_idxs.dim() == 3
    if D not in SUPPORTED_D:
        raise ValueError(f"D ({D}) must be one of {SUPPORTED_D}")
    if topk_idxs.dtype not in (torch.int32, torch.int64):
        topk_idxs = topk_idxs.to(torch.int64)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    K = topk_idxs.shape[-1]

    def ok(t):
        return t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0

    if not ok(q):
        q = q.contiguous()
    if not ok(kv):
        kv = kv.contiguous()
    attn_sink = attn_sink.contiguous()
    if row_len is not None:
        assert row_len.is_cuda and row_len.shape == (B, S), "row_len must be [B, S] on the GPU"
        if row_len.dtype != torch.int32:
            row_len = row_len.to(torch.int32)
    o = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=q.device)
    L = _lib.load()
    with torch.cuda.device(q.device):
        rc = L.si_sparse_attn_fwd_ragged(
            q.data_ptr(), _lib.strides(q), kv.data_ptr(), _lib.strides(kv), attn_sink.data_ptr(),
            topk_idxs.data_ptr(), 1 if topk_idxs.dtype == torch.int64 else 0, _lib.strides(topk_idxs),
            B, S, H, D, N_kv, K, float(softmax_scale), _lib.qkv_dtype(q), o.data_ptr(), _lib.strides(o),
            lse.data_ptr(), _lib.strides(lse), None if row_len is None else row_len.data_ptr(),
            None if row_len is None else _lib.strides(row_len), _lib.stream_ptr(q.device))
    _lib.check(rc)
    return o, lse


def sparse_attn_fwd_kv2(
    q: torch.Tensor,
    kv: torch.Tensor,
    kv2: torch.Tensor,
    attn_sink: torch.Tensor,
    topk_idxs: torch.Tensor,
    softmax_scale: Optional[float] = None,
    *,
    row_len: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """:func:`sparse_attn_fwd` over the rows of ``[kv ; kv2]`` (concatenated
    along N) without building that tensor: index ``j < N1`` reads ``kv[:, j]``,
    ``N1 <= j < N1 + N2`` reads ``kv2[:, j - N1]``.  The CSA / HCA layout
    (``flash_sparse/csa.py:197-205``, ``hca.py:85-95``: window columns into
    the uncompressed KV, picks ``+ S`` into the compressed KV).  An extension
    with no reference counterpart; ``topk_idxs`` is int32 (the compositions'
    rows), other integer types are converted.  Same outputs as
    ``sparse_attn_fwd(q, torch.cat([kv, kv2], 1), ...)``.
    """
    assert q.is_cuda and kv.is_cuda and kv2.is_cuda
    _check_device(q.device, kv=kv, kv2=kv2, attn_sink=attn_sink, topk_idxs=topk_idxs, row_len=row_len)
    assert q.dim() == 4 and kv.dim() == 3 and kv2.dim() == 3
    assert q.dtype in (torch.bfloat16, torch.float16), f"Q must be bf16 or fp16, got {q.dtype}"
    assert kv.dtype == q.dtype and kv2.dtype == q.dtype
    assert attn_sink.dtype == torch.float32
    B, S, H, D = q.shape
    N1, N2 = kv.shape[1], kv2.shape[1]
    assert kv.shape == (B, N1, D) and kv2.shape == (B, N2, D), "q, kv and kv2 shape mismatch"
    assert attn_sink.shape == (H,)
    assert topk_idxs.dim() == 3 and topk_idxs.shape[:2] == (B, S)
    if D not in SUPPORTED_D:
        raise ValueError(f"D ({D}) must be one of {SUPPORTED_D}")
    if topk_idxs.dtype != torch.int32:
        topk_idxs = topk_idxs.to(torch.int32)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    K = topk_idxs.shape[-1]
    q, kv, kv2 = (t if _aligned(t) else t.contiguous() for t in (q, kv, kv2))
    attn_sink = attn_sink.contiguous()
    if row_len is not None:
        assert row_len.is_cuda and row_len.shape == (B, S), "row_len must be [B, S] on the GPU"
        if row_len.dtype != torch.int32:
            row_len = row_len.to(torch.int32)
    o = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=q.device)
    L = _lib.load()
    with torch.cuda.device(q.device):
        rc = L.si_sparse_attn_fwd_kv2(
            q.data_ptr(), _lib.strides(q), kv.data_ptr(), _lib.strides(kv), N1, kv2.data_ptr(), _lib.strides(kv2),
            N2, attn_sink.data_ptr(), topk_idxs.data_ptr(), _lib.strides(topk_idxs), B, S, H, D, K,
            float(softmax_scale), _lib.qkv_dtype(q), o.data_ptr(), _lib.strides(o), lse.data_ptr(),
            _lib.strides(lse), None if row_len is None else row_len.data_ptr(),
            None if row_len is None else _lib.strides(row_len), _lib.stream_ptr(q.device))
    _lib.check(rc)
    return o, lse


# Default cap on the backward's workspace: at most this, and at most a quarter
# of the device memory free at the call (the driver's free memory plus what
# the caching allocator holds unused).  At S = 64K, 64 heads, D = 576, K = 512
# a 2 GiB workspace runs the query rows in 27 chunks (one key sort for all of
# them) within 7 % of the time an 8 GiB one takes in 6.
BWD_WORKSPACE_CAP = 2 << 30


def _aligned(t: torch.Tensor) -> bool:
    return t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0


def sparse_attn_bwd(
    q: torch.Tensor,
    kv: torch.Tensor,
    attn_sink: torch.Tensor,
    topk_idxs: torch.Tensor,
    o: torch.Tensor,
    lse: torch.Tensor,
    do: torch.Tensor,
    softmax_scale: Optional[float] = None,
    *,
    block_h: Optional[int] = None,
    workspace_bytes: Optional[int] = None,
    row_len: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward of :func:`sparse_attn_fwd` from its saved ``o`` and ``lse``.

    Returns ``(dq, dkv, dattn_sink)`` shaped and typed like ``q``, ``kv`` and
    ``attn_sink``.  ``workspace_bytes`` caps the scratch memory (default:
    ``BWD_WORKSPACE_CAP`` or a quarter of the free device memory, cached
    blocks included, whichever is smaller); the query rows are processed in as
    few chunks as fit it.
    ``row_len`` as in :func:`sparse_attn_fwd` (an extension): columns at or
    past it are masked and their tiles skipped.
    """
    del block_h
    assert q.is_cuda and kv.is_cuda and do.is_cuda
    _check_device(q.device, kv=kv, attn_sink=attn_sink, topk_idxs=topk_idxs, o=o, lse=lse, do=do, row_len=row_len)
    assert q.shape == do.shape, "do must match q shape"
    assert q.dtype == kv.dtype == do.dtype
    assert attn_sink.dtype == torch.float32
    assert lse.dtype == torch.float32
    assert q.dim() == 4 and kv.dim() == 3 and topk_idxs.dim() == 3
    B, S, H, D = q.shape
    B2, N_kv, D2 = kv.shape
    assert B2 == B and D2 == D, "q and kv shape mismatch"
    assert o.shape == q.shape and o.dtype == q.dtype
    assert lse.shape == (B, S, H) and attn_sink.shape == (H,)
    assert topk_idxs.shape[:2] == (B, S)
    assert q.dtype in (torch.bfloat16, torch.float16), f"Q must be bf16 or fp16, got {q.dtype}"
    if D not in SUPPORTED_D:
        raise ValueError(f"D ({D}) must be one of {SUPPORTED_D}")
    if topk_idxs.dtype not in (torch.int32, torch.int64):
        topk_idxs = topk_idxs.to(torch.int64)
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    K = topk_idxs.shape[-1]
    if row_len is not None:
        assert row_len.is_cuda and row_len.shape == (B, S), "row_len must be [B, S] on the GPU"
        if row_len.dtype != torch.int32:
            row_len = row_len.to(torch.int32)
    q, kv, o, do = (t if _aligned(t) else t.contiguous() for t in (q, kv, o, do))
    attn_sink = attn_sink.contiguous()
    dq = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device)
    dkv = torch.empty((B, N_kv, D), dtype=kv.dtype, device=q.device)
    dsink = torch.empty((H,), dtype=torch.float32, device=q.device)
    L = _lib.load()
    with torch.cuda.device(q.device):
        default_cap = workspace_bytes is None
        if workspace_bytes is None:
            # Memory the caching allocator holds but has not handed out counts
            # as free too: the driver's free figure alone moves with every
            # segment the allocator maps, and with it the workspace size,
            # which then misses the cached block and allocates anew.
            free, _ = torch.cuda.mem_get_info(q.device)
            cached = torch.cuda.memory_reserved(q.device) - torch.cuda.memory_allocated(q.device)
            workspace_bytes = min(BWD_WORKSPACE_CAP, (free + cached) // 4)
        need = L.si_sparse_attn_bwd_workspace_bytes(B, S, H, D, N_kv, K, int(workspace_bytes))
        if need < 0:
            raise ValueError(L.si_last_error().decode("utf-8", "replace"))
        try:
            ws = torch.empty((max(int(need), 16),), dtype=torch.uint8, device=q.device)
        except torch.OutOfMemoryError:
            if not default_cap:
                raise
            # The allocator's unused blocks may be split too finely to hold the
            # workspace: size it from the driver's free memory alone.
            free, _ = torch.cuda.mem_get_info(q.device)
            need = L.si_sparse_attn_bwd_workspace_bytes(B, S, H, D, N_kv, K, int(min(BWD_WORKSPACE_CAP, free // 4)))
            if need < 0:
                raise ValueError(L.si_last_error().decode("utf-8", "replace"))
            ws = torch.empty((max(int(need), 16),), dtype=torch.uint8, device=q.device)
        rc = L.si_sparse_attn_bwd_ragged(
            q.data_ptr(), _lib.strides(q), kv.data_ptr(), _lib.strides(kv), attn_sink.data_ptr(),
            topk_idxs.data_ptr(), 1 if topk_idxs.dtype == torch.int64 else 0, _lib.strides(topk_idxs),
            o.data_ptr(), _lib.strides(o), lse.data_ptr(), _lib.strides(lse), do.data_ptr(), _lib.strides(do),
            B, S, H, D, N_kv, K, float(softmax_scale), _lib.qkv_dtype(q), dq.data_ptr(), _lib.strides(dq),
            dkv.data_ptr(), _lib.strides(dkv), dsink.data_ptr(), ws.data_ptr(), ws.numel(),
            None if row_len is None else row_len.data_ptr(), None if row_len is None else _lib.strides(row_len),
            _lib.stream_ptr(q.device))
    _lib.check(rc)
    return dq, dkv, dsink


def sparse_attn_bwd_v2(q, kv, attn_sink, topk_idxs, o, lse, do, softmax_scale: Optional[float] = None, *,
                       block_h: Optional[int] = None, block_n: int = 64, block_q: int = 8,
                       k_max: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The reference's atomic-free backward variant (``sparse_attn_bwd_v2.py:381-416``).

    :func:`sparse_attn_bwd` already reduces dkv key by key without atomics (the
    idea v2 prototypes), so this is the same computation; the tiling knobs are
    accepted and ignored, and there is no ``k_max`` bound on the queries per key.
    """
    del block_h, block_n, block_q, k_max
    return sparse_attn_bwd(q, kv, attn_sink, topk_idxs, o, lse, do, softmax_scale)


def build_inverted_topk(topk_idxs: torch.Tensor, n_kv: int, k_max: int, *, block_k: int = 64
                        ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Inverted top-k index (``flash_sparse/triton/inverted_topk.py:75-128``).

    Returns ``(inv_topk [B, n_kv, k_max] int32, inv_count [B, n_kv] int32)``:
    ``inv_count[b, t]`` is the number of (query, slot) entries selecting key
    ``t`` (not clamped to ``k_max``), and the first ``min(count, k_max)``
    entries of ``inv_topk[b, t]`` are their query indices in ascending
    (query, slot) order (the reference leaves the order to its atomics); the
    rest are ``-1``.  Indices outside ``[0, n_kv)`` are ignored.
    """
    del block_k
    assert topk_idxs.is_cuda and topk_idxs.dim() == 3
    assert int(n_kv) >= 0 and int(k_max) >= 0, "n_kv and k_max must be non-negative"
    B, S, K = topk_idxs.shape
    if topk_idxs.dtype not in (torch.int32, torch.int64):
        topk_idxs = topk_idxs.to(torch.int64)
    inv_topk = torch.empty((B, n_kv, k_max), dtype=torch.int32, device=topk_idxs.device)
    inv_count = torch.empty((B, n_kv), dtype=torch.int32, device=topk_idxs.device)
    L = _lib.load()
    with torch.cuda.device(topk_idxs.device):
        need = L.si_build_inverted_topk_workspace_bytes(B, S, K, n_kv)
        if need < 0:
            raise ValueError(L.si_last_error().decode("utf-8", "replace"))
        ws = torch.empty((max(int(need), 16),), dtype=torch.uint8, device=topk_idxs.device)
        rc = L.si_build_inverted_topk(topk_idxs.data_ptr(), 1 if topk_idxs.dtype == torch.int64 else 0,
                                      _lib.strides(topk_idxs), B, S, K, n_kv, k_max, inv_topk.data_ptr(),
                                      inv_count.data_ptr(), ws.data_ptr(), ws.numel(),
                                      _lib.stream_ptr(topk_idxs.device))
    _lib.check(rc)
    return inv_topk, inv_count


class _SparseAttnFunc(torch.autograd.Function):
    """``flash_sparse/triton/__init__.py:19-44``: saves q, kv, attn_sink,
    topk_idxs, o and lse for the backward."""

    @staticmethod
    def forward(ctx, q, kv, attn_sink, topk_idxs, softmax_scale, row_len):
        o, lse = sparse_attn_fwd(q, kv, attn_sink, topk_idxs, softmax_scale, row_len=row_len)
        ctx.save_for_backward(q, kv, attn_sink, topk_idxs, o, lse, row_len)
        ctx.softmax_scale = softmax_scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, kv, attn_sink, topk_idxs, o, lse, row_len = ctx.saved_tensors
        dq, dkv, dsink = sparse_attn_bwd(q, kv, attn_sink, topk_idxs, o, lse, do.contiguous(), ctx.softmax_scale,
                                         row_len=row_len)
        return dq, dkv, dsink, None, None, None


class _SparseAttnKV2Func(torch.autograd.Function):
    """Autograd over two KV tensors: the forward reads both in place; the
    backward (which reads every selected row several times over anyway)
    runs on their concatenation and splits dkv."""

    @staticmethod
    def forward(ctx, q, kv, kv2, attn_sink, topk_idxs, softmax_scale, row_len):
        o, lse = sparse_attn_fwd_kv2(q, kv, kv2, attn_sink, topk_idxs, softmax_scale, row_len=row_len)
        ctx.save_for_backward(q, kv, kv2, attn_sink, topk_idxs, o, lse, row_len)
        ctx.softmax_scale = softmax_scale
        return o

    @staticmethod
    def backward(ctx, do):
        q, kv, kv2, attn_sink, topk_idxs, o, lse, row_len = ctx.saved_tensors
        n1 = kv.shape[1]
        dq, dkv, dsink = sparse_attn_bwd(q, torch.cat([kv, kv2], dim=1), attn_sink, topk_idxs, o, lse,
                                         do.contiguous(), ctx.softmax_scale, row_len=row_len)
        return dq, dkv[:, :n1], dkv[:, n1:], dsink, None, None, None


def sparse_attn_kv2(q, kv, kv2, attn_sink, topk_idxs, softmax_scale: Optional[float] = None, *,
                    row_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Differentiable :func:`sparse_attn_fwd_kv2` returning ``o`` (an extension used by the
    CSA / HCA compositions)."""
    return _SparseAttnKV2Func.apply(q, kv, kv2, attn_sink, topk_idxs, softmax_scale, row_len)


def sparse_attn(q, kv, attn_sink, topk_idxs, softmax_scale: Optional[float] = None, *,
                row_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Differentiable sparse attention returning ``o`` only (``flash_sparse/triton/__init__.py:48-60``).
    ``row_len`` as in :func:`sparse_attn_fwd` (an extension)."""
    return _SparseAttnFunc.apply(q, kv, attn_sink, topk_idxs, softmax_scale, row_len)


__all__ = ["sparse_attn_fwd", "sparse_attn_bwd", "sparse_attn_bwd_v2", "sparse_attn", "build_inverted_topk",
           "sparse_attn_fwd_kv2", "sparse_attn_kv2"]
