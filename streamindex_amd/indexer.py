"""Lightning indexer operators on MI355X (gfx950 HIP kernels via the C ABI).

Mirrors the reference's public operator surface:

* ``chunked_indexer_topk``  — ``flash_sparse/triton/chunked_indexer.py:47-160``
* ``indexer_score``         — ``flash_sparse/triton/indexer_score.py:123-179``
* ``indexer_score_topk``    — ``flash_sparse/triton/indexer_score.py:182-205``

Same argument names, meanings, output shapes/dtypes and exception types
(``AssertionError`` for device/shape checks, ``ValueError`` for unsupported
dimensions).  The implementation differs: the top-k path is one fused kernel
that keeps each query row's selection state in LDS and never writes a score
matrix, so ``chunk_s`` / ``chunk_t`` do not change the result (the
partition-merge top-k is exact for any partition) and no score workspace is
allocated at any sequence length.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

SUPPORTED_D = (32, 64, 128, 256)
MAX_HEADS = 256          # any H_I up to 256 (rows past 128 heads, 64 at D_I = 256, split over waves)
MAX_TOPK = 4096          # top_k above 2048 (1536 at D_I = 256) runs the head-split kernel
MAX_HEADS_Q = 64         # fp4 q / fp8 k indexer
MAX_TOPK_Q = 2048


def _check_common(q: torch.Tensor, k_idx: torch.Tensor, weights: torch.Tensor):
    assert q.is_cuda and k_idx.is_cuda and weights.is_cuda
    assert k_idx.device == q.device and weights.device == q.device, "q, k_idx and weights must share a device"
    assert q.dim() == 4 and k_idx.dim() == 3 and weights.dim() == 3
    B, S, H_I, D_I = q.shape
    B2, T, D_I2 = k_idx.shape
    assert B2 == B and D_I2 == D_I, f"q/k shape mismatch: q={tuple(q.shape)}, k={tuple(k_idx.shape)}"
    assert weights.shape == (B, S, H_I)
    if q.dtype != torch.bfloat16 or k_idx.dtype != torch.bfloat16:
        raise ValueError(f"q and k_idx must be bfloat16, got {q.dtype} / {k_idx.dtype}")
    if weights.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"weights must be float32 or bfloat16, got {weights.dtype}")
    if D_I not in SUPPORTED_D:
        raise ValueError(f"D_I ({D_I}) must be one of {SUPPORTED_D}")
    if H_I > MAX_HEADS:
        raise ValueError(f"H_I ({H_I}) must be <= {MAX_HEADS}")
    return B, S, H_I, D_I, T


def _prep(q, k_idx, weights):
    # The kernels take arbitrary batch/row strides but need 16-byte rows with a
    # contiguous head-dim; anything else is compacted once here.
    def ok(t, inner_dims):
        return t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0

    if not ok(q, 3):
        q = q.contiguous()
    if not ok(k_idx, 2):
        k_idx = k_idx.contiguous()
    return q, k_idx, weights


def indexer_score(q: torch.Tensor, k_idx: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
    """Lightning-indexer score matrix ``I(s,t) = Σ_h w[s,h]·relu(q[s,h]·k[t])``.

    Args:
      q: ``[B, S, H_I, D_I]`` bf16.  k_idx: ``[B, T, D_I]`` bf16.
      weights: ``[B, S, H_I]`` fp32 or bf16.
    Returns:
      ``[B, S, T]`` fp32 (no mask applied), as ``indexer_score.py:123-179``.
    """
    B, S, H_I, D_I, T = _check_common(q, k_idx, weights)
    q, k_idx, weights = _prep(q, k_idx, weights)
    scores = torch.empty((B, S, T), device=q.device, dtype=torch.float32)
    L = _lib.load()
    with torch.cuda.device(q.device):
        rc = L.si_indexer_score(
            q.data_ptr(), _lib.strides(q), k_idx.data_ptr(), _lib.strides(k_idx),
            weights.data_ptr(), 1 if weights.dtype == torch.bfloat16 else 0, _lib.strides(weights),
            B, S, T, H_I, D_I, scores.data_ptr(), _lib.strides(scores), _lib.stream_ptr(q.device))
    _lib.check(rc)
    return scores


def _topk_launch(q, k_idx, weights, top_k, causal_mask, causal_ratio):
    B, S, H_I, D_I, T = _check_common(q, k_idx, weights)
    if top_k <= 0:
        raise ValueError(f"top_k must be positive, got {top_k}")
    if top_k > MAX_TOPK:
        raise ValueError(f"top_k ({top_k}) must be <= {MAX_TOPK}")
    q, k_idx, weights = _prep(q, k_idx, weights)
    out_idx = torch.empty((B, S, top_k), dtype=torch.int64, device=q.device)
    out_scores = torch.empty((B, S, top_k), dtype=torch.float32, device=q.device)
    mask_ptr, mask_strides = None, None
    if causal_mask is not None:
        if causal_mask.dtype != torch.bool:
            causal_mask = causal_mask != 0
        assert causal_mask.is_cuda and causal_mask.device == q.device
        assert causal_mask.shape == (B, S, T), f"causal_mask must be [B,S,T]={(B, S, T)}"
        mask_ptr, mask_strides = causal_mask.data_ptr(), _lib.strides(causal_mask)
    ratio = 0 if causal_ratio is None else int(causal_ratio)
    if causal_ratio is not None and ratio <= 0:
        raise ValueError(f"causal_ratio must be a positive integer, got {causal_ratio}")
    L = _lib.load()
    with torch.cuda.device(q.device):
        rc = L.si_indexer_topk(
            q.data_ptr(), _lib.strides(q), k_idx.data_ptr(), _lib.strides(k_idx),
            weights.data_ptr(), 1 if weights.dtype == torch.bfloat16 else 0, _lib.strides(weights),
            mask_ptr, mask_strides, B, S, T, H_I, D_I, top_k, ratio,
            out_idx.data_ptr(), out_scores.data_ptr(), _lib.stream_ptr(q.device))
    _lib.check(rc)
    return out_idx, out_scores


def chunked_indexer_topk(
    q: torch.Tensor,
    k_idx: torch.Tensor,
    weights: torch.Tensor,
    top_k: int,
    *,
    causal_mask: Optional[torch.Tensor] = None,
    causal_ratio: Optional[int] = None,
    chunk_s: int = 4096,
    chunk_t: int = 4096,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Indexer + exact top-k per query row.  Returns ``(top_k_indices, top_k_scores)``.

    Args (as ``chunked_indexer.py:47-78``):
      q: ``[B, S, H_I, D_I]`` bf16.  k_idx: ``[B, T, D_I]`` bf16.
      weights: ``[B, S, H_I]`` fp32 (or bf16).
      top_k: entries selected per query (output width is always ``top_k``).
      causal_mask: optional ``[B, S, T]`` bool, True = legal.
      causal_ratio: optional int; key t is legal for query s iff
        ``t < (s + 1) // causal_ratio``.  Exclusive with ``causal_mask``.
      chunk_s, chunk_t: accepted for API compatibility.  The fused kernel
        needs no score workspace, so they bound nothing and cannot change the
        result; they must be positive as in the reference's range() loops.

    Returns:
      ``(idx [B,S,top_k] int64, scores [B,S,top_k] fp32)`` sorted best-first
      (score descending, smaller index first on ties), ``-1`` / ``-inf`` where
      a row has fewer than ``top_k`` legal keys.
    """
    assert q.is_cuda and k_idx.is_cuda and weights.is_cuda
    B, S, H_I, D_I = q.shape
    T = k_idx.shape[1]
    assert k_idx.shape == (B, T, D_I)
    assert weights.shape == (B, S, H_I)
    if causal_mask is not None:
        assert causal_mask.shape == (B, S, T)
        assert causal_ratio is None, "specify either causal_mask or causal_ratio, not both"
    if int(chunk_s) <= 0 or int(chunk_t) <= 0:
        raise ValueError(f"chunk_s and chunk_t must be positive, got {chunk_s}, {chunk_t}")
    return _topk_launch(q, k_idx, weights, top_k, causal_mask, causal_ratio)


def indexer_score_topk(
    q: torch.Tensor,
    k_idx: torch.Tensor,
    weights: torch.Tensor,
    top_k: int,
    *,
    causal_mask: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Indexer + top-k with output width ``min(top_k, T)`` (``indexer_score.py:182-205``).

    Runs the fused kernel; no ``[B,S,T]`` score matrix is materialised.  Slots
    past a row's legal-key count hold index ``-1`` and score ``-inf``.
    """
    B, S, H_I, D_I, T = _check_common(q, k_idx, weights)
    k = min(int(top_k), T)
    if k == 0:
        return (torch.empty((B, S, 0), dtype=torch.int64, device=q.device),
                torch.empty((B, S, 0), dtype=torch.float32, device=q.device))
    if causal_mask is not None:
        assert causal_mask.shape == (B, S, T)
    return _topk_launch(q, k_idx, weights, k, causal_mask, None)


__all__ = ["chunked_indexer_topk", "indexer_score", "indexer_score_topk"]


# ---------------------------------------------------------------------------
# Quantised inputs (the production V4 indexer dtypes)
# ---------------------------------------------------------------------------
def indexer_topk_q(
    q_fp4: torch.Tensor,
    q_scale: torch.Tensor,
    k_fp8: torch.Tensor,
    k_scale: torch.Tensor,
    weights: torch.Tensor,
    top_k: int,
    *,
    causal_mask: Optional[torch.Tensor] = None,
    causal_ratio: Optional[int] = None,
    check_scales: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Indexer + exact top-k over fp4 queries and fp8 keys.

    Args:
      q_fp4: ``[B, S, H_I, 64]`` uint8, e2m1 pairs (element 2i in the low
        nibble) of ``D_I = 128`` dims, as :func:`streamindex_amd.quant.fp4_act_quant`
        writes them.  q_scale: ``[B, S, H_I, 4]`` fp32, one power-of-two scale
        per 32 dims.
      k_fp8: ``[B, T, 128]`` ``torch.float8_e4m3fn``.  k_scale: ``[B, T]`` or
        ``[B, T, 1]`` fp32, one positive scale per key row
        (:func:`streamindex_amd.quant.act_quant` with ``block_size=128``).
      weights, top_k, causal_mask, causal_ratio: as :func:`chunked_indexer_topk`.
      check_scales: verify that ``q_scale`` holds powers of two (the kernel
        reads their exponent bits as UE8M0 scales).

    Returns ``(idx, scores)`` exactly as :func:`chunked_indexer_topk` does for
    the dequantised inputs ``q = value · q_scale``, ``k = value · k_scale``.
    """
    assert q_fp4.is_cuda and k_fp8.is_cuda and weights.is_cuda
    for name, t in (("q_scale", q_scale), ("k_fp8", k_fp8), ("k_scale", k_scale), ("weights", weights)):
        assert t.is_cuda and t.device == q_fp4.device, f"{name} must be a CUDA tensor on {q_fp4.device}"
    assert q_fp4.dim() == 4 and k_fp8.dim() == 3 and weights.dim() == 3
    B, S, H_I, Dh = q_fp4.shape
    B2, T, D_I = k_fp8.shape
    assert B2 == B and D_I == 2 * Dh, f"q/k shape mismatch: q={tuple(q_fp4.shape)}, k={tuple(k_fp8.shape)}"
    assert weights.shape == (B, S, H_I)
    assert q_scale.shape == (B, S, H_I, D_I // 32), f"q_scale must be [B,S,H_I,{D_I // 32}]"
    if k_scale.dim() == 3:
        assert k_scale.shape[2] == 1, "one key scale per row (act_quant block_size = D_I)"
        k_scale = k_scale[..., 0]
    assert k_scale.shape == (B, T)
    if q_fp4.dtype != torch.uint8 or k_fp8.dtype != torch.float8_e4m3fn:
        raise ValueError(f"q_fp4 must be uint8 and k_fp8 float8_e4m3fn, got {q_fp4.dtype} / {k_fp8.dtype}")
    if q_scale.dtype != torch.float32 or k_scale.dtype != torch.float32:
        raise ValueError("scales must be float32")
    if weights.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"weights must be float32 or bfloat16, got {weights.dtype}")
    if D_I != 128:
        raise ValueError(f"D_I ({D_I}) must be 128 for quantised inputs")
    if H_I > MAX_HEADS_Q:
        raise ValueError(f"H_I ({H_I}) must be <= {MAX_HEADS_Q} for quantised inputs")
    if top_k <= 0 or top_k > MAX_TOPK_Q:
        raise ValueError(f"top_k must be in [1, {MAX_TOPK_Q}], got {top_k}")
    if check_scales and q_scale.numel():
        m, _ = torch.frexp(q_scale)
        if not bool((m == 0.5).all()):
            raise ValueError("q_scale must hold powers of two (UE8M0)")
    ratio = 0 if causal_ratio is None else int(causal_ratio)
    if causal_ratio is not None and ratio <= 0:
        raise ValueError(f"causal_ratio must be a positive integer, got {causal_ratio}")

    def ok(t):
        return t.stride(-1) == 1 and all(s % 16 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0

    q_fp4 = q_fp4 if ok(q_fp4) else q_fp4.contiguous()
    k8 = k_fp8.view(torch.uint8)
    k8 = k8 if ok(k8) else k8.contiguous()
    q_scale = q_scale if q_scale.stride(-1) == 1 else q_scale.contiguous()
    out_idx = torch.empty((B, S, top_k), dtype=torch.int64, device=q_fp4.device)
    out_scores = torch.empty((B, S, top_k), dtype=torch.float32, device=q_fp4.device)
    mask_ptr, mask_strides = None, None
    if causal_mask is not None:
        # the checks chunked_indexer_topk applies (chunked_indexer.py:79-86): the
        # kernel reads the mask through its strides, so its shape and device matter
        assert causal_mask.is_cuda and causal_mask.device == q_fp4.device, "causal_mask must be on q's device"
        assert causal_mask.shape == (B, S, T), f"causal_mask must be [B,S,T]={(B, S, T)}, got {tuple(causal_mask.shape)}"
        assert causal_ratio is None, "specify either causal_mask or causal_ratio, not both"
        if causal_mask.dtype != torch.bool:
            causal_mask = causal_mask != 0
        mask_ptr, mask_strides = causal_mask.data_ptr(), _lib.strides(causal_mask)
    L = _lib.load()
    with torch.cuda.device(q_fp4.device):
        rc = L.si_indexer_topk_q(
            q_fp4.data_ptr(), _lib.strides(q_fp4), q_scale.data_ptr(), _lib.strides(q_scale),
            k8.data_ptr(), _lib.strides(k8), k_scale.data_ptr(), _lib.strides(k_scale),
            weights.data_ptr(), 1 if weights.dtype == torch.bfloat16 else 0, _lib.strides(weights),
            mask_ptr, mask_strides, B, S, T, H_I, D_I, top_k, ratio,
            out_idx.data_ptr(), out_scores.data_ptr(), _lib.stream_ptr(q_fp4.device))
    _lib.check(rc)
    return out_idx, out_scores


def chunked_indexer_topk_quantized(
    q: torch.Tensor,
    k_idx: torch.Tensor,
    weights: torch.Tensor,
    top_k: int,
    *,
    causal_mask: Optional[torch.Tensor] = None,
    causal_ratio: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``chunked_indexer_topk`` under the production V4 indexer dtypes:
    quantises bf16 ``q`` to fp4 (UE8M0 per 32 dims) and ``k_idx`` to fp8
    (one scale per row), then runs :func:`indexer_topk_q`."""
    from .quant import act_quant, fp4_act_quant

    q4, qs = fp4_act_quant(q, 32)
    k8, ks = act_quant(k_idx, k_idx.shape[-1])
    return indexer_topk_q(q4, qs, k8, ks, weights, top_k, causal_mask=causal_mask, causal_ratio=causal_ratio,
                          check_scales=False)
