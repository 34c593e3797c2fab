"""Compressed Sparse Attention (CSA) forward on MI355X.

Mirrors the reference's public CSA surface:

* ``build_csa_topk_idxs``  — ``flash_sparse/csa.py:30-83``
* ``flash_csa_forward``    — ``flash_sparse/csa.py:86-207``

A CSA query at position ``s`` attends to a sliding window of the uncompressed
KV (positions ``s-n_win+1 .. s``) and to the ``top_k`` compressed KV entries
the lightning indexer ranks highest among the causally legal ones
(``m·(i+1) - 1 <= s``, i.e. ``i < (s+1)//m``).  The attention index row is
``[window | compressed + S]`` in int32 with ``-1`` for masked slots, over
``kv_full = [kv ; kv_compressed]``.

MI355X design: the fused indexer kernel writes those int32 rows straight from
its per-row selection (window columns included), so neither a ``[B,S,T]``
score matrix, nor int64 indices, nor the torch mask/where/cat passes of the
reference exist; the sparse-attention kernel then consumes the rows as they
are.  ``build_csa_topk_idxs`` (for callers that already hold a score matrix)
runs one selection kernel over that matrix.

Deliberate differences (documented for drop-in users):

* ``use_triton``, ``use_chunked_indexer``, ``chunk_s``, ``chunk_t`` and
  ``auto_chunk_threshold_bytes`` are accepted and validated but select
  nothing: there is one implementation (the HIP kernels), its selection is
  exact for any partition, and it never materialises the score matrix, so
  every setting yields the same indices.
* Ties among equal scores rank the smaller compressed index first
  (``torch.topk`` leaves tie order unspecified).
* The attention reads ``kv`` and ``kv_compressed`` in place (two base
  pointers, :func:`streamindex_amd.sparse_attn.sparse_attn_fwd_kv2`) instead
  of the reference's ``torch.cat`` of the two (``csa.py:197-205``).
* Gradients flow through the sparse-attention autograd (the HIP backward) into
  ``q``, ``kv`` / ``kv_compressed`` and ``attn_sink``; the index rows carry none.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .indexer import _check_common, _prep, MAX_HEADS_Q, MAX_TOPK, MAX_TOPK_Q
from .sparse_attn import sparse_attn_kv2

__all__ = ["flash_csa_forward", "build_csa_topk_idxs", "csa_topk_idxs", "build_sliding_window_idxs", "csa_row_len"]


def build_sliding_window_idxs(B: int, S: int, n_win: int, device) -> torch.Tensor:
    """Sliding-window index rows ``[B, S, n_win]`` int64 (``flash_sparse/reference.py:460-475``).

    Column ``j`` of query ``s`` holds ``s - n_win + 1 + j``, or ``-1`` where that is negative.
    Built by the HIP index kernel (the HCA builder with no compressed columns).
    """
    out = torch.empty((B, S, n_win), dtype=torch.int32, device=device)
    _launch_hca(out, B, S, n_win, 0, 1, 0)
    return out.long()


def _launch_hca(out: torch.Tensor, B: int, S: int, n_win: int, n_comp: int, m_prime: int, offset: int) -> None:
    assert out.is_cuda and out.dtype == torch.int32 and out.stride(-1) == 1
    L = _lib.load()
    with torch.cuda.device(out.device):
        rc = L.si_hca_topk_idxs(B, S, n_win, n_comp, m_prime, offset, out.data_ptr(), _lib.strides(out),
                                _lib.stream_ptr(out.device))
    _lib.check(rc)


def csa_topk_idxs(q_idx: torch.Tensor, k_idx_compressed: torch.Tensor, indexer_weights: torch.Tensor, *,
                  n_win: int, top_k: int, m: int = 4, seq_len: Optional[int] = None,
                  return_scores: bool = False, quantized: bool = False):
    """Fused indexer + CSA index rows: ``[B, S, n_win + top_k]`` int32.

    One kernel scores every legal compressed key (``i < (s+1)//m``), keeps the
    exact top-``top_k`` per query and writes the attention index row:
    window columns first, then the picks plus ``seq_len`` (default ``S``),
    ``-1`` past the legal count.  With ``return_scores`` the picks' fp32
    scores ``[B, S, top_k]`` (``-inf`` padded) are returned too.  With
    ``quantized`` the indexer runs under the production V4 dtypes: ``q_idx``
    is quantised to fp4 (UE8M0 scale per 32 dims) and the keys to fp8 (one
    scale per row) and scored by the fp4 x fp8 kernel (``indexer_topk_q``).
    """
    B, S, H_I, D_I, T = _check_common(q_idx, k_idx_compressed, indexer_weights)
    if top_k <= 0 or top_k > MAX_TOPK:
        raise ValueError(f"top_k must be in [1, {MAX_TOPK}], got {top_k}")
    if n_win < 0:
        raise ValueError(f"n_win must be non-negative, got {n_win}")
    if m <= 0:
        raise ValueError(f"m must be a positive integer, got {m}")
    offset = S if seq_len is None else int(seq_len)
    q_idx, k_idx_compressed, indexer_weights = _prep(q_idx, k_idx_compressed, indexer_weights)
    out = torch.empty((B, S, n_win + top_k), dtype=torch.int32, device=q_idx.device)
    scores = torch.empty((B, S, top_k), dtype=torch.float32, device=q_idx.device) if return_scores else None
    L = _lib.load()
    if quantized:
        if D_I != 128 or H_I > MAX_HEADS_Q or top_k > MAX_TOPK_Q:
            raise ValueError(f"the quantised indexer needs D_I = 128, H_I <= {MAX_HEADS_Q} and top_k <= {MAX_TOPK_Q}")
        from .quant import act_quant, fp4_act_quant

        q4, qs = fp4_act_quant(q_idx, 32)
        k8, ks = act_quant(k_idx_compressed, D_I)
        k8u = k8.view(torch.uint8)
        ks = ks[..., 0].contiguous()
        with torch.cuda.device(q_idx.device):
            rc = L.si_csa_indexer_topk_q(
                q4.data_ptr(), _lib.strides(q4), qs.data_ptr(), _lib.strides(qs), k8u.data_ptr(), _lib.strides(k8u),
                ks.data_ptr(), _lib.strides(ks), indexer_weights.data_ptr(),
                1 if indexer_weights.dtype == torch.bfloat16 else 0, _lib.strides(indexer_weights),
                B, S, T, H_I, D_I, top_k, int(m), int(n_win), offset, out.data_ptr(), _lib.strides(out),
                scores.data_ptr() if scores is not None else None, _lib.stream_ptr(q_idx.device))
        _lib.check(rc)
        return (out, scores) if return_scores else out
    with torch.cuda.device(q_idx.device):
        rc = L.si_csa_indexer_topk(
            q_idx.data_ptr(), _lib.strides(q_idx), k_idx_compressed.data_ptr(), _lib.strides(k_idx_compressed),
            indexer_weights.data_ptr(), 1 if indexer_weights.dtype == torch.bfloat16 else 0,
            _lib.strides(indexer_weights), B, S, T, H_I, D_I, top_k, int(m), int(n_win), offset,
            out.data_ptr(), _lib.strides(out), scores.data_ptr() if scores is not None else None,
            _lib.stream_ptr(q_idx.device))
    _lib.check(rc)
    return (out, scores) if return_scores else out


def build_csa_topk_idxs(indexer_scores: torch.Tensor, n_win: int, top_k: int, *, seq_len: int,
                        n_compressed: int, m: int, device: torch.device) -> torch.Tensor:
    """CSA attention index rows from a materialised score matrix (``csa.py:30-83``).

    Args:
      indexer_scores: ``[B, S, n_compressed]`` fp32 raw indexer scores.
      n_win: sliding-window size.  top_k: compressed entries per query.
      seq_len: S (the compressed-region offset).  n_compressed: T.
      m: compression ratio (compressed entry i is legal for query s iff ``m·(i+1)-1 <= s``).
      device: output device (must be the scores' device).
    Returns:
      ``[B, S, n_win + top_k]`` int32: window indices, then the top-k legal
      compressed indices ``+ seq_len`` sorted by score, ``-1`` where a row has
      fewer than ``top_k`` legal (finite) entries.
    """
    B, S, T = indexer_scores.shape
    assert T == n_compressed
    assert S == seq_len
    assert indexer_scores.is_cuda
    if indexer_scores.dtype != torch.float32:
        indexer_scores = indexer_scores.float()
    if top_k <= 0 or top_k > MAX_TOPK:
        raise ValueError(f"top_k must be in [1, {MAX_TOPK}], got {top_k}")
    if n_win < 0 or m <= 0:
        raise ValueError(f"n_win must be >= 0 and m > 0, got {n_win}, {m}")
    out = torch.empty((B, S, n_win + top_k), dtype=torch.int32, device=indexer_scores.device)
    L = _lib.load()
    with torch.cuda.device(indexer_scores.device):
        rc = L.si_csa_scores_topk(indexer_scores.data_ptr(), _lib.strides(indexer_scores), B, S, T, top_k,
                                  int(m), int(n_win), int(seq_len), out.data_ptr(), _lib.strides(out),
                                  _lib.stream_ptr(indexer_scores.device))
    _lib.check(rc)
    return out


def flash_csa_forward(
    q: torch.Tensor,
    kv: torch.Tensor,
    kv_compressed: torch.Tensor,
    q_idx: torch.Tensor,
    k_idx_compressed: torch.Tensor,
    indexer_weights: torch.Tensor,
    attn_sink: torch.Tensor,
    *,
    n_win: int,
    top_k: int,
    m: int = 4,
    softmax_scale: Optional[float] = None,
    use_triton: bool = True,
    use_chunked_indexer: Optional[bool] = None,
    chunk_s: int = 1024,
    chunk_t: int = 4096,
    auto_chunk_threshold_bytes: int = 1 << 30,
    quantized_indexer: bool = False,
) -> torch.Tensor:
    """End-to-end CSA forward, prefill path, one layer (``csa.py:86-207``).

    Args:
      q: ``[B, S, n_h, d]`` bf16 RoPE-rotated queries.
      kv: ``[B, S, d]`` bf16 uncompressed KV (sliding-window source).
      kv_compressed: ``[B, S/m, d]`` bf16 compressed KV.
      q_idx: ``[B, S, n_I_h, c_I]`` bf16 indexer queries.
      k_idx_compressed: ``[B, S/m, c_I]`` bf16 indexer keys.
      indexer_weights: ``[B, S, n_I_h]`` fp32 per-head weights.
      attn_sink: ``[n_h]`` fp32.
      n_win, top_k, m: window size, compressed picks per query, compression ratio.
      softmax_scale: defaults to ``d ** -0.5``.
      use_triton, use_chunked_indexer, chunk_s, chunk_t, auto_chunk_threshold_bytes:
        accepted for compatibility; every setting runs the same exact HIP path.
      quantized_indexer: select with the fp4 x fp8 indexer (the production V4
        indexer dtypes, see :func:`csa_topk_idxs`) instead of bf16.
    Returns:
      ``o: [B, S, n_h, d]`` bf16.
    """
    del use_triton, use_chunked_indexer, auto_chunk_threshold_bytes
    B, S, n_h, d = q.shape
    assert kv.shape == (B, S, d)
    n_compressed = kv_compressed.shape[1]
    assert kv_compressed.shape == (B, n_compressed, d)
    assert k_idx_compressed.shape[1] == n_compressed
    if int(chunk_s) <= 0 or int(chunk_t) <= 0:
        raise ValueError(f"chunk_s and chunk_t must be positive, got {chunk_s}, {chunk_t}")
    topk_idxs = csa_topk_idxs(q_idx, k_idx_compressed, indexer_weights, n_win=n_win, top_k=top_k, m=m,
                              seq_len=S, quantized=quantized_indexer)
    row_len = csa_row_len(B, S, n_win, top_k, n_compressed, m, q.device)
    # the rows index [kv ; kv_compressed]; the kernel reads both in place
    return sparse_attn_kv2(q, kv, kv_compressed, attn_sink, topk_idxs, softmax_scale, row_len=row_len)


def csa_row_len(B: int, S: int, n_win: int, top_k: int, n_compressed: int, m: int, device) -> torch.Tensor:
    """``[B, S]`` int32 used columns of the fused CSA rows: the window, then
    ``min(top_k, n_compressed, (s+1)//m)`` picks (every legal key has a finite
    score, so a row holds that many); the ``-1`` rest is never run."""
    s = torch.arange(S, device=device)
    legal = torch.clamp((s + 1) // m, max=n_compressed)
    return (n_win + torch.clamp(legal, max=top_k)).to(torch.int32).expand(B, S)
