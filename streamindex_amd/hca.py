"""Heavily Compressed Attention (HCA) forward on MI355X.

Mirrors ``flash_sparse/hca.py:24-95`` (``build_hca_topk_idxs``,
``flash_hca_forward``).  HCA has no indexer: a query at position ``s``
attends to its sliding window of the uncompressed KV and to every causally
legal compressed entry (``m'·(i+1) - 1 <= s``), through the same
sparse-attention kernel as CSA.  The index rows are written by one HIP kernel
(one workgroup per query row) instead of the reference's torch
arange/where/cat passes.

``use_triton`` is accepted for compatibility and selects nothing (one HIP
implementation).  Gradients flow through ``sparse_attn``'s autograd.
"""

from __future__ import annotations

from typing import Optional

import torch

from .csa import _launch_hca
from .sparse_attn import sparse_attn_kv2

__all__ = ["flash_hca_forward", "build_hca_topk_idxs", "hca_row_len"]


def build_hca_topk_idxs(*, B: int, seq_len: int, n_win: int, n_compressed: int, m_prime: int,
                        device: torch.device) -> torch.Tensor:
    """``[B, S, n_win + n_compressed]`` int32 HCA index rows (``hca.py:24-51``).

    Window columns ``s-n_win+1 .. s`` (``-1`` below 0), then compressed entry
    ``i`` as ``i + seq_len`` where ``m_prime·(i+1) - 1 <= s``, else ``-1``.
    """
    if n_win < 0 or n_compressed < 0 or m_prime <= 0:
        raise ValueError(f"bad HCA shape: n_win={n_win}, n_compressed={n_compressed}, m_prime={m_prime}")
    device = torch.device(device)
    assert device.type == "cuda"
    out = torch.empty((B, seq_len, n_win + n_compressed), dtype=torch.int32, device=device)
    _launch_hca(out, B, seq_len, n_win, n_compressed, m_prime, seq_len)
    return out


def flash_hca_forward(
    q: torch.Tensor,
    kv: torch.Tensor,
    kv_compressed: torch.Tensor,
    attn_sink: torch.Tensor,
    *,
    n_win: int,
    m_prime: int = 128,
    softmax_scale: Optional[float] = None,
    use_triton: bool = True,
) -> torch.Tensor:
    """End-to-end HCA forward, prefill path, one layer (``hca.py:54-95``).

    Args:
      q: ``[B, S, n_h, d]`` bf16.  kv: ``[B, S, d]`` bf16 uncompressed KV.
      kv_compressed: ``[B, S/m_prime, d]`` bf16.  attn_sink: ``[n_h]`` fp32.
      n_win: sliding-window size.  m_prime: HCA compression ratio.
      softmax_scale: defaults to ``d ** -0.5``.
    Returns:
      ``o: [B, S, n_h, d]`` bf16.
    """
    del use_triton
    B, S, n_h, d = q.shape
    n_compressed = kv_compressed.shape[1]
    assert q.is_cuda
    topk_idxs = build_hca_topk_idxs(B=B, seq_len=S, n_win=n_win, n_compressed=n_compressed, m_prime=m_prime,
                                    device=q.device)
    row_len = hca_row_len(B, S, n_win, n_compressed, m_prime, q.device)
    # the rows index [kv ; kv_compressed]; the kernel reads both in place
    return sparse_attn_kv2(q, kv, kv_compressed, attn_sink, topk_idxs, softmax_scale, row_len=row_len)


def hca_row_len(B: int, S: int, n_win: int, n_compressed: int, m_prime: int, device) -> torch.Tensor:
    """``[B, S]`` int32 used columns of the HCA rows: the window, then the
    ``min(n_compressed, (s+1)//m_prime)`` legal compressed entries; the rest
    of each row is ``-1``, so attention never runs those tiles."""
    s = torch.arange(S, device=device)
    return (n_win + torch.clamp((s + 1) // m_prime, max=n_compressed)).to(torch.int32).expand(B, S)
