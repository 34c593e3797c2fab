"""Reference module path of ``streaming_indexer_topk``
(``flash_sparse/triton/indexer_streaming_topk.py:48``).

The reference parks this entry point (it always raises ``NotImplementedError``)
and describes the design it wants: the ``[B, S, T]`` score matrix never leaves
the chip, scores are packed with their indices as sortable keys that order
negative scores correctly, and only the top-k reaches HBM.  That is what the
fused HIP kernel behind ``chunked_indexer_topk`` does, so here the name runs it.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from streamindex_amd.indexer import chunked_indexer_topk


def streaming_indexer_topk(
    q: torch.Tensor,
    k_idx: torch.Tensor,
    weights: torch.Tensor,
    top_k: int,
    *,
    causal_mask: Optional[torch.Tensor] = None,
    causal_ratio: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused score + streaming exact top-k: ``(idx [B,S,top_k] int64, scores [B,S,top_k] fp32)``,
    with the arguments and results of ``chunked_indexer_topk``."""
    return chunked_indexer_topk(q, k_idx, weights, top_k, causal_mask=causal_mask, causal_ratio=causal_ratio)


__all__ = ["streaming_indexer_topk"]
