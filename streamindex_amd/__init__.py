"""StreamIndex for MI355X: the DeepSeek-V4 CSA hot path on gfx950.

Operators (hand-written HIP kernels behind the C ABI in
``include/streamindex.h``, loaded from ``streamindex_amd/lib/libstreamindex.so``):

* :func:`chunked_indexer_topk` — fused lightning-indexer score + exact top-k;
* :func:`indexer_score`, :func:`indexer_score_topk`;
* :func:`indexer_topk_q`, :func:`chunked_indexer_topk_quantized` — the indexer over fp4
  queries and fp8 keys (the production V4 indexer dtypes), and
  ``streamindex_amd.quant`` / ``streamindex_amd.compressor`` for the quantisers and the
  token compressor;
* :func:`sparse_attn_fwd`, :func:`sparse_attn_bwd`, :func:`sparse_attn` — MQA sparse attention
  with sink, its backward and the autograd wrapper;
* :func:`flash_csa_forward`, :func:`build_csa_topk_idxs`, :func:`csa_topk_idxs` —
  the CSA composition (fused indexer → window + compressed index rows → attention);
* :func:`flash_hca_forward`, :func:`build_hca_topk_idxs` — HCA (window + every
  legal compressed entry).

The same names are importable under the reference's module paths through the
``flash_sparse`` package (``flash_sparse.triton.chunked_indexer`` etc.).
"""

from .indexer import (chunked_indexer_topk, chunked_indexer_topk_quantized, indexer_score, indexer_score_topk,
                      indexer_topk_q)
from .sparse_attn import (build_inverted_topk, sparse_attn, sparse_attn_bwd, sparse_attn_bwd_v2, sparse_attn_fwd,
                          sparse_attn_fwd_kv2, sparse_attn_kv2)
from .csa import build_csa_topk_idxs, csa_topk_idxs, flash_csa_forward
from .hca import build_hca_topk_idxs, flash_hca_forward

__version__ = "0.1.0"

__all__ = [
    "chunked_indexer_topk",
    "chunked_indexer_topk_quantized",
    "indexer_topk_q",
    "indexer_score",
    "indexer_score_topk",
    "sparse_attn",
    "sparse_attn_bwd",
    "sparse_attn_bwd_v2",
    "build_inverted_topk",
    "sparse_attn_fwd",
    "sparse_attn_fwd_kv2",
    "sparse_attn_kv2",
    "flash_csa_forward",
    "build_csa_topk_idxs",
    "csa_topk_idxs",
    "flash_hca_forward",
    "build_hca_topk_idxs",
]
