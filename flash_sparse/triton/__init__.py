"""Reference module path ``flash_sparse.triton`` (see ``flash_sparse/triton/__init__.py:16-63``
in the reference): operators (and the sparse-attention backward) backed by the gfx950 HIP kernels."""

from streamindex_amd.indexer import chunked_indexer_topk, indexer_score, indexer_score_topk
from streamindex_amd.sparse_attn import sparse_attn, sparse_attn_bwd, sparse_attn_fwd

__all__ = ["sparse_attn", "sparse_attn_fwd", "sparse_attn_bwd", "chunked_indexer_topk", "indexer_score", "indexer_score_topk"]
