"""Reference module path of ``sparse_attn_bwd_v2`` (``flash_sparse/triton/sparse_attn_bwd_v2.py:381``)."""

from streamindex_amd.sparse_attn import sparse_attn_bwd_v2

__all__ = ["sparse_attn_bwd_v2"]
