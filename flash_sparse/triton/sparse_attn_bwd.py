"""Reference module path of ``sparse_attn_bwd`` (``flash_sparse/triton/sparse_attn_bwd.py:286``)."""

from streamindex_amd.sparse_attn import sparse_attn_bwd

__all__ = ["sparse_attn_bwd"]
