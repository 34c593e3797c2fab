"""Reference module path of ``sparse_attn_fwd`` (``flash_sparse/triton/sparse_attn_fwd.py:180``)."""

from streamindex_amd.sparse_attn import sparse_attn_fwd

__all__ = ["sparse_attn_fwd"]
