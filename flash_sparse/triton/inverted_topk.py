"""Reference module path of ``build_inverted_topk`` (``flash_sparse/triton/inverted_topk.py:75``)."""

from streamindex_amd.sparse_attn import build_inverted_topk

__all__ = ["build_inverted_topk"]
