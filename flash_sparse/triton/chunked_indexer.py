"""Reference module path of ``chunked_indexer_topk`` (``flash_sparse/triton/chunked_indexer.py:47``)."""

from streamindex_amd.indexer import chunked_indexer_topk

__all__ = ["chunked_indexer_topk"]
