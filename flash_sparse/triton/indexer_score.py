"""Reference module path of ``indexer_score`` / ``indexer_score_topk``
(``flash_sparse/triton/indexer_score.py:123,182``)."""

from streamindex_amd.indexer import indexer_score, indexer_score_topk

__all__ = ["indexer_score", "indexer_score_topk"]
