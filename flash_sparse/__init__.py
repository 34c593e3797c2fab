"""Reference-compatible import paths for the MI355X StreamIndex operators.

``flash_sparse.triton.chunked_indexer.chunked_indexer_topk`` and
``flash_sparse.triton.sparse_attn_fwd`` resolve to the gfx950 HIP
implementations in :mod:`streamindex_amd`; the ``triton`` name is kept only so
callers of the reference (``flash_sparse/triton/__init__.py:16,63``) switch
without edits.  Nothing here imports Triton.
"""

__version__ = "0.1.0"
