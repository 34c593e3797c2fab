"""Reference module path of ``softmax_gated_pool`` (``flash_sparse/utils/compression.py:13``)."""

from streamindex_amd.compressor import softmax_gated_pool

__all__ = ["softmax_gated_pool"]
