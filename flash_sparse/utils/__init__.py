"""Reference module path ``flash_sparse.utils`` (quantisation and compression helpers)."""
