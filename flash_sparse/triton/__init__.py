"""Reference module path ``flash_sparse.triton`` (``flash_sparse/triton/__init__.py:16-63`` in the
reference): ``sparse_attn`` (autograd), ``sparse_attn_fwd`` and ``sparse_attn_bwd``, backed by the
gfx950 HIP kernels.  Each name is imported from its submodule, as the reference does, so importing
``flash_sparse.triton.sparse_attn_fwd`` later cannot rebind the package attribute to the module."""

from flash_sparse.triton.sparse_attn_fwd import sparse_attn_fwd
from flash_sparse.triton.sparse_attn_bwd import sparse_attn_bwd
from streamindex_amd.sparse_attn import sparse_attn

__all__ = ["sparse_attn", "sparse_attn_fwd", "sparse_attn_bwd"]
