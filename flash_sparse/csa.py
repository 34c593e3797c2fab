"""Reference module path ``flash_sparse.csa`` (``flash_sparse/csa.py:27`` in the reference):
the CSA composition backed by the gfx950 HIP kernels."""

from streamindex_amd.csa import build_csa_topk_idxs, flash_csa_forward

__all__ = ["flash_csa_forward", "build_csa_topk_idxs"]
