"""Reference module path ``flash_sparse.hca`` (``flash_sparse/hca.py:21`` in the reference):
the HCA composition backed by the gfx950 HIP kernels."""

from streamindex_amd.hca import build_hca_topk_idxs, flash_hca_forward

__all__ = ["flash_hca_forward", "build_hca_topk_idxs"]
