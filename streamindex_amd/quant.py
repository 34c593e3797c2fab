"""FP8 / FP4 activation quantisation on MI355X (gfx950 HIP kernels via the C ABI).

Mirrors ``flash_sparse/utils/quantization.py`` of the reference:

* :func:`act_quant_simulate` (``quantization.py:19-37``) and
  :func:`fp4_act_quant_simulate` (``quantization.py:40-65``): quantise then
  dequantise, same signature, dtype and result — bit for bit, including the
  rounding to the input dtype after every step of the reference formula.

and adds the packed production formats that the reference's docstring names
(``quantization.py:3-9``, DeepSeek-V4's ``act_quant`` / ``fp4_act_quant``):

* :func:`act_quant` — fp8 e4m3 values (``torch.float8_e4m3fn``) and one fp32
  scale per block (``amax / 448``, or its power-of-two ceiling with
  ``scale_fmt="ue8m0"``);
* :func:`fp4_act_quant` — e2m1 values packed two per byte (element ``2i`` in
  the low nibble) and one power-of-two (UE8M0) scale per block of 32, the
  layout :func:`streamindex_amd.chunked_indexer_topk_fp8` reads.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _dtype_code(x: torch.Tensor) -> int:
    if x.dtype not in _DT:
        raise ValueError(f"dtype must be float32, bfloat16 or float16, got {x.dtype}")
    return _DT[x.dtype]


def _check_blocks(x: torch.Tensor, block_size: int) -> None:
    n = x.shape[-1]
    assert n % block_size == 0, f"last dim {n} must be divisible by block_size {block_size}"


def _simulate(x: torch.Tensor, block_size: int, fp4: bool) -> torch.Tensor:
    assert x.is_cuda, "x must be on the GPU"
    _check_blocks(x, block_size)
    dt = _dtype_code(x)
    xc = x.contiguous()
    y = torch.empty_like(xc)
    L = _lib.load()
    with torch.cuda.device(x.device):
        rc = L.si_quant_simulate(xc.data_ptr(), y.data_ptr(), dt, xc.numel(), block_size, int(fp4),
                                 _lib.stream_ptr(x.device))
    _lib.check(rc)
    return y


def act_quant_simulate(x: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """Per-block fp8 e4m3 quantise-dequantise (``quantization.py:19-37``)."""
    return _simulate(x, block_size, False)


def fp4_act_quant_simulate(x: torch.Tensor, block_size: int = 32) -> torch.Tensor:
    """Per-block fp4 e2m1 quantise-dequantise (``quantization.py:40-65``)."""
    return _simulate(x, block_size, True)


def act_quant(x: torch.Tensor, block_size: int = 128, scale_fmt: Optional[str] = None
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp8 e4m3 values and fp32 per-block scales (``x ≈ values · scale``).

    ``scale = max(amax, 1e-4) / 448``; with ``scale_fmt="ue8m0"`` the scale is
    rounded up to a power of two.  Values are ``x / scale`` clamped to ±448 and
    rounded to the nearest e4m3 value (ties to even).
    """
    assert x.is_cuda, "x must be on the GPU"
    _check_blocks(x, block_size)
    if scale_fmt not in (None, "ue8m0"):
        raise ValueError(f"scale_fmt must be None or 'ue8m0', got {scale_fmt!r}")
    dt = _dtype_code(x)
    xc = x.contiguous()
    y = torch.empty(xc.shape, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((*xc.shape[:-1], xc.shape[-1] // block_size), dtype=torch.float32, device=x.device)
    L = _lib.load()
    with torch.cuda.device(x.device):
        rc = L.si_quant_pack(xc.data_ptr(), y.data_ptr(), s.data_ptr(), dt, xc.numel(), block_size, 0,
                             int(scale_fmt == "ue8m0"), _lib.stream_ptr(x.device))
    _lib.check(rc)
    return y, s


def fp4_act_quant(x: torch.Tensor, block_size: int = 32) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp4 e2m1 values packed two per byte and power-of-two per-block scales.

    ``scale = 2^ceil(log2(max(amax, 6·2^-126) / 6))`` (UE8M0), values are the
    nearest e2m1 value to ``x / scale`` (ties to the even code); returns
    ``(packed uint8 [..., n/2], scale fp32 [..., n/block_size])``.
    """
    assert x.is_cuda, "x must be on the GPU"
    _check_blocks(x, block_size)
    dt = _dtype_code(x)
    xc = x.contiguous()
    y = torch.empty((*xc.shape[:-1], xc.shape[-1] // 2), dtype=torch.uint8, device=x.device)
    s = torch.empty((*xc.shape[:-1], xc.shape[-1] // block_size), dtype=torch.float32, device=x.device)
    L = _lib.load()
    with torch.cuda.device(x.device):
        rc = L.si_quant_pack(xc.data_ptr(), y.data_ptr(), s.data_ptr(), dt, xc.numel(), block_size, 1, 1,
                             _lib.stream_ptr(x.device))
    _lib.check(rc)
    return y, s


__all__ = ["act_quant_simulate", "fp4_act_quant_simulate", "act_quant", "fp4_act_quant"]
