"""Seeded synthetic inputs with the V4-Flash indexer / CSA distributions.

Distributions follow the reference's harness (``eval/test_v4_indexer_parity.py:67-105``)
as restated for this build's configs: ``q ~ N(0,1)·D_I^-1/2`` and
``k_idx ~ N(0,1)·D_I^-1/2`` in bf16, ``weights ~ N(0,1)`` fp32.

Small problems are drawn on a CPU ``torch.Generator`` in the order q, k_idx,
weights and copied to the device.  Large ones (q above 2^26 elements: the
benchmark configs) are drawn on the device by ``si_fill_normal``, a
counter-based generator whose element i of a tensor depends only on (seed,
tensor stream, i): the tensors are bit-identical on every box and ROCm
version, any slice can be recomputed on the CPU (``oracle.synth_normal``), and
no multi-GiB host tensor is needed.  Each tensor has its own stream id
(``STREAMS``); the value is rounded once, after the scale, to the tensor's
dtype.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

CPU_DRAW_LIMIT = 1 << 26  # elements of q above which inputs are drawn on-device

# Counter-based stream id of each synthetic tensor.
STREAMS = {"indexer.q": 1, "indexer.k": 2, "indexer.w": 3,
           "attn.q": 11, "attn.kv": 12, "attn.sink": 13,
           "csa.q": 21, "csa.kv": 22, "csa.kvc": 23, "csa.sink": 24}


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def device_normal(shape, dtype, *, seed: int, stream: int, scale: float = 1.0, device="cuda") -> torch.Tensor:
    """A new contiguous CUDA tensor of N(0,1)·scale drawn by ``si_fill_normal``
    (bf16 or fp32)."""
    from . import _lib

    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"device_normal draws bf16 or fp32, not {dtype}")
    t = torch.empty(shape, dtype=dtype, device=device)
    L = _lib.load()
    with torch.cuda.device(t.device):
        rc = L.si_fill_normal(t.data_ptr(), 1 if dtype == torch.bfloat16 else 0, t.numel(), int(seed), int(stream),
                              float(scale), _lib.stream_ptr(t.device))
    _lib.check(rc)
    return t


def indexer_inputs(B: int, S: int, H: int, D: int, T: Optional[int] = None, *, ratio: int = 4, seed: int = 2026,
                   device="cuda", weights_dtype=torch.float32, q_scale: Optional[float] = None,
                   k_scale: Optional[float] = None):
    """Returns ``(q [B,S,H,D] bf16, k_idx [B,T,D] bf16, weights [B,S,H])`` with T = S // ratio by default."""
    device = torch.device(device)
    T = S // ratio if T is None else T
    qs = D ** -0.5 if q_scale is None else q_scale
    ks = D ** -0.5 if k_scale is None else k_scale
    if device.type == "cuda" and B * S * H * D > CPU_DRAW_LIMIT:
        q = device_normal((B, S, H, D), torch.bfloat16, seed=seed, stream=STREAMS["indexer.q"], scale=qs, device=device)
        k = device_normal((B, T, D), torch.bfloat16, seed=seed, stream=STREAMS["indexer.k"], scale=ks, device=device)
        w = device_normal((B, S, H), torch.float32, seed=seed, stream=STREAMS["indexer.w"], device=device)
        return q, k, w.to(weights_dtype)
    g = _gen(seed)
    q = torch.randn(B, S, H, D, generator=g, dtype=torch.bfloat16) * qs
    k = torch.randn(B, T, D, generator=g, dtype=torch.bfloat16) * ks
    w = torch.randn(B, S, H, generator=g, dtype=torch.float32).to(weights_dtype)
    return q.to(device), k.to(device), w.to(device)


def sparse_attn_inputs(B: int, S: int, H: int, D: int, N_kv: int, *, seed: int = 2027, device="cuda",
                       q_scale: float = 1.0, kv_scale: float = 1.0):
    """Returns ``(q [B,S,H,D] bf16, kv [B,N_kv,D] bf16, attn_sink [H] fp32)``."""
    device = torch.device(device)
    if device.type == "cuda" and B * S * H * D > CPU_DRAW_LIMIT:
        q = device_normal((B, S, H, D), torch.bfloat16, seed=seed, stream=STREAMS["attn.q"], scale=q_scale,
                          device=device)
        kv = device_normal((B, N_kv, D), torch.bfloat16, seed=seed, stream=STREAMS["attn.kv"], scale=kv_scale,
                           device=device)
        sink = device_normal((H,), torch.float32, seed=seed, stream=STREAMS["attn.sink"], device=device)
        return q, kv, sink
    g = _gen(seed)
    q = torch.randn(B, S, H, D, generator=g, dtype=torch.bfloat16) * q_scale
    kv = torch.randn(B, N_kv, D, generator=g, dtype=torch.bfloat16) * kv_scale
    sink = torch.randn(H, generator=g, dtype=torch.float32)
    return q.to(device), kv.to(device), sink.to(device)


def csa_attn_inputs(B: int, S: int, H: int, D: int, T: int, *, seed: int = 2027, device="cuda",
                    scale: float = 1.0):
    """Attention-side CSA inputs: ``(q [B,S,H,D], kv [B,S,D], kv_compressed [B,T,D])``
    bf16 ~ N(0,1)·scale and ``attn_sink [H]`` fp32 ~ N(0,1).  Large tensors are
    drawn on the device directly in their dtype (no second copy at S = 1M,
    where q alone is 72 GiB)."""
    device = torch.device(device)
    shapes = ((B, S, H, D), (B, S, D), (B, T, D))
    if device.type == "cuda" and B * S * H * D > CPU_DRAW_LIMIT:
        out = [device_normal(shape, torch.bfloat16, seed=seed, stream=STREAMS[name], scale=scale, device=device)
               for shape, name in zip(shapes, ("csa.q", "csa.kv", "csa.kvc"))]
        out.append(device_normal((H,), torch.float32, seed=seed, stream=STREAMS["csa.sink"], device=device))
        return tuple(out)
    g = _gen(seed)
    out = []
    for shape in shapes:
        t = torch.randn(*shape, generator=g, dtype=torch.bfloat16)
        if scale != 1.0:
            t.mul_(scale)
        out.append(t.to(device))
    out.append(torch.randn(H, generator=g, dtype=torch.float32).to(device))
    return tuple(out)


def causal_random_topk(B: int, S: int, K: int, ratio: int, *, seed: int = 7, device="cuda") -> torch.Tensor:
    """Random distinct causal-legal compressed indices per row (``-1`` past the
    legal count), for attention tests that do not run the indexer first."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    out = torch.full((B, S, K), -1, dtype=torch.int64)
    for s in range(S):
        lim = (s + 1) // ratio
        n = min(K, lim)
        if n == 0:
            continue
        for b in range(B):
            out[b, s, :n] = torch.randperm(lim, generator=g)[:n]
    return out.to(device)


def legal_pairs(S: int, T: int, ratio: int) -> int:
    """Σ_s min(T, (s+1)//ratio): causally legal (query, key) pairs."""
    total = 0
    # closed form over blocks of `ratio` queries sharing one limit
    full = min(S, T * ratio)
    # s in [0, full): limit = (s+1)//ratio
    q, r = divmod(full, ratio)
    # sum_{s=0}^{full-1} floor((s+1)/ratio) = sum_{m=1}^{full} floor(m/ratio)
    total += ratio * (q * (q - 1) // 2) + q * (r + 1) if full > 0 else 0
    if S > full:
        total += (S - full) * T
    return total


def indexer_flops(S: int, T: int, H: int, D: int, ratio: Optional[int]) -> float:
    """Algorithmic FLOPs of the score stage (2·H·D per legal (s,t) pair)."""
    pairs = S * T if ratio is None else legal_pairs(S, T, ratio)
    return 2.0 * H * D * pairs


def _check_legal_pairs():  # pragma: no cover - used by tests
    for S in (1, 3, 4, 5, 17, 64):
        for T in (0, 1, 3, 16, 100):
            for r in (1, 2, 4):
                brute = sum(min(T, (s + 1) // r) for s in range(S))
                assert legal_pairs(S, T, r) == brute, (S, T, r)
    return True


__all__ = ["indexer_inputs", "sparse_attn_inputs", "csa_attn_inputs", "causal_random_topk", "legal_pairs",
           "indexer_flops", "device_normal", "STREAMS"]
del math
