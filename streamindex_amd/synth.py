"""Seeded synthetic inputs with the V4-Flash indexer / CSA distributions.

Distributions follow the reference's harness (``eval/test_v4_indexer_parity.py:67-105``)
as restated for this build's configs: ``q ~ N(0,1)·D_I^-1/2`` and
``k_idx ~ N(0,1)·D_I^-1/2`` in bf16, ``weights ~ N(0,1)`` fp32, drawn in the
order q, k_idx, weights from one generator.  Small problems are drawn on a CPU
generator (bit-reproducible across machines) and copied to the device; large
ones are drawn on the device generator to avoid multi-GiB host tensors.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

CPU_DRAW_LIMIT = 1 << 26  # elements of q above which inputs are drawn on-device


def _gen(device: torch.device, seed: int, on_device: bool) -> torch.Generator:
    g = torch.Generator(device=device if on_device else "cpu")
    g.manual_seed(seed)
    return g


def indexer_inputs(B: int, S: int, H: int, D: int, T: Optional[int] = None, *, ratio: int = 4, seed: int = 2026,
                   device="cuda", weights_dtype=torch.float32, q_scale: Optional[float] = None,
                   k_scale: Optional[float] = None):
    """Returns ``(q [B,S,H,D] bf16, k_idx [B,T,D] bf16, weights [B,S,H])`` with T = S // ratio by default."""
    device = torch.device(device)
    T = S // ratio if T is None else T
    on_dev = device.type == "cuda" and B * S * H * D > CPU_DRAW_LIMIT
    g = _gen(device, seed, on_dev)
    where = device if on_dev else "cpu"
    qs = D ** -0.5 if q_scale is None else q_scale
    ks = D ** -0.5 if k_scale is None else k_scale
    q = torch.randn(B, S, H, D, generator=g, device=where, dtype=torch.bfloat16) * qs
    k = torch.randn(B, T, D, generator=g, device=where, dtype=torch.bfloat16) * ks
    w = torch.randn(B, S, H, generator=g, device=where, dtype=torch.float32).to(weights_dtype)
    return q.to(device), k.to(device), w.to(device)


def sparse_attn_inputs(B: int, S: int, H: int, D: int, N_kv: int, *, seed: int = 2027, device="cuda",
                       q_scale: float = 1.0, kv_scale: float = 1.0):
    """Returns ``(q [B,S,H,D] bf16, kv [B,N_kv,D] bf16, attn_sink [H] fp32)``."""
    device = torch.device(device)
    on_dev = device.type == "cuda" and B * S * H * D > CPU_DRAW_LIMIT
    g = _gen(device, seed, on_dev)
    where = device if on_dev else "cpu"
    q = torch.randn(B, S, H, D, generator=g, device=where, dtype=torch.bfloat16) * q_scale
    kv = torch.randn(B, N_kv, D, generator=g, device=where, dtype=torch.bfloat16) * kv_scale
    sink = torch.randn(H, generator=g, device=where, dtype=torch.float32)
    return q.to(device), kv.to(device), sink.to(device)


def csa_attn_inputs(B: int, S: int, H: int, D: int, T: int, *, seed: int = 2027, device="cuda",
                    scale: float = 1.0):
    """Attention-side CSA inputs: ``(q [B,S,H,D], kv [B,S,D], kv_compressed [B,T,D])``
    bf16 ~ N(0,1)·scale and ``attn_sink [H]`` fp32 ~ N(0,1).  Large tensors are
    drawn on the device and scaled in place (no second copy at S = 1M, where q
    alone is 72 GiB)."""
    device = torch.device(device)
    on_dev = device.type == "cuda" and B * S * H * D > CPU_DRAW_LIMIT
    g = _gen(device, seed, on_dev)
    where = device if on_dev else "cpu"
    out = []
    for shape in ((B, S, H, D), (B, S, D), (B, T, D)):
        t = torch.randn(*shape, generator=g, device=where, dtype=torch.bfloat16)
        if scale != 1.0:
            t.mul_(scale)
        out.append(t.to(device))
    out.append(torch.randn(H, generator=g, device=where, dtype=torch.float32).to(device))
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
           "indexer_flops"]
del math
