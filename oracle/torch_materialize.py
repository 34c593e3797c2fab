"""The reference's CPU indexer path, restated op for op in torch fp32 — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` import this
module.  It is the CPU baseline that the benchmark reports beside the GPU
kernel, and it is checked against the C oracle (``si_oracle.c``) in
``tests/test_oracle.py``; the product (``streamindex_amd``) never uses it.

Ops, in the reference's order (file:line in the reference tree):

1. ``einsum("bshd,btd->bsht", q.float(), k.float())`` —
   ``flash_sparse/reference.py:164-165``, ``eval/test_v4_indexer_parity.py:121``;
2. ReLU — ``reference.py:166`` (``relu_``);
3. ``(scores * weights.unsqueeze(-1)).sum(dim=2)`` — ``reference.py:168``,
   ``eval/test_v4_indexer_parity.py:122``;
4. illegal ``t >= (s+1)//ratio`` filled with ``-inf`` —
   ``eval/test_v4_indexer_parity.py:124-128``;
5. ``topk(min(top_k, T), dim=-1)`` — ``:129-130``;
6. post-mask: picks ``>= (s+1)//ratio`` become ``-1`` — ``:132-136``.
"""

from __future__ import annotations

import os
import platform
import statistics
import time
from typing import Optional

import torch


def materialize_topk(q: torch.Tensor, k_idx: torch.Tensor, weights: torch.Tensor, top_k: int,
                     ratio: int):
    """Returns ``(topk_idxs int64 [B,S,min(k,T)], topk_scores fp32)`` exactly as the
    reference's materialise path computes them (CPU, fp32)."""
    B, S, _, _ = q.shape
    T = k_idx.shape[1]
    scores = torch.einsum("bshd,btd->bsht", q.float(), k_idx.float())
    scores.relu_()
    scores = (scores * weights.float().unsqueeze(-1)).sum(dim=2)
    t = torch.arange(T).repeat(S, 1)
    boundary = torch.arange(1, S + 1).unsqueeze(1) // ratio
    illegal = t >= boundary
    scores = scores.masked_fill(illegal.unsqueeze(0), float("-inf"))
    k_eff = min(top_k, T)
    vals, idx = scores.topk(k_eff, dim=-1)
    invalid = idx >= boundary.unsqueeze(0)
    idx = torch.where(invalid, torch.full_like(idx, -1), idx)
    return idx, vals


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_threads() -> int:
    """Threads to use on this host: the cores this process may run on, capped
    by OMP_NUM_THREADS where the host sets it (a GPU box's share of a larger
    machine)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover - non-Linux
        n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def time_materialize(q, k_idx, weights, top_k: int, ratio: int, *, threads: Optional[int] = None,
                     warmup: int = 1, repeats: int = 3) -> dict:
    """Times :func:`materialize_topk` on the CPU: ``warmup`` untimed runs, then
    ``repeats`` timed runs with ``time.perf_counter``."""
    threads = host_threads() if threads is None else threads
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        out = None
        for _ in range(warmup):
            out = materialize_topk(q, k_idx, weights, top_k, ratio)
        runs = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            out = materialize_topk(q, k_idx, weights, top_k, ratio)
            runs.append((time.perf_counter() - t0) * 1e3)
    finally:
        torch.set_num_threads(prev)
    return {"ms": statistics.median(runs), "runs_ms": runs, "threads": threads, "os_cpu_count": os.cpu_count(),
            "cpu_model": cpu_model(), "out": out}


__all__ = ["materialize_topk", "time_materialize", "cpu_model", "host_threads"]
