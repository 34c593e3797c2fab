"""Writes the small golden fixtures under tests/golden/ (inputs + expected outputs).

The reference ships no data files and its CUDA-seeded inputs are not
reproducible here, so these vectors are produced by this repository's CPU
oracle (oracle/) — itself pinned by tests/test_oracle.py — from seeded numpy
inputs.  They freeze the expected outputs so that any later change to the
oracle or the kernels that moves a result is caught.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def bf16(rng, shape, scale):
    return O.f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32) * scale)


def indexer_case(name, S, H, D, T, top_k, ratio, seed, scale=None, tie_rows=0):
    rng = np.random.default_rng(seed)
    sc = D ** -0.5 if scale is None else scale
    q = bf16(rng, (S, H, D), sc)
    k = bf16(rng, (T, D), sc)
    if tie_rows:
        k[tie_rows:2 * tie_rows] = k[:tie_rows]  # duplicated keys -> exact score ties
    w = rng.standard_normal((S, H)).astype(np.float32)
    idx, val, _ = O.indexer_topk_rows(q, k, w, top_k, causal_ratio=ratio)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), q=q, k=k, w=w, top_k=top_k,
                        ratio=-1 if ratio is None else ratio, idx=idx, score=val)


def attn_case(name, S, H, D, N, K, seed):
    rng = np.random.default_rng(seed)
    q = bf16(rng, (S, H, D), 1.0)
    kv = bf16(rng, (N, D), 1.0)
    sink = rng.standard_normal(H).astype(np.float32)
    idx = rng.integers(0, N, (S, K)).astype(np.int64)
    idx[rng.random((S, K)) < 0.2] = -1
    idx[0, :] = -1  # one fully masked row
    scale = D ** -0.5
    o, lse = O.sparse_attn_rows(q, kv, sink, idx, scale)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), q=q, kv=kv, sink=sink, idx=idx, scale=scale,
                        o=o.astype(np.float32), lse=lse.astype(np.float32))


def main():
    indexer_case("indexer_v4_causal", S=16, H=64, D=128, T=8, top_k=4, ratio=2, seed=1)
    indexer_case("indexer_small_unmasked", S=40, H=16, D=32, T=70, top_k=12, ratio=None, seed=2, scale=0.5)
    indexer_case("indexer_ties", S=24, H=16, D=64, T=48, top_k=20, ratio=None, seed=3, tie_rows=16)
    attn_case("attn_d576", S=3, H=16, D=576, N=40, K=24, seed=4)
    attn_case("attn_d64", S=10, H=16, D=64, N=32, K=20, seed=5)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
