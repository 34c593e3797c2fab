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


def attn_bwd_case(name, S, H, D, N, K, seed):
    # the forward's o (rounded to bf16, as the kernel saves it) and lse feed the backward
    rng = np.random.default_rng(seed)
    q = bf16(rng, (S, H, D), 0.5)
    kv = bf16(rng, (N, D), 0.5)
    sink = rng.standard_normal(H).astype(np.float32)
    idx = rng.integers(0, N, (S, K)).astype(np.int64)
    idx[rng.random((S, K)) < 0.2] = -1
    idx[1, :] = -1  # one fully masked row
    idx[2, :4] = idx[2, 4]  # a key selected several times by one row
    scale = D ** -0.5
    o, lse = O.sparse_attn_rows(q, kv, sink, idx, scale)
    o_bits = O.f32_to_bf16_bits(o.astype(np.float32))
    do = bf16(rng, (S, H, D), 1.0)
    lse = lse.astype(np.float32)
    dq, dkv, dsink = O.sparse_attn_bwd_rows(q, kv, o_bits, do, sink, lse, idx, scale)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), q=q, kv=kv, sink=sink, idx=idx, scale=scale, o=o_bits,
                        lse=lse, do=do, dq=dq.astype(np.float32), dkv=dkv.astype(np.float32),
                        dsink=dsink.astype(np.float32))


def quant_case(name, rows, cols, seed):
    # fp32 and bf16 inputs: simulations (fp8 blocks of 128, fp4 blocks of 32) and packed formats
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32) * np.exp2(rng.integers(-6, 6, (rows, 1)))
    x[0, :32] = 1e-7  # a block below the amax clamp
    x[1, :32] = np.array([0, 0.25, 0.75, 1.25, 2.5, 3.5, 5, 6] * 4, np.float32)  # e2m1 ties at scale 1
    xb = O.round_to(x.astype(np.float32), "bfloat16")
    out = {"x": x, "xb": xb}
    for tag, arr, dt in (("f32", x, "float32"), ("bf16", xb, "bfloat16")):
        out[f"sim8_{tag}"] = O.act_quant_simulate(arr, dt, 128)
        out[f"sim4_{tag}"] = O.fp4_act_quant_simulate(arr, dt, 32)
        v8, s8 = O.fp8_pack(arr, 128)
        v8p, s8p = O.fp8_pack(arr, 128, pow2=True)
        v4, s4 = O.fp4_pack(arr, 32)
        out.update({f"v8_{tag}": v8, f"s8_{tag}": s8, f"v8p_{tag}": v8p, f"s8p_{tag}": s8p, f"v4_{tag}": v4,
                    f"s4_{tag}": s4})
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)


def csa_rows_case(name, S, T, m, top_k, n_win, n_comp_hca, m_prime, seed):
    # index rows of build_csa_topk_idxs (from a score matrix with ties and -inf) and build_hca_topk_idxs
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal((S, T)).astype(np.float32)
    scores[:, 3] = scores[:, 5]  # exact ties
    scores[S // 2, :T // 2] = -np.inf  # legal entries that may never be picked
    rows = np.arange(S)
    csa = O.csa_scores_topk_rows(scores, rows, m, top_k, n_win, S).astype(np.int32)
    hca = O.hca_idx_rows(rows, n_win, n_comp_hca, m_prime, S).astype(np.int32)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), scores=scores, m=m, top_k=top_k, n_win=n_win,
                        n_comp_hca=n_comp_hca, m_prime=m_prime, csa=csa, hca=hca)


def main():
    indexer_case("indexer_v4_causal", S=16, H=64, D=128, T=8, top_k=4, ratio=2, seed=1)
    indexer_case("indexer_small_unmasked", S=40, H=16, D=32, T=70, top_k=12, ratio=None, seed=2, scale=0.5)
    indexer_case("indexer_ties", S=24, H=16, D=64, T=48, top_k=20, ratio=None, seed=3, tie_rows=16)
    attn_case("attn_d576", S=3, H=16, D=576, N=40, K=24, seed=4)
    attn_case("attn_d64", S=10, H=16, D=64, N=32, K=20, seed=5)
    attn_bwd_case("attn_bwd_d64", S=6, H=16, D=64, N=24, K=16, seed=6)
    attn_bwd_case("attn_bwd_d576", S=3, H=16, D=576, N=40, K=40, seed=7)
    quant_case("quant_blocks", rows=4, cols=256, seed=8)
    csa_rows_case("csa_rows", S=40, T=12, m=4, top_k=6, n_win=5, n_comp_hca=9, m_prime=4, seed=9)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
