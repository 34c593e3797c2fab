"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every stored output exactly (indices) or to
float32 rounding (scores / attention outputs).
GPU: the HIP kernels reproduce the stored outputs — exact index lists for
the indexer (including the exact-tie case), 2e-2 for attention outputs.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
INDEXER = sorted(glob.glob(os.path.join(HERE, "indexer_*.npz")))
ATTN = sorted(glob.glob(os.path.join(HERE, "attn_*.npz")))


def _ratio(z):
    r = int(z["ratio"])
    return None if r < 0 else r


@pytest.mark.parametrize("path", INDEXER, ids=os.path.basename)
def test_oracle_reproduces_indexer_fixture(path):
    z = np.load(path)
    idx, val, _ = O.indexer_topk_rows(z["q"], z["k"], z["w"], int(z["top_k"]), causal_ratio=_ratio(z))
    assert np.array_equal(idx, z["idx"])
    assert np.array_equal(val, z["score"])


@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_oracle_reproduces_attn_fixture(path):
    z = np.load(path)
    o, lse = O.sparse_attn_rows(z["q"], z["kv"], z["sink"], z["idx"], float(z["scale"]))
    assert np.array_equal(o.astype(np.float32), z["o"])
    assert np.array_equal(lse.astype(np.float32), z["lse"])


def _t(bits, dev):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("path", INDEXER, ids=os.path.basename)
def test_gpu_matches_indexer_fixture(cuda_device, path):
    from streamindex_amd import chunked_indexer_topk

    z = np.load(path)
    q = _t(z["q"], cuda_device).unsqueeze(0)
    k = _t(z["k"], cuda_device).unsqueeze(0)
    w = torch.from_numpy(z["w"]).to(cuda_device).unsqueeze(0)
    idx, sc = chunked_indexer_topk(q, k, w, int(z["top_k"]), causal_ratio=_ratio(z))
    torch.cuda.synchronize()
    assert np.array_equal(idx[0].cpu().numpy(), z["idx"])
    ref = z["score"]
    got = sc[0].cpu().numpy().astype(np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(fin, np.isfinite(got))
    assert np.abs(got[fin] - ref[fin]).max() <= 1e-4 * (np.abs(ref[fin]).max() + 1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_gpu_matches_attn_fixture(cuda_device, path):
    from streamindex_amd import sparse_attn_fwd

    z = np.load(path)
    q = _t(z["q"], cuda_device).unsqueeze(0)
    kv = _t(z["kv"], cuda_device).unsqueeze(0)
    sink = torch.from_numpy(z["sink"]).to(cuda_device)
    idx = torch.from_numpy(z["idx"]).to(cuda_device).unsqueeze(0)
    o, lse = sparse_attn_fwd(q, kv, sink, idx, float(z["scale"]))
    torch.cuda.synchronize()
    assert np.abs(o[0].float().cpu().numpy() - z["o"]).max() <= 2e-2
    assert np.abs(lse[0].cpu().numpy() - z["lse"]).max() <= 2e-3 * max(1.0, np.abs(z["lse"]).max())
