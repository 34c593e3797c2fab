"""GPU parity of the head-split top-k kernel (indexer_topk_split.h) against
the CPU oracle: the shapes past one wave's registers or the four-row LDS
budget -- H_I up to 256 at every head dim, top_k up to 4096.

The reference accepts any power-of-two H_I >= 16 and D_I
(flash_sparse/triton/indexer_score.py:145-150) and any top_k
(flash_sparse/triton/chunked_indexer.py:47-57); its tests use H_I <= 64 and
top_k <= 512 (tests/test_chunked_indexer.py:17-72), so these cases extend its
own with the same gate (tests/indexer_check.py): exact valid counts and
padding, sorted output with index-ascending ties, scores within 1e-4 of the
oracle, exact index sets wherever the k-th boundary gap is wide.  Which
kernel runs is asserted through si_indexer_topk_plan.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import _lib, chunked_indexer_topk, indexer_score, synth
from streamindex_amd.csa import csa_topk_idxs
from tests.conftest import bf16_bits
from tests.indexer_check import check_indexer

pytestmark = pytest.mark.gpu

SPLIT = 3


def _kernel(S, T, H, D, top_k, ratio=None):
    kern, cap = ctypes.c_int32(), ctypes.c_int32()
    rc = _lib.load().si_indexer_topk_plan(S, T, H, D, top_k, ratio or 0, ctypes.byref(kern), ctypes.byref(cap))
    assert rc == 0
    return kern.value


def _inputs(B, S, H, D, T, seed, wdtype=torch.float32):
    return synth.indexer_inputs(B, S, H, D, T, seed=seed, weights_dtype=wdtype)


@pytest.mark.parametrize("H,D,top_k,ratio", [
    (256, 128, 512, 4),     # 256 heads, V4 dims otherwise
    (256, 128, 2048, None),
    (192, 64, 700, None),
    (160, 32, 100, 2),
    (256, 32, 1152, None),
    (256, 64, 1153, None),  # capacity 4608 below 2048
    (96, 256, 512, None),   # D_I = 256: two waves of 64 heads
    (128, 256, 1000, 4),
    (256, 256, 300, None),  # four waves of 64 heads
    (200, 256, 1536, None),
])
def test_many_heads(cuda_device, H, D, top_k, ratio):
    S = 64
    T = 2600 if ratio is None else S // ratio
    assert _kernel(S, T, H, D, top_k, ratio) == SPLIT
    q, k, w = _inputs(1, S, H, D, T, 11 + H + D + top_k)
    idx, sc = chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio)
    torch.cuda.synchronize()
    check_indexer(q, k, w, top_k, idx, sc, causal_ratio=ratio, label=f"H={H},D={D},k={top_k}")


@pytest.mark.parametrize("H,D,top_k", [(64, 128, 4096), (64, 128, 2049), (16, 32, 3000), (128, 64, 4096),
                                       (48, 256, 2500), (64, 256, 4096), (256, 128, 4096)])
def test_large_topk(cuda_device, H, D, top_k):
    S, T = 48, 6000
    assert _kernel(S, T, H, D, top_k) == SPLIT
    q, k, w = _inputs(1, S, H, D, T, 21 + H + D + top_k)
    idx, sc = chunked_indexer_topk(q, k, w, top_k)
    torch.cuda.synchronize()
    check_indexer(q, k, w, top_k, idx, sc, label=f"H={H},D={D},k={top_k}")


def test_large_topk_causal_v4_dims(cuda_device):
    # V4-Flash dims with top_k = 4096 over causal rows: rows shorter than
    # top_k pad with -1 / -inf, longer rows select exactly
    S = 4096 * 4 + 512
    rows = np.r_[np.arange(0, 40), np.arange(S - 40, S), np.arange(16380, 16400)]
    q, k, w = _inputs(1, S, 64, 128, None, 31)
    idx, sc = chunked_indexer_topk(q, k, w, 4096, causal_ratio=4)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 4096, idx, sc, causal_ratio=4, rows=rows, label="k=4096 causal")


@pytest.mark.parametrize("top_k,T", [(4096, 9000), (2500, 6000)])
def test_large_topk_rising_scores(cuda_device, top_k, T):
    # every key beats the floor: a compaction every tile once the buffer is full
    B, S, H, D = 1, 8, 16, 32
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    q[..., 0] = 1.0
    k = torch.zeros(B, T, D, dtype=torch.bfloat16)
    k[0, :, 0] = torch.linspace(0.01, 8.0, T).to(torch.bfloat16)
    w = torch.ones(B, S, H, dtype=torch.float32)
    q, k, w = q.cuda(), k.cuda(), w.cuda()
    idx, sc = chunked_indexer_topk(q, k, w, top_k)
    torch.cuda.synchronize()
    check_indexer(q, k, w, top_k, idx, sc, label=f"rising k={top_k}")


def test_exact_ties_many_heads(cuda_device):
    # 8 distinct key rows repeated: every score ties in groups of T/8; the
    # order is (score desc, index asc) across the 4096-key merge too
    B, S, H, D, T = 1, 16, 192, 64, 4800
    g = torch.Generator().manual_seed(5)
    base = torch.randn(8, D, generator=g).to(torch.bfloat16)
    k = base.repeat(T // 8, 1).unsqueeze(0)
    q = torch.randn(B, S, H, D, generator=g).to(torch.bfloat16)
    w = torch.randn(B, S, H, generator=g)
    q, k, w = q.cuda(), k.cuda(), w.cuda()
    for K in (100, 3000):
        idx, sc = chunked_indexer_topk(q, k, w, K)
        torch.cuda.synchronize()
        ref = O.indexer_scores(bf16_bits(q[0]), bf16_bits(k[0]), w[0].cpu().numpy(), np.arange(S))
        ridx, _ = O.topk(ref, np.full(S, T, dtype=np.int64), K)
        assert np.array_equal(idx[0].cpu().numpy(), ridx), f"K={K}"
        check_indexer(q, k, w, K, idx, sc, label=f"ties K={K}")


def test_mask_batch_bf16_weights_short_keys(cuda_device):
    # explicit bool mask, batch 2, bf16 weights, T < 64 and T < top_k
    for (T, K) in ((37, 3000), (900, 2100)):
        q, k, w = _inputs(2, 40, 224, 64, T, 41 + T, wdtype=torch.bfloat16)
        mask = (torch.rand(2, 40, T, generator=torch.Generator().manual_seed(T)) < 0.6).cuda()
        mask[1, 3] = False
        idx, sc = chunked_indexer_topk(q, k, w, K, causal_mask=mask)
        torch.cuda.synchronize()
        check_indexer(q, k, w, K, idx, sc, mask=mask, label=f"mask T={T}")
        assert bool((idx[1, 3] == -1).all())


def test_csa_rows_many_heads(cuda_device):
    # CSA index rows from the head-split kernel: window columns, then picks + S
    S, H, D, m, n_win, K = 512, 256, 128, 4, 64, 100
    q, k, w = _inputs(1, S, H, D, None, 51)
    rows = csa_topk_idxs(q, k, w, n_win=n_win, top_k=K, m=m)
    idx, sc = chunked_indexer_topk(q, k, w, K, causal_ratio=m)
    torch.cuda.synchronize()
    r = rows[0].cpu().numpy()
    win = np.array([[t if t >= 0 else -1 for t in range(s - n_win + 1, s + 1)] for s in range(S)])
    assert np.array_equal(r[:, :n_win], win)
    picks = r[:, n_win:].astype(np.int64)
    assert np.array_equal(np.where(picks >= 0, picks - S, -1), idx[0].cpu().numpy())
    check_indexer(q, k, w, K, idx, sc, causal_ratio=m, rows=np.arange(0, S, 7), label="csa H=256")


@pytest.mark.parametrize("H,D", [(256, 128), (160, 64), (128, 256), (256, 256)])
def test_score_matrix_many_heads(cuda_device, H, D):
    # the materialised scores run one launch per head group, later ones adding
    q, k, w = _inputs(1, 24, H, D, 333, 61 + H)
    s = indexer_score(q, k, w)
    torch.cuda.synchronize()
    ref = O.indexer_scores(bf16_bits(q[0]), bf16_bits(k[0]), w[0].cpu().numpy())
    got = s[0].cpu().double().numpy()
    assert np.abs(got - ref).max() <= 1e-4 * (np.abs(ref).max() + np.abs(ref).mean())
