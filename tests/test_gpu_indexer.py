"""GPU parity of the fused indexer top-k / score kernels against the CPU oracle.

Cases mirror the reference's own tests and harness
(tests/test_chunked_indexer.py:17-72, tests/test_triton_indexer_score.py:25-92,
eval/test_v4_indexer_parity.py:205-289) plus the edge cases the reference
handles implicitly (T < top_k, rows with no legal key, explicit bool mask,
exact score ties, batch > 1, bf16 weights).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import chunked_indexer_topk, indexer_score, indexer_score_topk, synth
from tests.conftest import bf16_bits
from tests.indexer_check import check_indexer

pytestmark = pytest.mark.gpu


def _inputs(B, S, H, D, T, seed, scale=None, dev="cuda", wdtype=torch.float32):
    return synth.indexer_inputs(B, S, H, D, T, seed=seed, device=dev, q_scale=scale, k_scale=scale,
                                weights_dtype=wdtype)


def test_reference_small_unmasked(cuda_device):
    # tests/test_chunked_indexer.py:18-47 shape: S=64, H=16, D=32, T=256, K=32, chunks 16/64
    q, k, w = _inputs(1, 64, 16, 32, 256, 900, scale=0.5)
    idx, sc = chunked_indexer_topk(q, k, w, top_k=32, chunk_s=16, chunk_t=64)
    torch.cuda.synchronize()
    assert idx.shape == (1, 64, 32) and idx.dtype == torch.int64
    assert sc.shape == (1, 64, 32) and sc.dtype == torch.float32
    check_indexer(q, k, w, 32, idx, sc, label="small")


def test_reference_unaligned(cuda_device):
    # tests/test_chunked_indexer.py:51-72: S=47, T=73, K=16, chunks 10/20
    q, k, w = _inputs(1, 47, 16, 32, 73, 901, scale=0.5)
    idx, sc = chunked_indexer_topk(q, k, w, top_k=16, chunk_s=10, chunk_t=20)
    torch.cuda.synchronize()
    assert idx.shape == (1, 47, 16)
    valid = idx >= 0
    assert bool((idx[valid] < 73).all())
    check_indexer(q, k, w, 16, idx, sc, label="unaligned")


@pytest.mark.parametrize("S", [2048, 4096])
def test_v4_flash_causal(cuda_device, S):
    # eval/test_v4_indexer_parity.py dims: H=64, D=128, k=512, ratio 4, chunks 2048/8192
    q, k, w = _inputs(1, S, 64, 128, None, 2026)
    idx, sc = chunked_indexer_topk(q, k, w, 512, causal_ratio=4, chunk_s=2048, chunk_t=8192)
    torch.cuda.synchronize()
    st = check_indexer(q, k, w, 512, idx, sc, causal_ratio=4, label=f"v4flash S={S}")
    assert st[0]["recall_mean"] >= 0.999
    # rows s < ratio-1 have no legal key at all
    assert bool((idx[0, :3] == -1).all()) and bool(torch.isneginf(sc[0, :3]).all())


def test_t_smaller_than_topk(cuda_device):
    q, k, w = _inputs(1, 256, 64, 128, None, 31)  # T = 64 < top_k = 512
    idx, sc = chunked_indexer_topk(q, k, w, 512, causal_ratio=4)
    torch.cuda.synchronize()
    assert idx.shape == (1, 256, 512)
    check_indexer(q, k, w, 512, idx, sc, causal_ratio=4, label="T<k")


@pytest.mark.parametrize("H,D", [(16, 32), (16, 64), (32, 128), (48, 64), (64, 32), (64, 64), (64, 128),
                                 (80, 128), (96, 64), (128, 32), (128, 64), (128, 128), (16, 256), (64, 256)])
def test_head_shapes(cuda_device, H, D):
    q, k, w = _inputs(1, 128, H, D, 300, 40 + H + D)
    idx, sc = chunked_indexer_topk(q, k, w, 40)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 40, idx, sc, label=f"H={H},D={D}")


@pytest.mark.parametrize("H,D,top_k,ratio", [(128, 128, 512, 4), (128, 128, 1024, None), (128, 128, 2048, None),
                                             (64, 256, 512, 4), (64, 256, 1536, None), (100, 64, 700, 2)])
def test_wide_rows(cuda_device, H, D, top_k, ratio):
    """H_I up to 128 (one workgroup per CU) and D_I = 256 at several
    selection capacities, causal and not, through the oracle gate; the score
    matrix of the same shapes against the oracle."""
    S, T = 96, 2500 if ratio is None else 96 // ratio
    q, k, w = _inputs(1, S, H, D, T, 7 + H + D + top_k)
    idx, sc = chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio)
    torch.cuda.synchronize()
    check_indexer(q, k, w, top_k, idx, sc, causal_ratio=ratio, label=f"H={H},D={D},k={top_k}")
    s = indexer_score(q[:, :16], k, w[:, :16])
    torch.cuda.synchronize()
    ref = O.indexer_scores(bf16_bits(q[0, :16]), bf16_bits(k[0]), w[0, :16].cpu().numpy())
    assert np.allclose(s[0].cpu().numpy(), ref, rtol=1e-4, atol=1e-4 * np.abs(ref).mean())


@pytest.mark.parametrize("top_k", [1, 7, 64, 65, 100, 128, 129, 256, 257, 512, 513, 640, 641, 700, 1024, 1152,
                                   1153, 1536, 1537, 2048])
def test_topk_widths(cuda_device, top_k):
    q, k, w = _inputs(1, 96, 64, 128, 3000, 50 + top_k)
    idx, sc = chunked_indexer_topk(q, k, w, top_k)
    torch.cuda.synchronize()
    check_indexer(q, k, w, top_k, idx, sc, label=f"k={top_k}")


def test_long_rows_many_merges(cuda_device):
    # T = 20000 legal keys per row forces many candidate-buffer merges
    q, k, w = _inputs(1, 40, 64, 128, 20000, 61)
    idx, sc = chunked_indexer_topk(q, k, w, 512)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 512, idx, sc, label="long rows")


def test_increasing_scores_worst_case(cuda_device):
    # Scores that rise with t defeat the threshold filter (every key is a
    # candidate): exactness must not depend on the filter rate.
    B, S, H, D, T = 1, 16, 16, 32, 4096
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    q[..., 0] = 1.0
    k = torch.zeros(B, T, D, dtype=torch.bfloat16)
    k[0, :, 0] = torch.linspace(0.01, 8.0, T).to(torch.bfloat16)
    w = torch.ones(B, S, H, dtype=torch.float32)
    q, k, w = q.cuda(), k.cuda(), w.cuda()
    idx, sc = chunked_indexer_topk(q, k, w, 300)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 300, idx, sc, label="rising")


@pytest.mark.parametrize("top_k,T", [(1100, 6000), (700, 4096), (2000, 6000)])
def test_increasing_scores_wide_selections(cuda_device, top_k, T):
    # The rising-score worst case at the wide capacities (1536: two
    # workgroups per CU, 4096): a compaction every few tiles.
    B, S, H, D = 1, 12, 16, 32
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16)
    q[..., 0] = 1.0
    k = torch.zeros(B, T, D, dtype=torch.bfloat16)
    k[0, :, 0] = torch.linspace(0.01, 8.0, T).to(torch.bfloat16)
    w = torch.ones(B, S, H, dtype=torch.float32)
    q, k, w = q.cuda(), k.cuda(), w.cuda()
    idx, sc = chunked_indexer_topk(q, k, w, top_k)
    torch.cuda.synchronize()
    check_indexer(q, k, w, top_k, idx, sc, label=f"rising k={top_k}")


def test_long_rows_v4_pro_topk(cuda_device):
    # top_k = 1024 (the V4-Pro setting) over 20000 legal keys, then a bool mask at top_k = 1000
    q, k, w = _inputs(1, 40, 64, 128, 20000, 62)
    idx, sc = chunked_indexer_topk(q, k, w, 1024)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 1024, idx, sc, label="long rows k=1024")
    q, k, w = _inputs(1, 64, 64, 128, 4096, 63)
    mask = torch.rand(1, 64, 4096, generator=torch.Generator().manual_seed(1)) < 0.7
    idx, sc = chunked_indexer_topk(q, k, w, 1000, causal_mask=mask.cuda())
    torch.cuda.synchronize()
    check_indexer(q, k, w, 1000, idx, sc, mask=mask.cuda(), label="masked k=1000")


def test_exact_ties_prefer_smaller_index(cuda_device):
    # 8 distinct key rows repeated: scores tie exactly in groups of 8.  The
    # order must be (score desc, index asc), docs/streaming_topk.md:301-312.
    B, S, H, D, T, K = 1, 32, 16, 64, 64, 20
    g = torch.Generator().manual_seed(5)
    base = torch.randn(8, D, generator=g).to(torch.bfloat16)
    k = base.repeat(T // 8, 1).unsqueeze(0)
    q = torch.randn(B, S, H, D, generator=g).to(torch.bfloat16)
    w = torch.randn(B, S, H, generator=g)
    q, k, w = q.cuda(), k.cuda(), w.cuda()
    idx, sc = chunked_indexer_topk(q, k, w, K)
    torch.cuda.synchronize()
    rows = np.arange(S)
    ref = O.indexer_scores(bf16_bits(q[0]), bf16_bits(k[0]), w[0].cpu().numpy(), rows)
    ridx, _ = O.topk(ref, np.full(S, T, dtype=np.int64), K)
    assert np.array_equal(idx[0].cpu().numpy(), ridx)
    check_indexer(q, k, w, K, idx, sc, label="ties")


def test_causal_mask_tensor(cuda_device):
    B, S, H, D, T = 2, 80, 32, 64, 200
    q, k, w = _inputs(B, S, H, D, T, 71)
    g = torch.Generator().manual_seed(72)
    mask = (torch.rand(B, S, T, generator=g) < 0.3)
    mask[0, 5] = False  # one row with no legal key
    mask = mask.cuda()
    idx, sc = chunked_indexer_topk(q, k, w, 48, causal_mask=mask, chunk_s=32, chunk_t=64)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 48, idx, sc, mask=mask, label="mask")
    assert bool((idx[0, 5] == -1).all())


def test_batch_and_bf16_weights(cuda_device):
    q, k, w = _inputs(3, 200, 64, 128, None, 81, wdtype=torch.bfloat16)
    idx, sc = chunked_indexer_topk(q, k, w, 32, causal_ratio=4)
    torch.cuda.synchronize()
    check_indexer(q, k, w, 32, idx, sc, causal_ratio=4, label="batch/bf16w")


def test_strided_inputs(cuda_device):
    # non-contiguous q (a slice along S with stride) and k_idx (slice along T)
    q0, k0, w0 = _inputs(1, 160, 64, 128, 400, 91)
    q, k, w = q0[:, ::2], k0[:, 100:300], w0[:, ::2]
    idx, sc = chunked_indexer_topk(q, k, w, 64, causal_ratio=2)
    torch.cuda.synchronize()
    check_indexer(q.contiguous(), k.contiguous(), w.contiguous(), 64, idx, sc, causal_ratio=2, label="strided")


def test_indexer_score_matches_oracle(cuda_device):
    # tests/test_triton_indexer_score.py:25-60 shapes
    for (S, H, D, T, seed, scale) in [(64, 16, 64, 128, 300, 0.5), (32, 64, 128, 64, 301, 0.3), (70, 48, 32, 333, 302, 1.0)]:
        q, k, w = _inputs(1, S, H, D, T, seed, scale=scale)
        sc = indexer_score(q, k, w)
        torch.cuda.synchronize()
        assert sc.shape == (1, S, T) and sc.dtype == torch.float32
        ref = O.indexer_scores(bf16_bits(q[0]), bf16_bits(k[0]), w[0].cpu().numpy())
        got = sc[0].cpu().double().numpy()
        scale_ = np.abs(ref).mean() + 1e-30
        assert np.abs(got - ref).max() <= 1e-4 * (np.abs(ref).max() + scale_)


def test_indexer_score_topk_width(cuda_device):
    q, k, w = _inputs(1, 32, 16, 64, 64, 302)
    i1, v1 = indexer_score_topk(q, k, w, 16)
    i2, v2 = indexer_score_topk(q, k, w, 100)  # width min(k, T) = 64
    torch.cuda.synchronize()
    assert i1.shape == (1, 32, 16) and i2.shape == (1, 32, 64)
    check_indexer(q, k, w, 16, i1, v1, label="score_topk")
    check_indexer(q, k, w, 64, i2, v2, label="score_topk full")


def test_empty_and_degenerate(cuda_device):
    q, k, w = _inputs(1, 8, 16, 32, 0, 3)  # T = 0
    idx, sc = chunked_indexer_topk(q, k, w, 4, causal_ratio=4)
    torch.cuda.synchronize()
    assert bool((idx == -1).all()) and bool(torch.isneginf(sc).all())
    q, k, w = _inputs(1, 0, 16, 32, 16, 3)  # S = 0
    idx, sc = chunked_indexer_topk(q, k, w, 4)
    assert idx.shape == (1, 0, 4)


def test_invalid_arguments_raise(cuda_device):
    q, k, w = _inputs(1, 16, 16, 32, 16, 3)
    with pytest.raises(AssertionError):
        chunked_indexer_topk(q, k[:, :, :16], w, 4)
    with pytest.raises(AssertionError):
        chunked_indexer_topk(q, k, w, 4, causal_mask=torch.ones(1, 16, 16, dtype=torch.bool, device="cuda"),
                             causal_ratio=4)
    with pytest.raises(ValueError):
        chunked_indexer_topk(q, k, w, 4097)
    with pytest.raises(ValueError):
        chunked_indexer_topk(q.float(), k, w, 4)
    with pytest.raises(ValueError):
        q5, k5, w5 = _inputs(1, 16, 16, 48, 16, 3)
        chunked_indexer_topk(q5, k5, w5, 4)
    # the head limit: H_I > 256
    for (H, D, kk) in ((257, 64, 4), (300, 256, 4)):
        qq, kk_, ww = _inputs(1, 8, H, D, 16, 4)
        with pytest.raises(ValueError):
            chunked_indexer_topk(qq, kk_, ww, kk)
