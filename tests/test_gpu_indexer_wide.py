"""The two bf16 top-k kernels agree bit for bit, and the four-M-block one
matches the oracle.

si_indexer_topk runs indexer_topk_kernel (two workgroups per CU, one query
row per wave) or, for D_I = 128 with H_I in (96, 128], or H_I in (32, 64]
and rows of at least 64K legal keys, indexer_topk_wide_kernel (one wave per
SIMD holding four 32-head blocks: two query rows, or one row of up to 128
heads).  The
runtime switch si_indexer_set_topk_kernel forces either one, so the wide
kernel is exercised here at sizes the oracle checks in seconds: every case
compares the two kernels' indices and scores for exact equality (same fp32
operation order, same exact selection) and a subset also goes through the
oracle gate of tests/indexer_check.py.  Shapes cover the wide kernel's
parts: partial head blocks, both selection capacities it uses (1024 for
top_k <= 192, 1536 / 2048 above), tiles crossing T, T < 64 and T < top_k,
the explicit mask, batch 2, S not a multiple of its 8-row workgroup, bf16
weights, exact score ties, rows long enough for repeated compactions, the
CSA output rows, and config[2] in full.
"""

from __future__ import annotations

import pytest
import torch

from streamindex_amd import _lib, chunked_indexer_topk, synth
from streamindex_amd.csa import csa_topk_idxs
from tests.indexer_check import check_indexer

pytestmark = pytest.mark.gpu

AUTO, NARROW, WIDE = 0, 1, 2


def _set_mode(mode: int) -> int:
    prev = _lib.load().si_indexer_set_topk_kernel(mode)
    assert prev >= 0
    return prev


@pytest.fixture
def modes(cuda_device):
    yield
    _set_mode(AUTO)


def _both(fn):
    """fn() under the narrow and the wide kernel; returns (narrow, wide)."""
    _set_mode(NARROW)
    a = fn()
    _set_mode(WIDE)
    b = fn()
    _set_mode(AUTO)
    torch.cuda.synchronize()
    return a, b


def _same(a, b, label):
    for x, y, name in zip(a, b, ("indices", "scores")):
        assert torch.equal(x, y), f"{label}: {name} differ between the two kernels"


def _inputs(B, S, H, T, seed, wdtype=torch.float32, scale=None):
    return synth.indexer_inputs(B, S, H, 128, T, seed=seed, q_scale=scale, k_scale=scale, weights_dtype=wdtype)


@pytest.mark.parametrize("S,H,top_k,oracle", [
    (2048, 64, 512, True),    # V4-Flash dims, capacity 1536
    (4096, 64, 512, False),
    (4096, 64, 192, True),    # capacity 1024
    (2048, 64, 1, False),
    (2048, 64, 64, False),
    (2048, 64, 193, False),
    (4096, 64, 640, False),
    (4096, 64, 1024, True),
    (4096, 64, 1152, False),  # the largest top_k the wide kernel serves at H_I <= 64
    (2048, 48, 512, True),    # partial head block
    (2048, 40, 100, False),
    (2048, 128, 512, True),   # one 128-head row per wave, capacity 2048
    (2048, 100, 512, False),
    (2048, 128, 1152, False),
])
def test_causal_kernels_agree(modes, S, H, top_k, oracle):
    q, k, w = _inputs(1, S, H, None, 3000 + S + H + top_k)
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, top_k, causal_ratio=4))
    _same(a, b, f"S={S} H={H} k={top_k}")
    if oracle:
        check_indexer(q, k, w, top_k, b[0], b[1], causal_ratio=4, label=f"wide S={S} H={H} k={top_k}")


@pytest.mark.parametrize("S,T,top_k", [(256, 1000, 512), (100, 37, 16), (64, 63, 100), (300, 4097, 256),
                                       (515, 2000, 700)])
def test_unbounded_rows_and_tail_tiles(modes, S, T, top_k):
    q, k, w = _inputs(1, S, 64, T, 4000 + S + T)
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, top_k))
    _same(a, b, f"S={S} T={T}")
    check_indexer(q, k, w, top_k, b[0], b[1], label=f"wide S={S} T={T} k={top_k}")


def test_batch_mask_and_bf16_weights(modes):
    B, S, T = 2, 515, 900
    q, k, w = _inputs(B, S, 64, T, 4100, wdtype=torch.bfloat16)
    g = torch.Generator().manual_seed(7)
    mask = (torch.rand(B, S, T, generator=g) < 0.6).cuda()
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, 300, causal_mask=mask))
    _same(a, b, "mask")
    check_indexer(q, k, w, 300, b[0], b[1], mask=mask, label="wide mask bf16-w")
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, 300, causal_ratio=2))
    _same(a, b, "batch 2 causal")


def test_exact_ties_rank_smaller_index_first(modes):
    q, k, w = _inputs(1, 1024, 64, 2000, 4200)
    q.zero_()  # every score is exactly 0
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, 512))
    _same(a, b, "ties")
    expect = torch.arange(512, device=q.device).expand(1, 1024, 512)
    assert torch.equal(b[0], expect)


def test_long_rows_compact_repeatedly(modes):
    # 16K keys per row: a selection buffer of 1536 compacts many times per row
    q, k, w = _inputs(1, 64, 64, 16384, 4300)
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, 512))
    _same(a, b, "long rows")
    check_indexer(q, k, w, 512, b[0], b[1], label="wide long rows")


def test_csa_rows_agree(modes):
    S, m, n_win, top_k = 4096, 4, 128, 512
    qi, ki, w = synth.indexer_inputs(1, S, 64, 128, S // m, seed=4400)
    a, b = _both(lambda: csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m, return_scores=True))
    _same(a, b, "csa rows")


def test_auto_picks_by_row_length(modes):
    # the automatic choice gives the same result as either forced kernel
    q, k, w = _inputs(1, 2048, 64, None, 4500)
    _set_mode(AUTO)
    auto = chunked_indexer_topk(q, k, w, 512, causal_ratio=4)
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, 512, causal_ratio=4))
    _same(auto, a, "auto vs narrow")
    _same(auto, b, "auto vs wide")


@pytest.mark.parametrize("top_k,zero_q", [(100, False), (512, False), (1100, False), (512, True)])
def test_mass_ties_through_compactions(modes, top_k, zero_q):
    # 6,000 keys made of 7 distinct rows repeated: every score is shared by ~857
    # keys, so a compaction's count on the score word jumps by hundreds, past
    # every window, and the 64-bit (score, index) bisection sets the floor; with q = 0 every score is
    # +0 and the picks are the top_k smallest indices.  Both kernels, against
    # the oracle's (score desc, index asc) order.
    import numpy as np

    from oracle import oracle as O
    from tests.conftest import bf16_bits

    S, H, D, T = 24, 64, 128, 6000
    g = torch.Generator().manual_seed(777 + top_k)
    base = torch.randn(7, D, generator=g).to(torch.bfloat16)
    k = base.repeat(T // 7 + 1, 1)[:T].unsqueeze(0).cuda()
    q = torch.randn(1, S, H, D, generator=g).to(torch.bfloat16)
    if zero_q:
        q.zero_()
    q = q.cuda()
    w = torch.randn(1, S, H, generator=g).cuda()
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, top_k))
    _same(a, b, f"mass ties k={top_k}")
    ref = O.indexer_scores(bf16_bits(q[0]), bf16_bits(k[0]), w[0].cpu().numpy(), np.arange(S))
    ridx, _ = O.topk(ref, np.full(S, T, dtype=np.int64), top_k)
    assert np.array_equal(a[0][0].cpu().numpy(), ridx)
    if zero_q:
        assert np.array_equal(ridx, np.tile(np.arange(top_k), (S, 1)))


def test_config2_full_size_kernels_agree(modes):
    # BASELINE config[2] (S=262,144, T=65,536, k=512): the automatic choice runs the
    # four-M-block kernel here; the two kernels agree on every one of the 134M outputs.
    q, k, w = synth.indexer_inputs(1, 262144, 64, 128, ratio=4, seed=2026)
    a, b = _both(lambda: chunked_indexer_topk(q, k, w, 512, causal_ratio=4))
    _same(a, b, "config[2]")
    _set_mode(AUTO)
    auto = chunked_indexer_topk(q, k, w, 512, causal_ratio=4)
    torch.cuda.synchronize()
    _same(auto, b, "config[2] auto")
