"""GPU parity of the CSA / HCA composition against the CPU oracle.

Cases mirror the reference's own tests (tests/test_csa_correctness.py:25-181,
tests/test_hca_correctness.py:25-60) at their shapes, plus the V4-Flash shape
(64 heads, d = 576, H_I = 64, D_I = 128, n_win = 128, top_k = 512) and the
edges the reference handles implicitly (n_win > S, T < top_k, rows with no
legal compressed entry, batch > 1, -inf scores).

Gates: window / HCA index rows bit-exact; compressed picks through the same
indexer gate as chunked_indexer_topk (tests/indexer_check.py); index rows from
a materialised score matrix bit-exact against the oracle's selection over the
same fp32 scores; attention output |o - o_ref| <= 2e-2 against the oracle
attention over the same index rows, and the reference's own correlation
metric < 5e-3 (tests/test_csa_correctness.py:16-22,75).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import (build_csa_topk_idxs, build_hca_topk_idxs, csa_topk_idxs, flash_csa_forward,
                             flash_hca_forward, indexer_score, synth)
from streamindex_amd.csa import build_sliding_window_idxs
from tests.conftest import bf16_bits
from tests.indexer_check import check_rows

pytestmark = pytest.mark.gpu


def _norm_corr(a: torch.Tensor, b: torch.Tensor) -> float:
    # tests/test_csa_correctness.py:16-22
    a32 = a.detach().float().reshape(-1)
    b32 = b.detach().float().reshape(-1)
    denom = (a32 * a32 + b32 * b32).sum()
    if denom.item() == 0.0:
        return 0.0
    return float((1.0 - 2.0 * (a32 * b32).sum() / denom).item())


def _csa_inputs(B, S, n_h, d, n_I_h, c_I, m, seed, scale=0.5, idx_scale=None):
    g = torch.Generator().manual_seed(seed)
    T = S // m
    isc = scale if idx_scale is None else idx_scale
    q = torch.randn(B, S, n_h, d, generator=g, dtype=torch.bfloat16) * scale
    kv = torch.randn(B, S, d, generator=g, dtype=torch.bfloat16) * scale
    kvc = torch.randn(B, T, d, generator=g, dtype=torch.bfloat16) * scale
    qi = torch.randn(B, S, n_I_h, c_I, generator=g, dtype=torch.bfloat16) * isc
    ki = torch.randn(B, T, c_I, generator=g, dtype=torch.bfloat16) * isc
    w = torch.randn(B, S, n_I_h, generator=g, dtype=torch.float32)
    sink = torch.randn(n_h, generator=g, dtype=torch.float32)
    return [t.cuda() for t in (q, kv, kvc, qi, ki, w, sink)]


def _check_csa_rows(rows_gpu, scores_gpu, qi, ki, w, m, n_win, top_k, S, rows=None, label=""):
    """Window columns exact; compressed columns through the indexer gate."""
    B = qi.shape[0]
    T = ki.shape[1]
    rows = np.arange(S, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
    got = rows_gpu.cpu().numpy()
    gv = scores_gpu.cpu().numpy()
    for b in range(B):
        g = got[b][rows]
        assert np.array_equal(g[:, :n_win], O.window_idxs(rows, n_win)), f"{label}: window columns"
        comp = g[:, n_win:].astype(np.int64)
        valid = comp >= 0
        assert np.all(comp[valid] >= S) and np.all(comp[valid] < S + T), f"{label}: offset"
        comp = np.where(valid, comp - S, -1)
        sc = O.indexer_scores(bf16_bits(qi[b]), bf16_bits(ki[b]), w[b].float().cpu().numpy(), rows)
        check_rows(sc, O.legal_limits(rows, T, m), top_k, comp, gv[b][rows], label=f"{label}[b={b}]")


def _oracle_attn(q, kv_full, sink, idx_rows, scale, rows):
    o_ref = []
    lse_ref = []
    for b in range(q.shape[0]):
        o, l = O.sparse_attn_rows(bf16_bits(q[b][torch.as_tensor(rows, device=q.device)]), bf16_bits(kv_full[b]),
                                  sink.cpu().numpy(), idx_rows[b][rows].astype(np.int64), scale)
        o_ref.append(o)
        lse_ref.append(l)
    return np.stack(o_ref), np.stack(lse_ref)


@pytest.mark.parametrize("S,n_win", [(1, 1), (64, 16), (300, 128), (100, 0), (5000, 128)])
def test_window_builder_exact(cuda_device, S, n_win):
    got = build_sliding_window_idxs(2, S, n_win, cuda_device)
    assert got.dtype == torch.int64 and got.shape == (2, S, n_win)
    ref = O.window_idxs(np.arange(S), n_win)
    g = got.cpu().numpy()
    assert np.array_equal(g[0], ref) and np.array_equal(g[1], ref)


@pytest.mark.parametrize("B,S,n_win,mp", [(1, 64, 16, 8), (2, 32, 8, 4), (1, 4096, 128, 128), (1, 17, 0, 3),
                                          (1, 9, 4, 1)])
def test_hca_idxs_exact(cuda_device, B, S, n_win, mp):
    n_comp = S // mp
    got = build_hca_topk_idxs(B=B, seq_len=S, n_win=n_win, n_compressed=n_comp, m_prime=mp, device=cuda_device)
    assert got.dtype == torch.int32 and got.shape == (B, S, n_win + n_comp)
    ref = O.hca_idx_rows(np.arange(S), n_win, n_comp, mp, S)
    for b in range(B):
        assert np.array_equal(got[b].cpu().numpy(), ref)


@pytest.mark.parametrize("B,S,n_I_h,c_I,m,n_win,top_k", [
    (1, 64, 16, 32, 4, 16, 8),      # tests/test_csa_correctness.py:29-31
    (1, 32, 64, 64, 4, 16, 8),      # :84-86 (V4-Pro indexer dims)
    (2, 200, 16, 32, 4, 8, 64),     # T < top_k: every row padded, batch 2
    (1, 2048, 64, 128, 4, 128, 512),  # V4-Flash
])
def test_fused_csa_rows_match_oracle(cuda_device, B, S, n_I_h, c_I, m, n_win, top_k):
    _, _, _, qi, ki, w, _ = _csa_inputs(B, S, 4, 32, n_I_h, c_I, m, seed=S + top_k,
                                        idx_scale=c_I ** -0.5)
    rows_gpu, sc = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m, return_scores=True)
    torch.cuda.synchronize()
    assert rows_gpu.dtype == torch.int32 and rows_gpu.shape == (B, S, n_win + top_k)
    # rows s < m-1 have no legal compressed entry
    assert bool((rows_gpu[:, : m - 1, n_win:] == -1).all())
    _check_csa_rows(rows_gpu, sc, qi, ki, w, m, n_win, top_k, S, label=f"fused S={S}")
    # without the score output the index rows are identical
    rows2 = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m)
    assert torch.equal(rows2, rows_gpu)


@pytest.mark.parametrize("S,m,n_win,top_k", [(64, 4, 16, 8), (47, 4, 5, 16), (1024, 4, 128, 512), (300, 2, 8, 2048)])
def test_build_csa_topk_idxs_from_scores_exact(cuda_device, S, m, n_win, top_k):
    T = S // m
    qi, ki, w = synth.indexer_inputs(1, S, 16, 32, T, seed=S, device=cuda_device)
    scores = indexer_score(qi, ki, w)
    if S == 47:
        scores[0, :, 2] = float("-inf")  # legal -inf scores are never picked
    got = build_csa_topk_idxs(scores, n_win, top_k, seq_len=S, n_compressed=T, m=m, device=cuda_device)
    torch.cuda.synchronize()
    assert got.dtype == torch.int32 and got.shape == (1, S, n_win + top_k)
    ref = O.csa_scores_topk_rows(scores[0].cpu().double().numpy(), np.arange(S), m, top_k, n_win, S)
    assert np.array_equal(got[0].cpu().numpy(), ref)


def test_build_csa_topk_idxs_ties_rank_smaller_index_first(cuda_device):
    S, m, n_win, top_k = 256, 2, 4, 16
    T = S // m
    scores = torch.zeros(2, S, T, device=cuda_device)
    scores[:, :, ::3] = 1.0
    got = build_csa_topk_idxs(scores, n_win, top_k, seq_len=S, n_compressed=T, m=m, device=cuda_device)
    ref = O.csa_scores_topk_rows(scores[0].cpu().double().numpy(), np.arange(S), m, top_k, n_win, S)
    for b in range(2):
        assert np.array_equal(got[b].cpu().numpy(), ref)


@pytest.mark.parametrize("B,S,n_h,d,n_I_h,c_I,m,n_win,top_k,seed", [
    (1, 64, 16, 64, 16, 32, 4, 16, 8, 400),     # tests/test_csa_correctness.py:26-75
    (1, 32, 128, 64, 64, 64, 4, 16, 8, 401),    # :79-125 (V4-Pro head count)
    (2, 96, 16, 128, 16, 32, 4, 200, 8, 402),   # n_win > S, batch 2
])
def test_flash_csa_forward_matches_oracle(cuda_device, B, S, n_h, d, n_I_h, c_I, m, n_win, top_k, seed):
    q, kv, kvc, qi, ki, w, sink = _csa_inputs(B, S, n_h, d, n_I_h, c_I, m, seed)
    o = flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=n_win, top_k=top_k, m=m)
    rows_gpu, sc = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m, return_scores=True)
    torch.cuda.synchronize()
    assert o.shape == (B, S, n_h, d) and o.dtype == torch.bfloat16
    _check_csa_rows(rows_gpu, sc, qi, ki, w, m, n_win, top_k, S, label="csa")
    rows = np.arange(S)
    kv_full = torch.cat([kv, kvc], dim=1)
    o_ref, _ = _oracle_attn(q, kv_full, sink, rows_gpu.cpu().numpy(), d ** -0.5, rows)
    err = np.abs(o.float().cpu().numpy() - o_ref).max()
    assert err <= 2e-2, f"max |o - o_ref| = {err}"
    assert _norm_corr(o.cpu(), torch.from_numpy(o_ref)) < 5e-3


def test_flash_csa_forward_v4_flash_shape(cuda_device):
    # V4-Flash: 64 heads, d = 576, indexer H_I = 64, D_I = 128, n_win = 128, top_k = 512
    B, S, n_h, d, m, n_win, top_k = 1, 4096, 64, 576, 4, 128, 512
    q, kv, kvc, qi, ki, w, sink = _csa_inputs(B, S, n_h, d, 64, 128, m, seed=404, scale=1.0, idx_scale=128 ** -0.5)
    o = flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=n_win, top_k=top_k, m=m)
    rows_gpu = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(7).choice(S, 48, replace=False))
    rows = np.concatenate([[0, 1, 2, 3, 127, 128], rows, [S - 1]])
    o_ref, _ = _oracle_attn(q, torch.cat([kv, kvc], dim=1), sink, rows_gpu.cpu().numpy(), d ** -0.5, rows)
    got = o[0][torch.as_tensor(rows, device=o.device)].float().cpu().numpy()
    err = np.abs(got - o_ref[0]).max()
    assert err <= 2e-2, f"max |o - o_ref| = {err}"


def test_flash_csa_chunk_arguments_do_not_change_the_result(cuda_device):
    # tests/test_csa_correctness.py:128-181: chunked and unchunked paths agree
    q, kv, kvc, qi, ki, w, sink = _csa_inputs(1, 64, 16, 64, 16, 32, 4, seed=403)
    a = flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=16, top_k=8, m=4, use_chunked_indexer=False)
    b = flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=16, top_k=8, m=4, use_chunked_indexer=True,
                          chunk_s=16, chunk_t=8)
    c = flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=16, top_k=8, m=4, use_triton=False)
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("B,S,n_h,d,mp,n_win,seed", [
    (1, 64, 16, 64, 8, 16, 500),     # tests/test_hca_correctness.py:26-60
    (2, 32, 16, 64, 4, 8, 501),      # :64-80 shapes
    (1, 2048, 64, 576, 128, 128, 502),  # V4 HCA ratio and window at d = 576
])
def test_flash_hca_forward_matches_oracle(cuda_device, B, S, n_h, d, mp, n_win, seed):
    g = torch.Generator().manual_seed(seed)
    nc = S // mp
    q = (torch.randn(B, S, n_h, d, generator=g, dtype=torch.bfloat16) * 0.5).cuda()
    kv = (torch.randn(B, S, d, generator=g, dtype=torch.bfloat16) * 0.5).cuda()
    kvc = (torch.randn(B, nc, d, generator=g, dtype=torch.bfloat16) * 0.5).cuda()
    sink = torch.randn(n_h, generator=g, dtype=torch.float32).cuda()
    o = flash_hca_forward(q, kv, kvc, sink, n_win=n_win, m_prime=mp)
    torch.cuda.synchronize()
    assert o.shape == (B, S, n_h, d)
    rows = np.arange(S) if S <= 64 else np.concatenate([np.arange(0, S, 97), [S - 1]])
    idx = O.hca_idx_rows(np.arange(S), n_win, nc, mp, S)
    o_ref, _ = _oracle_attn(q, torch.cat([kv, kvc], dim=1), sink, np.stack([idx] * B), d ** -0.5, rows)
    got = o[:, torch.as_tensor(rows, device=o.device)].float().cpu().numpy()
    err = np.abs(got - o_ref).max()
    assert err <= 2e-2, f"max |o - o_ref| = {err}"
    assert _norm_corr(torch.from_numpy(got), torch.from_numpy(o_ref)) < 5e-3


def _grad_check(fwd, q, kv, kvc, sink, rows, do, label):
    """Gradients of a CSA / HCA forward through autograd against the oracle
    backward over the same index rows and [kv ; kv_compressed] (the selection
    itself is not differentiable, as in the reference)."""
    from oracle import oracle as O
    from streamindex_amd import sparse_attn_fwd

    qr, kvr, kvcr, sr = (t.clone().requires_grad_(True) for t in (q, kv, kvc, sink))
    o = fwd(qr, kvr, kvcr, sr)
    o.backward(do)
    S = q.shape[1]
    kv_full = torch.cat([kv, kvc], 1)
    o2, lse = sparse_attn_fwd(q, kv_full, sink, rows)
    assert torch.equal(o.detach(), o2)
    bits = lambda t: t[0].cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    rdq, rdkv, rds = O.sparse_attn_bwd_rows(bits(q), bits(kv_full), bits(o2), bits(do), sink.cpu().numpy(),
                                            lse[0].cpu().numpy(), rows[0].cpu().numpy().astype(np.int64),
                                            q.shape[-1] ** -0.5)
    for name, got, ref in (("dq", qr.grad[0], rdq), ("dkv", kvr.grad[0], rdkv[:S]), ("dkv_c", kvcr.grad[0], rdkv[S:])):
        g = got.float().cpu().numpy()
        assert np.linalg.norm(g - ref) <= 1e-2 * np.linalg.norm(ref) + 1e-6, f"{label} {name}"
    assert np.abs(sr.grad.cpu().numpy() - rds).max() <= 1e-3 * max(1.0, np.abs(rds).max()), f"{label} dsink"


def test_csa_and_hca_backward(cuda_device):
    # the intent of tests/test_gradient_check.py:7-14 (CSA / HCA backward), checked
    # against the oracle instead of torch.autograd.gradcheck (bf16 inputs)
    from streamindex_amd import build_hca_topk_idxs, csa_topk_idxs, flash_csa_forward, flash_hca_forward

    B, S, n_h, d, m, n_win, top_k = 1, 256, 16, 64, 4, 16, 24
    T = S // m
    qi, ki, w = synth.indexer_inputs(B, S, 64, 128, T, seed=31)
    q, kv, kvc, sink = synth.csa_attn_inputs(B, S, n_h, d, T, seed=32, scale=0.5)
    g = torch.Generator().manual_seed(33)
    do = (torch.randn(B, S, n_h, d, generator=g) * 0.5).to(torch.bfloat16).cuda()
    rows = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m)
    _grad_check(lambda a, b, c, s: flash_csa_forward(a, b, c, qi, ki, w, s, n_win=n_win, top_k=top_k, m=m),
                q, kv, kvc, sink, rows, do, "csa")
    mp = 16
    kvc_h = kvc[:, :S // mp].contiguous()
    rows_h = build_hca_topk_idxs(B=B, seq_len=S, n_win=n_win, n_compressed=S // mp, m_prime=mp, device=q.device)
    _grad_check(lambda a, b, c, s: flash_hca_forward(a, b, c, s, n_win=n_win, m_prime=mp), q, kv, kvc_h, sink,
                rows_h.int(), do, "hca")
