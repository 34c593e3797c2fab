"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

The reference holds no golden vectors for this path (no data files at all), so each
oracle function is pinned by checks a plausible mistake would fail:

* brute force in plain Python loops on tiny inputs;
* the reference's own formula executed by torch on the CPU (the library the
  reference calls: einsum / relu / sum / masked_fill / topk / softmax), i.e.
  reference.py:165-168 and eval/test_v4_indexer_parity.py:121-136 run through
  an independent implementation;
* closed forms and invariants (ReLU zero region, single head, linearity in
  w, legal-count formula, partition-merge invariance, sink-augmented softmax,
  one-key and all-masked rows, masking == truncation);
* planted mistakes in copies of the oracle (no ReLU, mask off by one, wrong
  tie order, sink added to the numerator) that these checks must reject.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _rand_bf16(rng, shape, scale=1.0):
    return O.f32_to_bf16_bits(rng.standard_normal(shape).astype(np.float32) * scale)


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------
def test_bf16_roundtrip_matches_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(10000).astype(np.float32) * 10
    ours = O.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    back = O.bf16_bits_to_f64(ours)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).double().numpy())


# ---------------------------------------------------------------------------
# score  I(s,t) = Σ_h w[s,h] relu(q[s,h]·k[t])
# ---------------------------------------------------------------------------
def _brute_scores(qf, kf, w):
    S, H, D = qf.shape
    T = kf.shape[0]
    out = [[0.0] * T for _ in range(S)]
    for s in range(S):
        for t in range(T):
            acc = 0.0
            for h in range(H):
                dot = sum(float(qf[s, h, d]) * float(kf[t, d]) for d in range(D))
                acc += float(w[s, h]) * max(0.0, dot)
            out[s][t] = acc
    return np.array(out)


def test_scores_brute_force_tiny():
    rng = np.random.default_rng(1)
    qb, kb = _rand_bf16(rng, (3, 2, 4)), _rand_bf16(rng, (5, 4))
    w = rng.standard_normal((3, 2)).astype(np.float32)
    got = O.indexer_scores(qb, kb, w)
    ref = _brute_scores(O.bf16_bits_to_f64(qb), O.bf16_bits_to_f64(kb), w.astype(np.float64))
    assert np.allclose(got, ref, rtol=0, atol=1e-12)
    assert np.allclose(O.np_indexer_scores(O.bf16_bits_to_f64(qb), O.bf16_bits_to_f64(kb), w.astype(np.float64)),
                       ref, rtol=0, atol=1e-12)


def test_scores_brute_force_key_blocks_and_causal_limit():
    # T not a multiple of the oracle's 8-key vector blocks; D, H beyond the tiny case
    rng = np.random.default_rng(11)
    S, H, D, T = 5, 3, 16, 21
    qb, kb = _rand_bf16(rng, (S, H, D)), _rand_bf16(rng, (T, D))
    w = rng.standard_normal((S, H)).astype(np.float32)
    ref = _brute_scores(O.bf16_bits_to_f64(qb), O.bf16_bits_to_f64(kb), w.astype(np.float64))
    full = O.indexer_scores(qb, kb, w)
    assert np.allclose(full, ref, rtol=0, atol=1e-12)
    rows = np.array([4, 0, 2, 3])
    lim = np.array([0, 7, 21, 9])
    got = O.indexer_scores(qb, kb, w, rows, lim=lim)
    for r, (s, L) in enumerate(zip(rows, lim)):
        # the legal prefix is bit-identical to the unlimited scores; the rest is NaN
        assert np.array_equal(got[r, :L].view(np.uint64), full[s, :L].view(np.uint64))
        assert np.isnan(got[r, L:]).all()


def test_scores_match_torch_reference_formula():
    # reference.py:165-168 executed by torch on the CPU in fp32
    rng = np.random.default_rng(2)
    S, H, D, T = 40, 16, 64, 90
    qb, kb = _rand_bf16(rng, (S, H, D), 0.5), _rand_bf16(rng, (T, D), 0.5)
    w = rng.standard_normal((S, H)).astype(np.float32)
    q = torch.from_numpy(qb.view(np.int16)).view(torch.bfloat16).unsqueeze(0)
    k = torch.from_numpy(kb.view(np.int16)).view(torch.bfloat16).unsqueeze(0)
    wt = torch.from_numpy(w).unsqueeze(0)
    qk = torch.einsum("bshd,btd->bsht", q.float(), k.float()).relu()
    ref = (qk * wt.unsqueeze(-1)).sum(dim=2)[0].double().numpy()
    got = O.indexer_scores(qb, kb, w)
    scale = np.abs(ref).mean()
    assert np.abs(got - ref).max() <= 1e-5 * scale
    got32 = O.indexer_scores(qb, kb, w, precision="f32")
    assert np.abs(got32 - ref).max() <= 1e-5 * scale


def test_scores_relu_zero_region_and_single_head():
    rng = np.random.default_rng(3)
    S, H, D, T = 6, 8, 32, 20
    kb = _rand_bf16(rng, (T, D))
    kf = O.bf16_bits_to_f64(kb)
    # q_h = -k_0 direction for every head: q·k_0 < 0 -> key 0 scores exactly 0 for w >= 0
    qf = np.repeat(-kf[0][None, None, :], S, axis=0).repeat(H, axis=1)
    qb = O.f32_to_bf16_bits(qf.astype(np.float32))
    w = np.abs(rng.standard_normal((S, H))).astype(np.float32)
    sc = O.indexer_scores(qb, kb, w)
    assert np.all(sc[:, 0] == 0.0)
    # single active head: score = w * relu(q.k)
    w1 = np.zeros((S, H), dtype=np.float32)
    w1[:, 3] = rng.standard_normal(S).astype(np.float32)
    qb2 = _rand_bf16(rng, (S, H, D))
    sc1 = O.indexer_scores(qb2, kb, w1)
    dots = O.bf16_bits_to_f64(qb2)[:, 3, :] @ kf.T
    assert np.allclose(sc1, w1[:, 3:4].astype(np.float64) * np.maximum(dots, 0), rtol=0, atol=1e-12)


def test_scores_linear_in_weights():
    rng = np.random.default_rng(4)
    S, H, D, T = 9, 16, 32, 33
    qb, kb = _rand_bf16(rng, (S, H, D)), _rand_bf16(rng, (T, D))
    w1 = rng.standard_normal((S, H)).astype(np.float32)
    w2 = rng.standard_normal((S, H)).astype(np.float32)
    w12 = (w1.astype(np.float64) + w2).astype(np.float32)
    lhs = O.indexer_scores(qb, kb, w12)
    rhs = O.indexer_scores(qb, kb, w1) + O.indexer_scores(qb, kb, w2)
    err_w = np.abs(w12.astype(np.float64) - (w1.astype(np.float64) + w2)).max()
    assert np.abs(lhs - rhs).max() <= 1e-9 + err_w * 100


def test_scores_row_selection_and_batches_independent():
    rng = np.random.default_rng(5)
    S, H, D, T = 20, 16, 32, 17
    qb, kb = _rand_bf16(rng, (S, H, D)), _rand_bf16(rng, (T, D))
    w = rng.standard_normal((S, H)).astype(np.float32)
    full = O.indexer_scores(qb, kb, w)
    rows = np.array([19, 0, 7, 7], dtype=np.int64)
    assert np.array_equal(O.indexer_scores(qb, kb, w, rows), full[rows])


# ---------------------------------------------------------------------------
# causal mask  t < (s+1)//ratio
# ---------------------------------------------------------------------------
def test_legal_limits_closed_form():
    for ratio in (1, 2, 4, 8):
        for T in (0, 1, 5, 64):
            rows = np.arange(300)
            lim = O.legal_limits(rows, T, ratio)
            brute = np.array([sum(1 for t in range(T) if t < (s + 1) // ratio) for s in rows])
            assert np.array_equal(lim, brute)
            assert np.all(lim[: ratio - 1] == 0)  # rows s < ratio-1 have no legal key
    assert np.array_equal(O.legal_limits(np.arange(5), 7, None), np.full(5, 7))


def test_mask_matches_reference_illegal_matrix():
    # eval/test_v4_indexer_parity.py:124-127: illegal = arange(T) >= arange(1,S+1)//ratio
    S, T, ratio = 37, 11, 4
    illegal = (torch.arange(T).repeat(S, 1) >= torch.arange(1, S + 1).unsqueeze(1) // ratio).numpy()
    lim = O.legal_limits(np.arange(S), T, ratio)
    legal = np.arange(T)[None, :] < lim[:, None]
    assert np.array_equal(legal, ~illegal)


# ---------------------------------------------------------------------------
# top-k selection
# ---------------------------------------------------------------------------
def test_topk_brute_force_and_padding():
    rng = np.random.default_rng(6)
    n, T, k = 30, 25, 8
    sc = rng.standard_normal((n, T))
    sc[3, :] = 0.0            # full tie row
    sc[4, 5:9] = sc[4, 2]     # partial ties
    lim = rng.integers(0, T + 1, n)
    idx, val = O.topk(sc, lim, k)
    for r in range(n):
        pairs = sorted(((-sc[r, t], t) for t in range(int(lim[r]))))[:k]
        exp_i = [t for _, t in pairs] + [-1] * (k - len(pairs))
        exp_v = [-v for v, _ in pairs] + [-np.inf] * (k - len(pairs))
        assert list(idx[r]) == exp_i
        assert np.array_equal(val[r], np.array(exp_v))
    i2, v2 = O.np_topk(sc, lim, k)
    assert np.array_equal(idx, i2) and np.array_equal(val, v2)


def test_topk_matches_torch_topk_without_ties():
    # eval/test_v4_indexer_parity.py:128-136 via torch: mask -> topk(min(k,T)) -> post-mask -1
    rng = np.random.default_rng(7)
    S, T, k, ratio = 64, 40, 12, 4
    sc = rng.standard_normal((S, T))
    illegal = torch.arange(T).repeat(S, 1) >= torch.arange(1, S + 1).unsqueeze(1) // ratio
    t_sc = torch.from_numpy(sc).masked_fill(illegal, float("-inf"))
    t_val, t_idx = t_sc.topk(min(k, T), dim=-1)
    boundary = torch.arange(1, S + 1).unsqueeze(1) // ratio
    t_idx = torch.where(t_idx >= boundary, torch.full_like(t_idx, -1), t_idx)
    idx, val = O.topk(sc, O.legal_limits(np.arange(S), T, ratio), k)
    assert np.array_equal(idx, t_idx.numpy())
    fin = np.isfinite(val)
    assert np.array_equal(fin, np.isfinite(t_val.numpy()))
    assert np.array_equal(val[fin], t_val.numpy()[fin])


def test_topk_with_bool_mask():
    rng = np.random.default_rng(8)
    n, T, k = 12, 30, 6
    sc = rng.standard_normal((n, T))
    mask = rng.random((n, T)) < 0.25
    idx, val = O.topk(sc, np.full(n, T, dtype=np.int64), k, mask.astype(np.uint8))
    for r in range(n):
        legal = [t for t in range(T) if mask[r, t]]
        best = sorted(legal, key=lambda t: (-sc[r, t], t))[:k]
        assert list(idx[r, : len(best)]) == best
        assert np.all(idx[r, len(best):] == -1)


@pytest.mark.parametrize("chunk_t", [1, 3, 7, 16, 64, 200])
def test_partition_merge_invariance(chunk_t):
    # docs/streaming_topk.md:81-143: top-k is invariant under partition-then-merge,
    # including chunks narrower than k (the cT < k branch the ablation breaks).
    rng = np.random.default_rng(9)
    n, T, k, ratio = 47, 73, 16, 1
    sc = np.round(rng.standard_normal((n, T)), 1)  # many exact ties
    lim = O.legal_limits(np.arange(n), T, ratio)
    gi, gv = O.topk(sc, lim, k)
    ci, cv = O.np_chunked_topk(sc, lim, k, chunk_t)
    assert np.array_equal(gi, ci) and np.array_equal(gv, cv)


def test_full_pipeline_against_torch_materialize():
    # _materialize_topk (eval/test_v4_indexer_parity.py:111-137) through torch, vs the C oracle
    rng = np.random.default_rng(10)
    S, H, D, k, ratio = 96, 16, 32, 10, 4
    T = S // ratio
    qb, kb = _rand_bf16(rng, (S, H, D), D ** -0.5), _rand_bf16(rng, (T, D), D ** -0.5)
    w = rng.standard_normal((S, H)).astype(np.float32)
    q = torch.from_numpy(qb.view(np.int16)).view(torch.bfloat16).unsqueeze(0).double()
    kk = torch.from_numpy(kb.view(np.int16)).view(torch.bfloat16).unsqueeze(0).double()
    score = (torch.einsum("bshd,btd->bsht", q, kk).relu() * torch.from_numpy(w).double().unsqueeze(0).unsqueeze(-1)).sum(2)
    illegal = torch.arange(T).repeat(S, 1) >= torch.arange(1, S + 1).unsqueeze(1) // ratio
    score = score.masked_fill(illegal.unsqueeze(0), float("-inf"))
    t_idx = score.topk(min(k, T), dim=-1)[1]
    boundary = torch.arange(1, S + 1).unsqueeze(1) // ratio
    t_idx = torch.where(t_idx >= boundary.unsqueeze(0), torch.full_like(t_idx, -1), t_idx)[0].numpy()
    idx, _, _ = O.indexer_topk_rows(qb, kb, w, k, causal_ratio=ratio)
    rec = O.set_overlap_recall(t_idx, idx)
    assert rec.min() == 1.0


# ---------------------------------------------------------------------------
# recall metric (eval/test_v4_indexer_parity.py:164-199)
# ---------------------------------------------------------------------------
def test_set_overlap_recall_cases():
    a = np.array([[1, 2, 3, -1], [-1, -1, -1, -1], [-1, -1, -1, -1], [5, 6, 7, 8], [0, 1, 2, 3]])
    b = np.array([[3, 2, 1, -1], [-1, -1, -1, -1], [4, -1, -1, -1], [5, 6, -1, 9], [9, 8, 7, 6]])
    assert np.allclose(O.set_overlap_recall(a, b), [1.0, 1.0, 0.0, 0.5, 0.0])
    # against a torch restatement of the reference's vectorised form
    rng = np.random.default_rng(11)
    A = rng.integers(-1, 20, (3, 50, 8))
    B = rng.integers(-1, 20, (3, 50, 8))
    sa, sb = torch.from_numpy(A), torch.from_numpy(B)
    va, vb = sa >= 0, sb >= 0
    sa2 = torch.where(va, sa, torch.full_like(sa, -2))
    sb2 = torch.where(vb, sb, torch.full_like(sb, -3))
    match = (sa2.unsqueeze(-1) == sb2.unsqueeze(-2)) & va.unsqueeze(-1)
    # the reference counts duplicate hits per slot; with distinct sets it equals the set formula
    ours = O.set_overlap_recall(A, B)
    for i in range(3):
        for s in range(50):
            ua = {x for x in A[i, s] if x >= 0}
            if len(ua) == int(va[i, s].sum()):
                cnt = float(match[i, s].any(-1).sum())
                ref = 1.0 if (not ua and not vb[i, s].any()) else (0.0 if not ua else cnt / len(ua))
                assert math.isclose(ours[i, s], ref)


# ---------------------------------------------------------------------------
# sparse attention (reference.py:44-130)
# ---------------------------------------------------------------------------
def _attn_inputs(rng, n, H, D, N, K, frac_masked=0.25):
    qb = _rand_bf16(rng, (n, H, D), 0.5)
    kvb = _rand_bf16(rng, (N, D), 0.5)
    sink = rng.standard_normal(H).astype(np.float32)
    idx = rng.integers(0, N, (n, K))
    idx[rng.random((n, K)) < frac_masked] = -1
    return qb, kvb, sink, idx


def test_attn_c_matches_numpy():
    rng = np.random.default_rng(12)
    qb, kvb, sink, idx = _attn_inputs(rng, 7, 8, 32, 50, 20)
    o, lse = O.sparse_attn_rows(qb, kvb, sink, idx, 0.2)
    o2, l2 = O.np_sparse_attn(O.bf16_bits_to_f64(qb), O.bf16_bits_to_f64(kvb), sink.astype(np.float64), idx, 0.2)
    assert np.allclose(o, o2, atol=1e-12) and np.allclose(lse, l2, atol=1e-12)


def test_attn_dense_fallthrough_equals_torch_softmax_with_sink():
    # tests/test_against_reference.py:109-135: all keys selected == softmax over keys ∪ {sink}
    rng = np.random.default_rng(13)
    n, H, D, N = 5, 4, 16, 12
    qb, kvb, sink, _ = _attn_inputs(rng, n, H, D, N, N)
    idx = np.tile(np.arange(N), (n, 1))
    o, lse = O.sparse_attn_rows(qb, kvb, sink, idx, D ** -0.5)
    q = torch.from_numpy(O.bf16_bits_to_f64(qb))
    kv = torch.from_numpy(O.bf16_bits_to_f64(kvb))
    s = torch.einsum("nhd,md->nhm", q, kv) * D ** -0.5
    logits = torch.cat([s, torch.from_numpy(sink).double().view(1, H, 1).expand(n, H, 1)], -1)
    p = logits.softmax(-1)[..., :N]
    assert np.allclose(o, torch.einsum("nhm,md->nhd", p, kv).numpy(), atol=1e-12)
    assert np.allclose(lse, torch.logsumexp(logits, -1).numpy(), atol=1e-12)


def test_attn_all_masked_and_single_key():
    rng = np.random.default_rng(14)
    n, H, D, N, K = 3, 4, 8, 10, 6
    qb, kvb, sink, _ = _attn_inputs(rng, n, H, D, N, K)
    idx = np.full((n, K), -1)
    idx[1, 2] = 4  # one valid key
    idx[2, :] = [11, 10, -5, 99, -1, 12]  # out-of-range entries count as masked
    o, lse = O.sparse_attn_rows(qb, kvb, sink, idx, 0.3)
    assert np.all(o[0] == 0) and np.allclose(lse[0], sink)
    assert np.all(o[2] == 0) and np.allclose(lse[2], sink)
    qf, kvf = O.bf16_bits_to_f64(qb), O.bf16_bits_to_f64(kvb)
    sc = qf[1] @ kvf[4] * 0.3
    expect = (np.exp(sc) / (np.exp(sc) + np.exp(sink.astype(np.float64))))[:, None] * kvf[4][None, :]
    assert np.allclose(o[1], expect, atol=1e-12)
    # sink = -inf and no valid key: zero output and the -1e30 LSE sentinel
    o3, l3 = O.sparse_attn_rows(qb[:1], kvb, np.full(H, -np.inf, dtype=np.float32), idx[:1], 0.3)
    assert np.all(o3 == 0) and np.all(l3 == -1.0e30)


def test_attn_masking_equals_truncation_and_order_invariance():
    rng = np.random.default_rng(15)
    qb, kvb, sink, idx = _attn_inputs(rng, 6, 8, 32, 40, 16, frac_masked=0.0)
    padded = np.concatenate([idx, -np.ones((6, 9), dtype=idx.dtype)], 1)
    o1, l1 = O.sparse_attn_rows(qb, kvb, sink, idx, 0.25)
    o2, l2 = O.sparse_attn_rows(qb, kvb, sink, padded, 0.25)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    perm = rng.permutation(16)
    o3, l3 = O.sparse_attn_rows(qb, kvb, sink, idx[:, perm], 0.25)
    assert np.allclose(o1, o3, atol=1e-12) and np.allclose(l1, l3, atol=1e-12)


# ---------------------------------------------------------------------------
# planted mistakes: the checks above must reject each mutated oracle
# ---------------------------------------------------------------------------
def _mut_scores_no_relu(qf, kf, w):
    return (np.einsum("shd,td->sht", qf, kf) * w[:, :, None]).sum(1)


def _mut_scores_relu_after_sum(qf, kf, w):
    return np.maximum((np.einsum("shd,td->sht", qf, kf) * w[:, :, None]).sum(1), 0)


def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(16)
    S, H, D, T = 6, 8, 16, 9
    qb, kb = _rand_bf16(rng, (S, H, D)), _rand_bf16(rng, (T, D))
    qf, kf = O.bf16_bits_to_f64(qb), O.bf16_bits_to_f64(kb)
    w = rng.standard_normal((S, H))
    ref = _brute_scores(qf, kf, w)
    for mut in (_mut_scores_no_relu, _mut_scores_relu_after_sum):
        assert not np.allclose(mut(qf, kf, w), ref, atol=1e-9), mut.__name__
    # mask off by one (t <= (s+1)//r) breaks the legal-count closed form
    rows = np.arange(40)
    wrong = np.minimum(T, (rows + 1) // 4 + 1)
    assert not np.array_equal(wrong, O.legal_limits(rows, T, 4))
    # index-descending tie order breaks the brute-force top-k check
    sc = np.zeros((1, 6))
    good, _ = O.topk(sc, np.array([6]), 3)
    assert list(good[0]) == [0, 1, 2]
    assert list(np.argsort(-sc[0], kind="stable")[::-1][:3]) != list(good[0])
    # sink in the numerator breaks the dense softmax closed form
    qa, kva, sink, _ = _attn_inputs(rng, 2, 4, 8, 6, 6)
    idx = np.tile(np.arange(6), (2, 1))
    o, _ = O.sparse_attn_rows(qa, kva, sink, idx, 0.5)
    qf2, kv2 = O.bf16_bits_to_f64(qa), O.bf16_bits_to_f64(kva)
    s = np.einsum("nhd,md->nhm", qf2, kv2) * 0.5
    p_wrong = np.exp(s) / np.exp(s).sum(-1, keepdims=True)  # sink dropped entirely
    assert not np.allclose(np.einsum("nhm,md->nhd", p_wrong, kv2), o, atol=1e-6)



# ---------------------------------------------------------------------------
# the CPU baseline (the reference's fp32 materialise path, op for op)
# ---------------------------------------------------------------------------
def _torch_inputs(rng, S, H, D, T):
    qb, kb = _rand_bf16(rng, (S, H, D), D ** -0.5), _rand_bf16(rng, (T, D), D ** -0.5)
    w = rng.standard_normal((S, H)).astype(np.float32)
    q = torch.from_numpy(qb.view(np.int16)).view(torch.bfloat16).unsqueeze(0)
    k = torch.from_numpy(kb.view(np.int16)).view(torch.bfloat16).unsqueeze(0)
    return qb, kb, w, q, k, torch.from_numpy(w).unsqueeze(0)


@pytest.mark.parametrize("S,T,k", [(128, 32, 10), (96, 24, 40), (4096 // 16, 1024 // 16, 512 // 16)])
def test_torch_materialize_baseline_matches_c_oracle(S, T, k):
    from oracle.torch_materialize import materialize_topk

    rng = np.random.default_rng(S + T + k)
    H, D, ratio = 16, 32, 4
    qb, kb, w, q, kk, wt = _torch_inputs(rng, S, H, D, T)
    t_idx, t_val = materialize_topk(q, kk, wt, k, ratio)
    assert t_idx.shape == (1, S, min(k, T)) and t_idx.dtype == torch.int64 and t_val.dtype == torch.float32
    ref_idx, ref_val, _ = O.indexer_topk_rows(qb, kb, w, min(k, T), causal_ratio=ratio)
    got = t_idx[0].numpy()
    # fp32 scores of distinct Gaussian keys: same sets and order as the fp64 oracle
    assert O.set_overlap_recall(ref_idx, got).min() == 1.0
    fin = np.isfinite(ref_val)
    assert np.array_equal(got >= 0, fin)
    assert np.allclose(t_val[0].numpy()[fin], ref_val[fin], rtol=1e-5, atol=1e-6)
    # rows s < ratio - 1 have no legal key: every slot is -1 after the post-mask
    assert np.all(got[: ratio - 1] == -1)


def test_torch_materialize_post_mask_is_needed():
    """Without the post-mask the -inf slots of short rows carry arbitrary
    indices, which the recall metric would count as wrong picks."""
    from oracle.torch_materialize import materialize_topk

    rng = np.random.default_rng(5)
    S, H, D, T, k, ratio = 64, 16, 32, 16, 8, 4
    qb, kb, w, q, kk, wt = _torch_inputs(rng, S, H, D, T)
    idx, val = materialize_topk(q, kk, wt, k, ratio)
    short = torch.isinf(val[0])
    assert bool(short.any()) and bool((idx[0][short] == -1).all())
    assert bool((idx[0][~short] >= 0).all())


# ---------------------------------------------------------------------------
# fp16 operands of the attention oracle
# ---------------------------------------------------------------------------
def test_f16_decoder_matches_numpy_on_every_bit_pattern():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))  # exact, signed zeros included


def test_attn_oracle_f16_matches_numpy_restatement():
    """The C oracle on fp16 operands equals the numpy restatement run on the
    same values; the same values as bf16 bits give a different answer (the
    flag selects the decoding)."""
    rng = np.random.default_rng(21)
    n, H, D, N, K = 5, 4, 32, 40, 12
    q = (rng.standard_normal((n, H, D)) * 0.7).astype(np.float16)
    kv = (rng.standard_normal((N, D)) * 0.7).astype(np.float16)
    sink = rng.standard_normal(H).astype(np.float32)
    idx = rng.integers(-1, N, size=(n, K))
    o, lse = O.sparse_attn_rows(q.view(np.uint16), kv.view(np.uint16), sink, idx, D ** -0.5, f16=True)
    ro, rl = O.np_sparse_attn(q.astype(np.float64), kv.astype(np.float64), sink, idx, D ** -0.5)
    assert np.allclose(o, ro, rtol=1e-12, atol=1e-12) and np.allclose(lse, rl, rtol=1e-12, atol=1e-12)
    wrong, _ = O.sparse_attn_rows(q.view(np.uint16), kv.view(np.uint16), sink, idx, D ** -0.5)
    assert not np.allclose(wrong, ro, atol=1e-3)
    # backward: fp16 finite differences of the fp16-valued forward are what the
    # bf16 path's tests pin; here the flag must select the same decoding
    do = (rng.standard_normal((n, H, D)) * 0.5).astype(np.float16)
    of16 = o.astype(np.float16)
    dq, dkv, ds = O.sparse_attn_bwd_rows(q.view(np.uint16), kv.view(np.uint16), of16.view(np.uint16),
                                         do.view(np.uint16), sink, lse.astype(np.float32), idx, D ** -0.5, f16=True)
    dq2, dkv2, ds2 = O.np_sparse_attn_bwd(q.astype(np.float64), kv.astype(np.float64), of16.astype(np.float64),
                                          do.astype(np.float64), sink, lse.astype(np.float32).astype(np.float64), idx,
                                          D ** -0.5)
    assert np.allclose(dq, dq2, rtol=1e-10, atol=1e-12) and np.allclose(dkv, dkv2, rtol=1e-10, atol=1e-12)
    assert np.allclose(ds, ds2, rtol=1e-10, atol=1e-12)
