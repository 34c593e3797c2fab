"""Pins the CSA / HCA index-row oracle functions (oracle/oracle.py) on the CPU.

Each function is checked against (1) a brute-force loop over the definition,
(2) the reference's own torch formula (flash_sparse/reference.py:460-475,
flash_sparse/csa.py:59-83, flash_sparse/hca.py:40-51) executed with torch on
the CPU, and (3) planted mistakes that these checks must reject (window off by
one, mask off by one, offset forgotten, -inf picks kept).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _brute_window(S, n_win):
    out = np.full((S, n_win), -1, dtype=np.int64)
    for s in range(S):
        lo = max(0, s - n_win + 1)
        # the window [lo, s] fills the LAST columns: column j <-> key s - n_win + 1 + j
        for t in range(lo, s + 1):
            out[s, t - (s - n_win + 1)] = t
    return out


def _torch_window(S, n_win):
    # flash_sparse/reference.py:460-475 run through torch
    base = torch.arange(S).unsqueeze(-1)
    offsets = torch.arange(n_win).unsqueeze(0)
    idx = (base - n_win + 1) + offsets
    legal = (idx >= 0) & (idx <= base)
    return torch.where(legal, idx, torch.full_like(idx, -1)).numpy()


@pytest.mark.parametrize("S,n_win", [(1, 1), (5, 3), (20, 7), (64, 16), (40, 128), (300, 128), (10, 0)])
def test_window_brute_force_and_torch(S, n_win):
    rows = np.arange(S)
    got = O.window_idxs(rows, n_win)
    assert got.shape == (S, n_win)
    assert np.array_equal(got, _brute_window(S, n_win))
    assert np.array_equal(got, _torch_window(S, n_win))
    # invariants: valid count min(n_win, s+1), valid entries are exactly [max(0,s-n_win+1), s] ascending
    for s in range(S):
        v = got[s][got[s] >= 0]
        assert len(v) == min(n_win, s + 1)
        assert np.array_equal(v, np.arange(max(0, s - n_win + 1), s + 1))


def test_csa_mask_equivalence():
    # csa.py:59-63 (m(i+1)-1 <= s) is the indexer's causal_ratio predicate i < (s+1)//m
    for m in range(1, 9):
        for s in range(0, 200):
            for i in range(0, 60):
                assert (m * (i + 1) - 1 <= s) == (i < (s + 1) // m)


def _torch_build_csa(scores, n_win, top_k, m):
    # flash_sparse/csa.py:55-83 (function-level body) run through torch on the CPU
    B, S, T = scores.shape
    block_last = (torch.arange(T) + 1) * m - 1
    q_pos = torch.arange(S).unsqueeze(-1)
    legal = q_pos >= block_last
    masked = scores.masked_fill(~legal.unsqueeze(0), float("-inf"))
    k_eff = min(top_k, T)
    sel, top = masked.topk(k_eff, dim=-1)
    invalid = torch.isinf(sel) & (sel < 0)
    top = top.masked_fill(invalid, -1)
    if k_eff < top_k:
        top = torch.cat([top, torch.full((B, S, top_k - k_eff), -1, dtype=top.dtype)], dim=-1)
    base = torch.arange(S).unsqueeze(-1)
    idx = (base - n_win + 1) + torch.arange(n_win).unsqueeze(0)
    win = torch.where((idx >= 0) & (idx <= base), idx, torch.full_like(idx, -1)).unsqueeze(0).expand(B, -1, -1)
    comp = torch.where(top >= 0, top + S, torch.full_like(top, -1))
    return torch.cat([win.long(), comp.long()], dim=-1).int()


@pytest.mark.parametrize("S,m,n_win,top_k", [(64, 4, 16, 8), (47, 4, 5, 16), (100, 2, 8, 64), (32, 4, 16, 3)])
def test_csa_scores_topk_matches_torch_reference(S, m, n_win, top_k):
    rng = np.random.default_rng(S + top_k)
    T = S // m
    sc = rng.standard_normal((1, S, T)).astype(np.float32)  # continuous: no ties
    ref = _torch_build_csa(torch.from_numpy(sc), n_win, top_k, m).numpy()
    got = O.csa_scores_topk_rows(sc[0].astype(np.float64), np.arange(S), m, top_k, n_win, S)
    assert got.shape == (S, n_win + top_k)
    assert np.array_equal(got, ref[0])


def test_csa_scores_topk_neg_inf_and_ties():
    # a legal -inf score is never a pick (csa.py:68-69); ties rank the smaller index first
    S, m, n_win, top_k = 24, 2, 4, 6
    sc = np.zeros((S, S // m))
    sc[:, 3] = -np.inf
    got = O.csa_scores_topk_rows(sc, np.arange(S), m, top_k, n_win, 1000)
    for s in range(S):
        lim = min(S // m, (s + 1) // m)
        legal = [i for i in range(lim) if i != 3]
        want = [1000 + i for i in legal[:top_k]] + [-1] * (top_k - min(top_k, len(legal)))
        assert list(got[s, n_win:]) == want


def test_csa_idx_rows_offset_and_padding():
    comp = np.array([[5, 2, -1], [-1, -1, -1], [0, 7, 3]])
    got = O.csa_idx_rows(comp, np.array([0, 1, 9]), 2, 100)
    assert got.tolist() == [[-1, 0, 105, 102, -1], [0, 1, -1, -1, -1], [8, 9, 100, 107, 103]]


def _brute_hca(S, n_win, n_comp, mp, off):
    out = np.full((S, n_win + n_comp), -1, dtype=np.int64)
    out[:, :n_win] = _brute_window(S, n_win)
    for s in range(S):
        for i in range(n_comp):
            # block i covers tokens [mp*i, mp*(i+1)); legal once its last token is <= s
            if all(t <= s for t in range(mp * i, mp * (i + 1))):
                out[s, n_win + i] = i + off
    return out


def _torch_hca(S, n_win, n_comp, mp):
    # flash_sparse/hca.py:40-51 run through torch on the CPU
    block_last = (torch.arange(n_comp) + 1) * mp - 1
    q_pos = torch.arange(S).unsqueeze(-1)
    legal = q_pos >= block_last
    base_idx = torch.arange(n_comp).view(1, -1).expand(S, -1)
    comp = torch.where(legal, base_idx, torch.full_like(base_idx, -1))
    comp = torch.where(comp >= 0, comp + S, torch.full_like(comp, -1))
    return torch.cat([torch.from_numpy(_torch_window(S, n_win)), comp], dim=-1).numpy()


@pytest.mark.parametrize("S,n_win,mp", [(64, 16, 8), (32, 8, 4), (300, 128, 128), (17, 0, 3), (9, 4, 1)])
def test_hca_brute_force_and_torch(S, n_win, mp):
    n_comp = S // mp
    got = O.hca_idx_rows(np.arange(S), n_win, n_comp, mp, S)
    assert np.array_equal(got, _brute_hca(S, n_win, n_comp, mp, S))
    assert np.array_equal(got, _torch_hca(S, n_win, n_comp, mp))


def test_planted_index_mistakes_are_caught():
    S, n_win = 40, 8
    rows = np.arange(S)
    good = O.window_idxs(rows, n_win)
    # window shifted by one (keys s-n_win .. s-1) fails brute force
    s = rows[:, None]
    t = s - n_win + np.arange(n_win)[None, :]
    assert not np.array_equal(np.where(t >= 0, t, -1), _brute_window(S, n_win))
    assert np.array_equal(good, _brute_window(S, n_win))
    # compressed mask off by one (i <= (s+1)//m) fails the HCA brute force
    i = np.arange(10)[None, :]
    wrong = np.where(i <= (s + 1) // 4, i + S, -1)
    assert not np.array_equal(wrong, _brute_hca(S, 0, 10, 4, S))
    # forgetting the +S offset fails the torch restatement
    sc = np.random.default_rng(3).standard_normal((1, S, S // 4)).astype(np.float32)
    ref = _torch_build_csa(torch.from_numpy(sc), n_win, 4, 4).numpy()[0]
    no_off = O.csa_scores_topk_rows(sc[0].astype(np.float64), rows, 4, 4, n_win, 0)
    assert not np.array_equal(no_off, ref)
    # keeping a selected -inf as a pick fails the -inf rule
    sc2 = np.full((S, 10), -np.inf)
    kept = O.topk(sc2, O.legal_limits(rows, 10, 4), 4)[0]
    assert (kept[rows >= 3] >= 0).any()  # the raw top-k lists legal -inf keys ...
    assert (O.csa_scores_topk_rows(sc2, rows, 4, 4, 0, 0) == -1).all()  # ... the CSA rows never do


@pytest.mark.parametrize("S,n_win,n_comp,m_prime", [(40, 5, 9, 4), (300, 16, 64, 4), (257, 8, 3, 128)])
def test_hca_row_len_matches_rows(S, n_win, n_comp, m_prime):
    # the column counts the HCA composition passes to attention: nothing
    # valid lies at or past them, and the last column before them is used
    from streamindex_amd.hca import hca_row_len

    rows = O.hca_idx_rows(np.arange(S), n_win, n_comp, m_prime, S)
    rl = hca_row_len(1, S, n_win, n_comp, m_prime, "cpu")[0].numpy()
    col = np.arange(rows.shape[1])
    assert np.all(rows[col[None, :] >= rl[:, None]] == -1)
    used = rl > n_win
    assert np.all(rows[np.arange(S)[used], rl[used] - 1] >= 0)


@pytest.mark.parametrize("S,T,m,top_k,n_win", [(40, 12, 4, 6, 5), (200, 50, 4, 16, 8), (64, 20, 2, 40, 3)])
def test_csa_row_len_matches_rows(S, T, m, top_k, n_win):
    # the fused CSA rows hold min(top_k, T, (s+1)//m) picks: finite scores,
    # so every legal key is pickable; columns past the count are -1
    from streamindex_amd.csa import csa_row_len

    rng = np.random.default_rng(S + T)
    scores = rng.standard_normal((S, T)).astype(np.float32)
    rows = O.csa_scores_topk_rows(scores, np.arange(S), m, top_k, n_win, S)
    rl = csa_row_len(1, S, n_win, top_k, T, m, "cpu")[0].numpy()
    col = np.arange(rows.shape[1])
    assert np.all(rows[col[None, :] >= rl[:, None]] == -1)
    inside = (col[None, :] < rl[:, None]) & (col[None, :] >= n_win)
    assert np.all(rows[inside] >= S)
