"""Parity checker for the indexer top-k: GPU result vs the CPU oracle on the
same inputs (rows of one batch).

Gates (stricter than the reference's own recall gates,
eval/test_v4_indexer_parity.py:272 and tests/test_chunked_indexer.py:47):

* padding: a row has exactly min(top_k, #legal) valid slots, then -1 / -inf;
* order: scores non-increasing; equal scores list the smaller index first;
* every returned (index, score) pair: index legal, score within
  SCORE_RTOL·(|ref| + row_scale) of the oracle's score at that index;
* exact index set wherever the oracle's k-th/(k+1)-th gap exceeds
  GAP_RTOL·row_scale (fp32 accumulation cannot flip such a boundary);
* mean set-overlap recall >= 0.999 over all checked rows.
"""

from __future__ import annotations

import numpy as np

from oracle import oracle as O

SCORE_RTOL = 1e-4
GAP_RTOL = 1e-4


def check_rows(scores_ref: np.ndarray, lim: np.ndarray, top_k: int, got_idx: np.ndarray, got_val: np.ndarray,
               mask_rows=None, label: str = "") -> dict:
    """scores_ref [n,T] float64 oracle scores; lim [n]; got_* [n,top_k]."""
    n, T = scores_ref.shape
    ref_idx, ref_val = O.topk(scores_ref, lim, top_k, mask_rows)
    nvalid_ref = (ref_idx >= 0).sum(1)
    nvalid_got = (got_idx >= 0).sum(1)
    assert np.array_equal(nvalid_ref, nvalid_got), f"{label}: valid-count mismatch"
    pos = np.arange(top_k)[None, :]
    pad = pos >= nvalid_ref[:, None]
    assert np.all(got_idx[pad] == -1), f"{label}: padding index not -1"
    assert np.all(np.isneginf(got_val[pad])), f"{label}: padding score not -inf"
    assert np.all(got_idx[~pad] >= 0), f"{label}: hole inside the valid prefix"
    # legality of every returned index
    rr, cc = np.nonzero(~pad)
    ii = got_idx[rr, cc]
    assert np.all(ii < lim[rr]), f"{label}: returned an illegal (future) key"
    if mask_rows is not None:
        assert np.all(mask_rows[rr, ii] != 0), f"{label}: returned a masked key"
    # scores at the returned indices
    row_scale = np.array([np.abs(scores_ref[r, : max(1, int(min(lim[r], T)))]).mean() if lim[r] > 0 else 1.0
                          for r in range(n)])
    ref_at = scores_ref[rr, ii]
    err = np.abs(got_val[rr, cc].astype(np.float64) - ref_at)
    tol = SCORE_RTOL * (np.abs(ref_at) + row_scale[rr]) + 1e-30
    bad = err > tol
    assert not bad.any(), f"{label}: {bad.sum()} scores off, worst {err.max():.3e} (tol {tol[bad].min():.3e})"
    # order: non-increasing, ties by smaller index
    for r in range(n):
        m = int(nvalid_got[r])
        v = got_val[r, :m]
        assert np.all(v[:-1] >= v[1:]), f"{label}: row {r} not sorted"
        tie = v[:-1] == v[1:]
        if tie.any():
            i = got_idx[r, :m]
            assert np.all(i[:-1][tie] < i[1:][tie]), f"{label}: row {r} tie order"
        # distinct indices
        assert len(set(got_idx[r, :m].tolist())) == m, f"{label}: row {r} duplicate index"
    # exact set where the boundary gap is wide
    rec = O.set_overlap_recall(ref_idx, got_idx)
    gaps = np.full(n, np.inf)
    for r in range(n):
        sel = ref_val[r][np.isfinite(ref_val[r])]
        if len(sel) < top_k:
            continue
        legal = scores_ref[r, : int(min(lim[r], T))]
        if mask_rows is not None:
            legal = legal[mask_rows[r, : int(min(lim[r], T))] != 0]
        if legal.size <= top_k:
            continue
        kth = sel[top_k - 1]
        if np.sum(legal >= kth) > top_k:
            gaps[r] = 0.0  # exact tie across the boundary: membership is decided by index
            continue
        nxt = np.max(legal[legal < kth]) if np.any(legal < kth) else -np.inf
        gaps[r] = kth - nxt
    wide = gaps > GAP_RTOL * row_scale
    assert np.all(rec[wide] == 1.0), f"{label}: {np.sum(rec[wide] < 1)} wide-gap rows differ"
    assert rec.mean() >= 0.999, f"{label}: mean recall {rec.mean():.5f}"
    return {"recall_mean": float(rec.mean()), "recall_min": float(rec.min()),
            "exact_rows": float((rec == 1.0).mean()), "narrow_gap_rows": int((~wide).sum()),
            "max_score_err": float(err.max()) if err.size else 0.0}


def check_indexer(q, k, w, top_k, got_idx, got_val, *, causal_ratio=None, mask=None, rows=None, label=""):
    """Torch tensors in, oracle comparison for every batch over `rows`."""
    import torch

    from tests.conftest import bf16_bits

    B, S, H, D = q.shape
    T = k.shape[1]
    rows = np.arange(S, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
    stats = []
    # only the checked rows leave the device (q is 16 GiB at S = 1M)
    sel = torch.as_tensor(rows, device=q.device)
    local = np.arange(len(rows), dtype=np.int64)
    for b in range(B):
        qb = bf16_bits(q[b].index_select(0, sel))
        kb = bf16_bits(k[b])
        wb = w[b].index_select(0, sel).float().cpu().numpy()
        lim = O.legal_limits(rows, T, causal_ratio)
        sc = O.indexer_scores(qb, kb, wb, local, lim=lim)
        mrows = None
        if mask is not None:
            mrows = mask[b].index_select(0, sel.to(mask.device)).cpu().numpy().astype(np.uint8)
        gi = got_idx[b].index_select(0, sel.to(got_idx.device)).cpu().numpy()
        gv = got_val[b].index_select(0, sel.to(got_val.device)).cpu().numpy()
        stats.append(check_rows(sc, lim, top_k, gi, gv, mrows, label=f"{label}[b={b}]"))
    return stats
