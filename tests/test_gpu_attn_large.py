"""Full-size sparse-attention parity at the BASELINE attention workloads.

* config[3]: ``sparse_attn_fwd`` at S=65,536, 64 heads, D=576, N_kv=16,384,
  k=512, softmax scale 576^-0.5, on config[1]'s own indexer output (the fused
  ``chunked_indexer_topk`` on seed 2026: int64, ``-1`` past the causal count);
* config[4]: the attention stage of ``flash_csa_forward`` at S=1,048,576
  (T=262,144, n_win=128, top_k=512, 64 heads, d=576).

The CPU oracle cannot run these whole, so sampled rows go through the oracle
(|o - o_ref| <= 2e-2, |lse - lse_ref| <= 2e-3, ``reference.py:44-130`` with the
sink folded once, ``sparse_attn_fwd.py:148-177``) and every row through
size-independent properties: finite outputs, and rows with no valid index
give o = 0 and lse = sink.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import chunked_indexer_topk, csa_topk_idxs, flash_csa_forward, sparse_attn_fwd, synth
from tests.conftest import bf16_bits

pytestmark = pytest.mark.gpu

O_TOL = 2e-2
LSE_TOL = 2e-3


def _say(msg):
    print(f"[test] {msg}", flush=True)


def _oracle_rows(q, kv, sink, idx, rows, scale):
    """Oracle attention for the sampled rows of batch 0 (only those rows and
    the keys they select leave the device)."""
    sel = torch.as_tensor(rows, device=q.device)
    ir = idx[0].index_select(0, sel).long()
    uniq = torch.unique(ir[ir >= 0])
    remap = torch.where(ir >= 0, torch.searchsorted(uniq, ir.clamp(min=0)), torch.full_like(ir, -1))
    ro, rl = O.sparse_attn_rows(bf16_bits(q[0].index_select(0, sel)), bf16_bits(kv[0].index_select(0, uniq)),
                                sink.cpu().numpy(), remap.cpu().numpy(), scale)
    return ro, rl


def _check_rows(o, lse, ro, rl, rows, label):
    sel = torch.as_tensor(rows, device=o.device)
    go = o[0].index_select(0, sel).float().cpu().numpy()
    gl = lse[0].index_select(0, sel).cpu().numpy()
    assert np.isfinite(go).all() and np.isfinite(gl).all(), f"{label}: non-finite sampled output"
    oe = float(np.abs(go - ro).max())
    le = float(np.abs(gl - rl).max())
    assert oe <= O_TOL, f"{label}: o error {oe:.3e}"
    assert le <= LSE_TOL * max(1.0, float(np.abs(rl).max())), f"{label}: lse error {le:.3e}"
    return oe, le


def _check_empty_rows(o, lse, sink, nvalid, label):
    empty = nvalid == 0
    if bool(empty.any()):
        oz = o[0][empty]
        assert bool((oz == 0).all()), f"{label}: a row without valid keys has o != 0"
        assert torch.allclose(lse[0][empty], sink.expand(int(empty.sum()), -1)), f"{label}: empty-row lse != sink"
    assert bool(torch.isfinite(lse).all()), f"{label}: non-finite lse"


def test_c3_sparse_attn_on_c1_indexer_output():
    S, T, H, D, top_k, ratio = 65536, 16384, 64, 576, 512, 4
    qi, ki, wi = synth.indexer_inputs(1, S, 64, 128, ratio=ratio, seed=2026, device="cuda")
    _say("config[3] indices: chunked_indexer_topk S=65536 T=16384 k=512 seed=2026")
    idx, _ = chunked_indexer_topk(qi, ki, wi, top_k, causal_ratio=ratio, chunk_s=2048, chunk_t=8192)
    del qi, ki, wi
    q, kv, sink = synth.sparse_attn_inputs(1, S, H, D, T, seed=2027, device="cuda")
    scale = D ** -0.5
    _say("config[3] sparse_attn_fwd S=65536 H=64 D=576 N_kv=16384 K=512 int64 indices")
    o, lse = sparse_attn_fwd(q, kv, sink, idx, scale)
    torch.cuda.synchronize()
    nvalid = (idx[0] >= 0).sum(-1)
    assert int(nvalid.max()) == top_k and int(nvalid[: ratio - 1].max()) == 0
    _check_empty_rows(o, lse, sink, nvalid, "config[3]")
    assert bool(torch.isfinite(o).all()), "config[3]: non-finite output"
    rng = np.random.default_rng(33)
    rows = np.unique(np.concatenate([[0, 3, 4, 7, 2047, 2048, S - 1], rng.choice(S, 96, replace=False)]))
    ro, rl = _oracle_rows(q, kv, sink, idx, rows, scale)
    oe, le = _check_rows(o, lse, ro, rl, rows, "config[3]")
    _say(f"config[3] sampled rows {len(rows)}: max |o err| {oe:.2e}, max |lse err| {le:.2e}")
    # the result does not depend on the order of a row's indices (the indexer
    # lists them best-first): the same rows with their indices sorted by key
    # (descending, so the -1 tail stays last) pass the same oracle gate
    sub = rows[-16:]
    subt = torch.as_tensor(sub, device=q.device)
    idx_s = torch.sort(idx[0].index_select(0, subt), dim=-1, descending=True).values.unsqueeze(0)
    o2, l2 = sparse_attn_fwd(q[:, subt], kv, sink, idx_s, scale)
    torch.cuda.synchronize()
    _check_rows(o2, l2, ro[-16:], rl[-16:], np.arange(16), "config[3] key-sorted indices")
    del q, kv, sink, idx, o, lse, o2, l2
    torch.cuda.empty_cache()


def test_c4_s1m_csa_attention_stage():
    """flash_csa_forward at S=1M: 256 sampled rows' compressed picks against
    the oracle's exact top-k (recall), 32 sampled rows' attention output
    against the oracle attention over the same index rows, every row's output
    finite."""
    from streamindex_amd.csa import csa_row_len

    S, m, n_win, top_k, n_h, d = 1 << 20, 4, 128, 512, 64, 576
    T = S // m
    qi, ki, w = synth.indexer_inputs(1, S, 64, 128, ratio=m, seed=2026, device="cuda")
    q, kv, kvc, sink = synth.csa_attn_inputs(1, S, n_h, d, T, seed=2027, device="cuda")
    _say("config[4] flash_csa_forward S=1048576 T=262144 n_win=128 k=512 h=64 d=576")
    o = flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=n_win, top_k=top_k, m=m)
    torch.cuda.synchronize()
    assert o.shape == (1, S, n_h, d) and o.dtype == torch.bfloat16
    for r0 in range(0, S, 1 << 16):  # row blocks: isfinite's temporaries of the whole 72 GiB output do not fit
        assert bool(torch.isfinite(o[0, r0:r0 + (1 << 16)]).all()), f"config[4]: non-finite output in rows {r0}+"
    _say("config[4] index rows: csa_topk_idxs S=1048576")
    rows_gpu = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m, seq_len=S)
    torch.cuda.synchronize()
    rng = np.random.default_rng(44)
    # compressed picks: recall of 256 sampled rows against the oracle's exact top-k
    prow = np.unique(np.concatenate([[3, 4, 4095, S - 1], rng.choice(S, 256, replace=False)]))
    sel = torch.as_tensor(prow, device=qi.device)
    lim = O.legal_limits(prow, T, m)
    sc = O.indexer_scores(bf16_bits(qi[0].index_select(0, sel)), bf16_bits(ki[0]),
                          w[0].index_select(0, sel).float().cpu().numpy(), np.arange(len(prow), dtype=np.int64),
                          lim=lim)
    ref_idx, _ = O.topk(sc, lim, top_k)
    got = rows_gpu[0].index_select(0, sel)[:, n_win:].long().cpu().numpy()
    assert np.array_equal(rows_gpu[0].index_select(0, sel)[:, :n_win].cpu().numpy(), O.window_idxs(prow, n_win))
    got = np.where(got >= 0, got - S, -1)
    rec = O.set_overlap_recall(ref_idx, got)
    assert rec.mean() >= 0.999 and rec.min() >= 0.99, f"config[4] recall {rec.mean():.5f} / min {rec.min():.4f}"
    del qi, ki, w
    # attention output of 32 sampled rows against the oracle over the same index rows
    arow = np.unique(np.concatenate([[0, 127, 128, S - 1], rng.choice(S, 32, replace=False)]))
    kv_full = torch.cat([kv, kvc], dim=1)
    ro, rl = _oracle_rows(q, kv_full, sink, rows_gpu, arow, d ** -0.5)
    sel = torch.as_tensor(arow, device=q.device)
    go = o[0].index_select(0, sel).float().cpu().numpy()
    oe = float(np.abs(go - ro).max())
    assert oe <= O_TOL, f"config[4]: o error {oe:.3e}"
    # the composition's attention equals sparse_attn_fwd over its index rows and row lengths
    rl_gpu = csa_row_len(1, S, n_win, top_k, T, m, q.device)
    o2, lse2 = sparse_attn_fwd(q[:, sel], kv_full, sink, rows_gpu[:, sel], d ** -0.5, row_len=rl_gpu[:, sel])
    torch.cuda.synchronize()
    assert torch.equal(o2[0], o[0].index_select(0, sel)), "composition != sparse_attn_fwd over its rows"
    assert float(np.abs(lse2[0].cpu().numpy() - rl).max()) <= LSE_TOL * max(1.0, float(np.abs(rl).max()))
    _say(f"config[4] recall {rec.mean():.5f} (min {rec.min():.4f}) on {len(prow)} rows; max |o err| {oe:.2e} "
         f"on {len(arow)} rows")
    del q, kv, kvc, sink, o, rows_gpu, kv_full, o2, lse2
    torch.cuda.empty_cache()
