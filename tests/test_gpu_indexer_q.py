"""GPU parity of the quantised-input indexer (fp4 queries, fp8 keys).

The oracle scores the dequantised inputs exactly: e2m1 values times
power-of-two scales and e4m3 values are all bf16-representable, so
I(s, t) = k_scale[t] * oracle_indexer_scores(q_deq, k_e4m3, w) in double,
and the GPU result goes through the same gate as the bf16 indexer
(tests/indexer_check.py: padding, order, scores within 1e-4, exact sets
wherever the k-th gap exceeds 1e-4 of the row scale, recall >= 0.999).
Shapes: the reference tests' ragged ones (S=47, T=73), causal ratio 4 and an
explicit mask, rows with no legal key, H_I = 16 / 40 / 64, top_k up to
1024, rows long enough to compact the selection buffer several times, and the
quantising wrapper on bf16 inputs.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import chunked_indexer_topk_quantized, indexer_topk_q, quant, synth
from tests.conftest import bf16_bits
from tests.indexer_check import check_rows

pytestmark = pytest.mark.gpu


def _dequant_bits(q4, qs, k8):
    """bf16 bit patterns of the dequantised q and of the raw e4m3 key values."""
    qv = O.fp4_unpack(q4.cpu().numpy()) * np.repeat(qs.cpu().numpy(), 32, axis=-1)
    qb = O.f32_to_bf16_bits(qv.astype(np.float32))
    assert np.array_equal(O.bf16_bits_to_f64(qb), qv), "dequantised q must be bf16-exact"
    kv = k8.float().cpu().numpy()
    return qb, O.f32_to_bf16_bits(kv)


def _check(q4, qs, k8, ks, w, top_k, idx, sc, *, ratio=None, mask=None, rows=None, label=""):
    B, S = q4.shape[:2]
    T = k8.shape[1]
    qb, kb = _dequant_bits(q4, qs, k8)
    rows = np.arange(S, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
    ksn = ks.reshape(B, T).cpu().numpy().astype(np.float64)
    out = []
    for b in range(B):
        lim = O.legal_limits(rows, T, ratio)
        ref = O.indexer_scores(qb[b], kb[b], w[b].float().cpu().numpy(), rows, lim=lim) * ksn[b][None, :]
        mrows = None if mask is None else mask[b].cpu().numpy().astype(np.uint8)[rows]
        out.append(check_rows(ref, lim, top_k, idx[b].cpu().numpy()[rows], sc[b].cpu().numpy()[rows], mrows,
                              label=f"{label}[b={b}]"))
    return out


def _inputs(B, S, T, H, seed):
    q, k, w = synth.indexer_inputs(B, S, H, 128, T, seed=seed)
    q4, qs = quant.fp4_act_quant(q, 32)
    k8, ks = quant.act_quant(k, 128)
    return q, k, w, q4, qs, k8, ks


@pytest.mark.parametrize("H,top_k", [(64, 64), (16, 32), (40, 200)])
def test_causal_ratio(cuda_device, H, top_k):
    # two batches of 603 rows: each batch's last eight-row workgroup holds
    # three rows
    B, S, T = 2, 603, 150
    _, _, w, q4, qs, k8, ks = _inputs(B, S, T, H, 11 + H)
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, top_k, causal_ratio=4)
    torch.cuda.synchronize()
    _check(q4, qs, k8, ks, w, top_k, idx, sc, ratio=4, label=f"q-ratio H{H}")


def test_ragged_no_bound_and_mask(cuda_device):
    # tests/test_chunked_indexer.py:51-72 shapes (S=47, T=73)
    B, S, T, H = 1, 47, 73, 64
    _, _, w, q4, qs, k8, ks = _inputs(B, S, T, H, 5)
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, 16)
    _check(q4, qs, k8, ks, w, 16, idx, sc, label="q-nobound")
    g = torch.Generator().manual_seed(5)
    mask = (torch.rand(B, S, T, generator=g) < 0.3).cuda()
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, 16, causal_mask=mask)
    _check(q4, qs, k8, ks, w, 16, idx, sc, mask=mask, label="q-mask")
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, 128)   # top_k > T: padding
    _check(q4, qs, k8, ks, w, 128, idx, sc, label="q-wide")


def test_large_topk_sampled_rows(cuda_device):
    B, S, T, H = 1, 8192, 2048, 64
    _, _, w, q4, qs, k8, ks = _inputs(B, S, T, H, 21)
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, 1024, causal_ratio=4)
    rows = np.random.default_rng(0).choice(S, 96, replace=False)
    rows[:3] = [0, 2, S - 1]   # no legal key, no legal key, full row
    _check(q4, qs, k8, ks, w, 1024, idx, sc, ratio=4, rows=rows, label="q-1024")


@pytest.mark.parametrize("top_k", [32, 192, 193, 512, 640])
def test_compacting_rows(cuda_device, top_k):
    # top_k <= 32, (32, 192] and (192, 512] run the 256-, 512- and 960-key
    # selection buffers with eight rows per workgroup, (512, 640] the
    # 1152-key one with four; rows of up to 4096 keys compact them several
    # times.  S = 8189 leaves the last (first scheduled) workgroup with five
    # active rows.
    B, S, T, H = 1, 8189, 4096, 64
    _, _, w, q4, qs, k8, ks = _inputs(B, S, T, H, 31 + top_k)
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, top_k, causal_ratio=2)
    rows = np.random.default_rng(top_k).choice(S, 40, replace=False)
    rows[:3] = [S - 1, S - 2, 2 * top_k]   # the longest rows, and one just past top_k legal keys
    _check(q4, qs, k8, ks, w, top_k, idx, sc, ratio=2, rows=rows, label=f"q-compact-{top_k}")


@pytest.mark.parametrize("zero_q", [False, True])
def test_mass_ties_through_compactions(cuda_device, zero_q):
    # 6,000 keys made of 7 distinct rows repeated (identical fp8 rows and
    # scales): every score is shared by ~857 keys, so the compactions set their
    # floors by the 64-bit (score, index) bisection; with q = 0 every score is
    # +0 and the picks are the top_k smallest indices.  Exact order against the
    # dequantised-input oracle (score desc, index asc).
    B, S, T, H, top_k = 1, 24, 6000, 64, 512
    g = torch.Generator().manual_seed(4242)
    base = torch.randn(7, 128, generator=g).to(torch.bfloat16)
    k = base.repeat(T // 7 + 1, 1)[:T].unsqueeze(0).cuda()
    q = torch.randn(B, S, H, 128, generator=g).to(torch.bfloat16)
    if zero_q:
        q.zero_()
    q = q.cuda()
    w = torch.randn(B, S, H, generator=g).cuda()
    q4, qs = quant.fp4_act_quant(q, 32)
    k8, ks = quant.act_quant(k, 128)
    idx, sc = indexer_topk_q(q4, qs, k8, ks, w, top_k)
    torch.cuda.synchronize()
    qb, kb = _dequant_bits(q4, qs, k8)
    ref = O.indexer_scores(qb[0], kb[0], w[0].cpu().numpy(), np.arange(S)) * ks.reshape(B, T).cpu().numpy()[0][None, :]
    ridx, _ = O.topk(ref, np.full(S, T, dtype=np.int64), top_k)
    assert np.array_equal(idx[0].cpu().numpy(), ridx)
    if zero_q:
        assert np.array_equal(ridx, np.tile(np.arange(top_k), (S, 1)))


def test_quantising_wrapper_and_validation(cuda_device):
    B, S, T, H = 1, 256, 64, 64
    q, k, w, q4, qs, k8, ks = _inputs(B, S, T, H, 3)
    idx, sc = chunked_indexer_topk_quantized(q, k, w, 32, causal_ratio=4)
    idx2, sc2 = indexer_topk_q(q4, qs, k8, ks, w, 32, causal_ratio=4)
    assert torch.equal(idx, idx2) and torch.equal(sc, sc2)
    with pytest.raises(ValueError):
        indexer_topk_q(q4, qs * 3.0, k8, ks, w, 32)   # not powers of two
    with pytest.raises(ValueError):
        indexer_topk_q(q4, qs, k8, ks, w, 4096)


def test_csa_rows_and_forward_quantized(cuda_device):
    from streamindex_amd import csa_topk_idxs, flash_csa_forward, sparse_attn

    B, S, H, n_win, top_k, m = 1, 512, 64, 32, 48, 4
    T = S // m
    _, _, w, q4, qs, k8, ks = _inputs(B, S, T, H, 17)
    q, k, _ = synth.indexer_inputs(B, S, H, 128, T, seed=17)
    rows, sc = csa_topk_idxs(q, k, w, n_win=n_win, top_k=top_k, m=m, return_scores=True, quantized=True)
    torch.cuda.synchronize()
    ref_win = O.window_idxs(np.arange(S, dtype=np.int64), n_win)
    assert np.array_equal(rows[0, :, :n_win].cpu().numpy(), ref_win)
    picks = rows[..., n_win:].long()
    picks = torch.where(picks >= 0, picks - S, picks)
    _check(q4, qs, k8, ks, w, top_k, picks, sc, ratio=m, label="csa-q")
    # the forward over those rows equals sparse attention over [kv ; kv_compressed]
    qa, kv, sink = synth.sparse_attn_inputs(B, S, 16, 64, S, seed=18)
    kvc = kv[:, :T].contiguous()
    o = flash_csa_forward(qa, kv, kvc, q, k, w, sink, n_win=n_win, top_k=top_k, m=m, quantized_indexer=True)
    o2 = sparse_attn(qa, torch.cat([kv, kvc], 1), sink, rows)
    assert torch.equal(o, o2)
