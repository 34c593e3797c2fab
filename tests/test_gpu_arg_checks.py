"""Argument checks that must fire before any kernel launch: a tensor on the
host (or another device) or a causal mask of the wrong shape would otherwise
hand the kernel a pointer it cannot read.  The reference asserts ``is_cuda``
and shapes in the same places (``chunked_indexer.py:79-86``,
``sparse_attn_fwd.py:205-215``)."""

from __future__ import annotations

import pytest
import torch

from streamindex_amd import indexer_topk_q, quant, sparse_attn_bwd, sparse_attn_fwd, synth

pytestmark = pytest.mark.gpu


def _attn():
    q, kv, sink = synth.sparse_attn_inputs(1, 8, 16, 64, 32, seed=3)
    idx = synth.causal_random_topk(1, 8, 8, 1, seed=4)
    o, lse = sparse_attn_fwd(q, kv, sink, idx)
    do = torch.randn_like(q)
    row_len = torch.full((1, 8), 8, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    return dict(q=q, kv=kv, attn_sink=sink, topk_idxs=idx, o=o, lse=lse, do=do, row_len=row_len)


@pytest.mark.parametrize("name", ["attn_sink", "topk_idxs", "row_len"])
def test_fwd_rejects_host_tensors(cuda_device, name):
    a = _attn()
    a[name] = a[name].cpu()
    with pytest.raises(AssertionError):
        sparse_attn_fwd(a["q"], a["kv"], a["attn_sink"], a["topk_idxs"], row_len=a["row_len"])


@pytest.mark.parametrize("name", ["attn_sink", "topk_idxs", "o", "lse", "do", "row_len"])
def test_bwd_rejects_host_tensors(cuda_device, name):
    a = _attn()
    a[name] = a[name].cpu()
    with pytest.raises(AssertionError):
        sparse_attn_bwd(a["q"], a["kv"], a["attn_sink"], a["topk_idxs"], a["o"], a["lse"], a["do"],
                        row_len=a["row_len"])


def _q_inputs():
    q, k, w = synth.indexer_inputs(1, 64, 16, 128, ratio=4, seed=5)
    q4, qs = quant.fp4_act_quant(q, 32)
    k8, ks = quant.act_quant(k, 128)
    return q4, qs, k8, ks, w


def test_quantized_indexer_rejects_bad_masks(cuda_device):
    q4, qs, k8, ks, w = _q_inputs()
    B, S, T = 1, 64, 16
    good = torch.ones((B, S, T), dtype=torch.bool, device="cuda")
    idx, _ = indexer_topk_q(q4, qs, k8, ks, w, 8, causal_mask=good)
    torch.cuda.synchronize()
    assert idx.shape == (B, S, 8)
    for bad in (torch.ones((B, S, T - 1), dtype=torch.bool, device="cuda"),   # too few keys
                torch.ones((B, S + 1, T), dtype=torch.bool, device="cuda"),   # too many rows
                good.cpu()):                                                   # host memory
        with pytest.raises(AssertionError):
            indexer_topk_q(q4, qs, k8, ks, w, 8, causal_mask=bad)
    with pytest.raises(AssertionError):  # mask and ratio are exclusive
        indexer_topk_q(q4, qs, k8, ks, w, 8, causal_mask=good, causal_ratio=4)
    with pytest.raises(AssertionError):  # scales on the host
        indexer_topk_q(q4, qs.cpu(), k8, ks, w, 8, causal_ratio=4)


def test_indexer_rejects_bad_masks(cuda_device):
    from streamindex_amd import chunked_indexer_topk, indexer_score_topk

    q, k, w = synth.indexer_inputs(1, 64, 16, 64, ratio=4, seed=6)
    bad = torch.ones((1, 64, 15), dtype=torch.bool, device="cuda")
    with pytest.raises(AssertionError):
        chunked_indexer_topk(q, k, w, 8, causal_mask=bad)
    with pytest.raises(AssertionError):
        indexer_score_topk(q, k, w, 8, causal_mask=bad)
    with pytest.raises(AssertionError):
        indexer_score_topk(q, k, w.cpu(), 8)
