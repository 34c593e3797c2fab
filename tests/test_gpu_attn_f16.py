"""fp16 sparse attention: the reference accepts fp16 q / kv besides bf16
(``flash_sparse/triton/sparse_attn_fwd.py:193,207``; its output is
``torch.empty_like(q)``, :241, and P is cast to the kv dtype before P.V, :145).

Forward and backward run on fp16 operands (v_mfma_f32_16x16x32_f16) and are
checked against the oracle reading the same fp16 values (double precision):
|o - o_ref| <= 1e-2, |lse - lse_ref| <= 2e-3 (fp16 rounds P and o to 11
significant bits, half the bf16 gate); dq and dkv within 1e-2 relative
Frobenius and 2e-2 of max|ref|, as for bf16.  Large scores make the lazy
rescale of the running maximum fire, which for fp16 must keep P below the
fp16 maximum.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import sparse_attn, sparse_attn_bwd, sparse_attn_fwd

pytestmark = pytest.mark.gpu

O_TOL = 1e-2
LSE_TOL = 2e-3


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _inputs(B, S, H, D, N, K, seed, q_scale=0.5, kv_scale=0.5, i64=False, mask_every=5):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, S, H, D, generator=g) * q_scale).half().cuda()
    kv = (torch.randn(B, N, D, generator=g) * kv_scale).half().cuda()
    sink = torch.randn(H, generator=g).cuda()
    idx = torch.randint(0, N, (B, S, K), generator=g)
    if mask_every:
        idx[:, :, ::mask_every] = -1
    idx = idx.to(torch.int64 if i64 else torch.int32).cuda()
    return q, kv, sink, idx


def _check_fwd(q, kv, sink, idx, o, lse, scale, label):
    assert o.dtype == torch.float16 and o.shape == q.shape
    for b in range(q.shape[0]):
        ro, rl = O.sparse_attn_rows(_bits(q[b]), _bits(kv[b]), sink.cpu().numpy(),
                                    idx[b].cpu().numpy().astype(np.int64), scale, f16=True)
        go = o[b].float().cpu().numpy()
        assert np.isfinite(go).all(), f"{label}: non-finite output"
        oe = np.abs(go - ro).max()
        le = np.abs(lse[b].cpu().numpy() - rl).max()
        assert oe <= O_TOL * max(1.0, np.abs(ro).max()), f"{label}[b={b}]: o error {oe:.3e}"
        assert le <= LSE_TOL * max(1.0, np.abs(rl).max()), f"{label}[b={b}]: lse error {le:.3e}"


@pytest.mark.parametrize("D,H,K,i64,q_scale", [(64, 16, 96, False, 0.5), (64, 16, 64, True, 8.0),
                                               (576, 64, 160, False, 0.5), (576, 64, 96, True, 4.0),
                                               (128, 80, 50, False, 1.0)])
def test_fwd_f16_matches_oracle(cuda_device, D, H, K, i64, q_scale):
    q, kv, sink, idx = _inputs(2, 24, H, D, 300, K, 70 + D + K, q_scale=q_scale, i64=i64)
    scale = D ** -0.5
    o, lse = sparse_attn_fwd(q, kv, sink, idx, scale)
    torch.cuda.synchronize()
    _check_fwd(q, kv, sink, idx, o, lse, scale, f"D{D}H{H}K{K}x{q_scale}")


def test_fwd_f16_row_len_and_empty_rows(cuda_device):
    D, H, K = 576, 64, 128
    q, kv, sink, idx = _inputs(1, 16, H, D, 200, K, 81)
    idx[0, 3] = -1  # a row without valid keys: o = 0, lse = sink
    rl = torch.tensor([[0, 1, 31, 32, 33, K, 70, 5, 0, 96, 128, 127, 64, 65, 2, 100]], dtype=torch.int32).cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, row_len=rl)
    col = torch.arange(K, device="cuda")
    masked = idx.masked_fill(col >= rl.unsqueeze(-1).long(), -1)
    o2, lse2 = sparse_attn_fwd(q, kv, sink, masked)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert bool((o[0, 3] == 0).all()) and torch.allclose(lse[0, 3], sink)
    _check_fwd(q, kv, sink, masked, o, lse, D ** -0.5, "row_len")


def _close(got, ref, label):
    nref = np.linalg.norm(ref)
    assert np.linalg.norm(got - ref) <= 1e-2 * nref + 1e-6, f"{label}: relative Frobenius error"
    assert np.abs(got - ref).max() <= 2e-2 * np.abs(ref).max() + 1e-6, f"{label}: max error"


@pytest.mark.parametrize("D,H,K,i64", [(64, 16, 64, False), (576, 64, 64, True), (256, 80, 40, False)])
def test_bwd_f16_matches_oracle(cuda_device, D, H, K, i64):
    B, S, N = 2, 32, 150
    q, kv, sink, idx = _inputs(B, S, H, D, N, K, 90 + D, i64=i64)
    g = torch.Generator().manual_seed(D)
    do = (torch.randn(B, S, H, D, generator=g) * 0.5).half().cuda()
    scale = D ** -0.5
    o, lse = sparse_attn_fwd(q, kv, sink, idx, scale)
    dq, dkv, dsink = sparse_attn_bwd(q, kv, sink, idx, o, lse, do, scale)
    torch.cuda.synchronize()
    assert dq.dtype == torch.float16 and dkv.dtype == torch.float16 and dsink.dtype == torch.float32
    rds = np.zeros(H)
    for b in range(B):
        rdq, rdkv, ds = O.sparse_attn_bwd_rows(_bits(q[b]), _bits(kv[b]), _bits(o[b]), _bits(do[b]),
                                               sink.cpu().numpy(), lse[b].cpu().numpy(),
                                               idx[b].cpu().numpy().astype(np.int64), scale, f16=True)
        _close(dq[b].float().cpu().numpy(), rdq, f"f16 dq[b={b}]")
        _close(dkv[b].float().cpu().numpy(), rdkv, f"f16 dkv[b={b}]")
        rds += ds
    delta = (o.float() * do.float()).sum(-1)
    bound = 1e-4 * (torch.exp(sink.view(1, 1, -1) - lse) * delta).abs().sum(dim=(0, 1)).cpu().numpy() + 1e-6
    assert np.all(np.abs(dsink.cpu().numpy() - rds) <= bound)
    # deterministic like the bf16 path
    dq2, dkv2, dsink2 = sparse_attn_bwd(q, kv, sink, idx, o, lse, do, scale)
    assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2) and torch.equal(dsink, dsink2)


def test_f16_through_autograd(cuda_device):
    # the reference test shape (tests/test_triton_sparse_attn_bwd.py:78-97) in fp16
    q, kv, sink, idx = _inputs(1, 32, 16, 64, 128, 64, 200, mask_every=4)
    qr, kvr, sr = (t.clone().requires_grad_(True) for t in (q, kv, sink))
    o = sparse_attn(qr, kvr, sr, idx, 64 ** -0.5)
    do = torch.randn_like(o)
    o.backward(do)
    o2, lse = sparse_attn_fwd(q, kv, sink, idx, 64 ** -0.5)
    dq, dkv, ds = sparse_attn_bwd(q, kv, sink, idx, o2, lse, do, 64 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(o.detach(), o2)
    assert torch.equal(qr.grad, dq) and torch.equal(kvr.grad, dkv) and torch.equal(sr.grad, ds)


def test_mixed_dtypes_rejected(cuda_device):
    q, kv, sink, idx = _inputs(1, 4, 16, 64, 32, 8, 5)
    with pytest.raises(AssertionError):
        sparse_attn_fwd(q, kv.bfloat16(), sink, idx)
    with pytest.raises(AssertionError):
        sparse_attn_fwd(q.float(), kv.float(), sink, idx)
    o, lse = sparse_attn_fwd(q, kv, sink, idx)
    with pytest.raises(AssertionError):
        sparse_attn_bwd(q, kv, sink, idx, o, lse, q.bfloat16())
