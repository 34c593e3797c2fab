"""GPU parity of the sparse-attention backward against the CPU oracle.

Cases mirror tests/test_triton_sparse_attn_bwd.py:78-188 of the reference
(end-to-end, dq-only, dkv-only, dsink-only and partial-masking shapes, all
through autograd) plus every supported D, H > 64 (two head groups), ragged K,
int64 indices, duplicate and out-of-range keys, chunked workspaces, empty
cases and the V4 shape D = 576 with sampled keys.

The oracle (oracle.sparse_attn_bwd_rows, double precision) takes the same
saved o (bf16) and lse (fp32) as the kernel.  Tolerances: the kernel rounds
P and dS to bf16 before the products (as the reference does), each
per-(query, slot) dkv row to bf16 before the fp32 key sum, and dq / dkv to
bf16 at the end, so for dq and dkv:
    ||got - ref||_F <= 1e-2 ||ref||_F   and   max|got - ref| <= 2e-2 max|ref|;
dsink is an fp32 sum of exact products: |got - ref| <= 1e-4 sum|terms| + 1e-6.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import sparse_attn, sparse_attn_bwd, sparse_attn_fwd, synth
from tests.conftest import bf16_bits

pytestmark = pytest.mark.gpu

REL_F = 1e-2
REL_MAX = 2e-2


def _close(got: np.ndarray, ref: np.ndarray, label: str):
    assert np.isfinite(got).all(), f"{label}: non-finite values"
    nref = np.linalg.norm(ref)
    err = np.linalg.norm(got - ref)
    assert err <= REL_F * nref + 1e-6, f"{label}: relative Frobenius error {err / max(nref, 1e-30):.3e}"
    mx = np.abs(got - ref).max() if got.size else 0.0
    assert mx <= REL_MAX * np.abs(ref).max() + 1e-6, f"{label}: max error {mx:.3e} vs max|ref| {np.abs(ref).max():.3e}"


def _inputs(B, S, H, D, N, K, seed, *, mask_every=5, oob=True, i64=False, masked_rows=False):
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=seed, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(seed)
    idx = torch.randint(0, max(N, 1), (B, S, K), generator=g, dtype=torch.int64)
    if mask_every > 0 and K > 0:
        idx[:, :, ::mask_every] = -1
    if oob and K > 2:
        idx[:, 1::3, 2] = N + 3  # out of range: masked like -1
    if masked_rows:
        idx[:, ::2] = -1  # rows with every index masked
    idx = idx.to(torch.int64 if i64 else torch.int32).cuda()
    do = (torch.randn(B, S, H, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
    return q, kv, sink, idx, do


def _oracle(q, kv, sink, idx, o, lse, do, scale, *, keys=None, rows=None):
    """Oracle gradients per batch: (dq [B,..] or rows subset, dkv [B,N|keys,D], dsink [H])."""
    B = q.shape[0]
    dqs, dkvs = [], []
    dsink = np.zeros(q.shape[2])
    for b in range(B):
        qb, ob, gb = bf16_bits(q[b]), bf16_bits(o[b]), bf16_bits(do[b])
        ib = idx[b].cpu().numpy().astype(np.int64)
        lb = lse[b].cpu().numpy()
        kb = bf16_bits(kv[b])
        sk = sink.cpu().numpy()
        if keys is None and rows is None:
            dq, dkv, ds = O.sparse_attn_bwd_rows(qb, kb, ob, gb, sk, lb, ib, scale)
            dqs.append(dq)
            dkvs.append(dkv)
            dsink += ds
        else:
            _, _, ds = O.sparse_attn_bwd_rows(qb, kb, ob, gb, sk, lb, ib, scale, want_dq=False, want_dkv=False)
            dsink += ds
            if rows is not None:
                dq, _, _ = O.sparse_attn_bwd_rows(qb[rows], kb, ob[rows], gb[rows], sk, lb[rows], ib[rows], scale,
                                                  want_dkv=False)
                dqs.append(dq)
            if keys is not None:
                sel = np.nonzero(np.isin(ib, keys).any(axis=1))[0]
                _, dkv, _ = O.sparse_attn_bwd_rows(qb[sel], kb, ob[sel], gb[sel], sk, lb[sel], ib[sel], scale,
                                                   keys=keys, want_dq=False)
                dkvs.append(dkv)
    return dqs, dkvs, dsink


def _dsink_bound(o, do, sink, lse):
    delta = (o.float() * do.float()).sum(-1)
    terms = torch.exp(sink.view(1, 1, -1) - lse) * delta
    return 1e-4 * terms.abs().sum(dim=(0, 1)).cpu().numpy() + 1e-6


def _run_and_check(B, S, H, D, N, K, seed, *, i64=False, mask_every=5, workspace_bytes=None, masked_rows=False,
                   label=""):
    q, kv, sink, idx, do = _inputs(B, S, H, D, N, K, seed, mask_every=mask_every, i64=i64, masked_rows=masked_rows)
    scale = D ** -0.5
    o, lse = sparse_attn_fwd(q, kv, sink, idx, scale)
    dq, dkv, dsink = sparse_attn_bwd(q, kv, sink, idx, o, lse, do, scale, workspace_bytes=workspace_bytes)
    torch.cuda.synchronize()
    rdq, rdkv, rds = _oracle(q, kv, sink, idx, o, lse, do, scale)
    for b in range(B):
        _close(dq[b].float().cpu().numpy(), rdq[b], f"{label} dq[b={b}]")
        _close(dkv[b].float().cpu().numpy(), rdkv[b], f"{label} dkv[b={b}]")
    assert np.all(np.abs(dsink.cpu().numpy() - rds) <= _dsink_bound(o, do, sink, lse)), f"{label} dsink"
    return q, kv, sink, idx, do, o, lse, (dq, dkv, dsink)


@pytest.mark.parametrize("D,H,K,i64", [(64, 16, 64, False), (128, 64, 96, True), (576, 64, 64, False),
                                       (32, 16, 40, True), (256, 80, 70, False), (512, 16, 33, True),
                                       (128, 192, 64, False), (576, 192, 40, True), (64, 260, 50, False)])
def test_bwd_matches_oracle(cuda_device, D, H, K, i64):
    _run_and_check(2, 40, H, D, 200, K, seed=300 + D + H, i64=i64, label=f"D{D}H{H}K{K}")


@pytest.mark.parametrize("D,H,i64,ws", [(576, 64, False, None), (64, 80, True, 1 << 20)])
def test_bwd_row_len(cuda_device, D, H, i64, ws):
    # Per-row column counts (0, inside a tile, on a tile edge, past K, random):
    # bit-identical to the backward over the tail-masked rows (whose dead
    # tiles run but contribute nothing), and equal to the oracle over them;
    # the second case also runs in several workspace chunks.
    B, S, N, K = 2, 24, 150, 100
    q, kv, sink, idx, do = _inputs(B, S, H, D, N, K, seed=900 + D, i64=i64)
    g = torch.Generator().manual_seed(D + 1)
    rl = torch.randint(0, K + 20, (B, S), generator=g, dtype=torch.int32)
    rl[:, :6] = torch.tensor([0, 1, 31, 32, 33, K], dtype=torch.int32)
    rl = rl.cuda()
    scale = D ** -0.5
    col = torch.arange(K, device="cuda")
    masked = idx.masked_fill(col >= rl.unsqueeze(-1).long(), -1)
    o, lse = sparse_attn_fwd(q, kv, sink, idx, scale, row_len=rl)
    dq, dkv, dsink = sparse_attn_bwd(q, kv, sink, idx, o, lse, do, scale, row_len=rl, workspace_bytes=ws)
    dq2, dkv2, dsink2 = sparse_attn_bwd(q, kv, sink, masked, o, lse, do, scale, workspace_bytes=ws)
    torch.cuda.synchronize()
    assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2) and torch.equal(dsink, dsink2)
    rdq, rdkv, rds = _oracle(q, kv, sink, masked, o, lse, do, scale)
    for b in range(B):
        _close(dq[b].float().cpu().numpy(), rdq[b], f"row_len dq[b={b}]")
        _close(dkv[b].float().cpu().numpy(), rdkv[b], f"row_len dkv[b={b}]")
    assert np.all(np.abs(dsink.cpu().numpy() - rds) <= _dsink_bound(o, do, sink, lse))


def test_reference_shapes_through_autograd(cuda_device):
    # tests/test_triton_sparse_attn_bwd.py:78-97 (seed 200, every 4th masked) and
    # :166-188 (B=2, every 3rd masked), gradients through torch.autograd
    for (B, S, H, D, N, K, every) in [(1, 32, 16, 64, 128, 64, 4), (2, 64, 16, 64, 256, 64, 3)]:
        q, kv, sink, idx, do = _inputs(B, S, H, D, N, K, 200 + every, mask_every=every, oob=False)
        qr, kvr, sr = (t.clone().requires_grad_(True) for t in (q, kv, sink))
        o = sparse_attn(qr, kvr, sr, idx, D ** -0.5)
        o.backward(do)
        o2, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
        assert torch.equal(o.detach(), o2)
        dq, dkv, ds = sparse_attn_bwd(q, kv, sink, idx, o2, lse, do, D ** -0.5)
        assert torch.equal(qr.grad, dq) and torch.equal(kvr.grad, dkv) and torch.equal(sr.grad, ds)
        rdq, rdkv, rds = _oracle(q, kv, sink, idx, o2, lse, do, D ** -0.5)
        for b in range(B):
            _close(dq[b].float().cpu().numpy(), rdq[b], "ref-shape dq")
            _close(dkv[b].float().cpu().numpy(), rdkv[b], "ref-shape dkv")
        assert np.all(np.abs(ds.cpu().numpy() - rds) <= _dsink_bound(o2, do, sink, lse))


def test_bwd_deterministic(cuda_device):
    q, kv, sink, idx, do = _inputs(1, 64, 64, 128, 96, 128, 41)
    o, lse = sparse_attn_fwd(q, kv, sink, idx)
    a = sparse_attn_bwd(q, kv, sink, idx, o, lse, do)
    b = sparse_attn_bwd(q, kv, sink, idx, o, lse, do)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_bwd_chunked_workspace(cuda_device):
    B, S, H, D, N, K = 2, 48, 64, 128, 150, 64
    from streamindex_amd import _lib
    one_row = _lib.load().si_sparse_attn_bwd_workspace_bytes(B, S, H, D, N, K, 0)
    assert one_row > 0
    # room for a handful of rows per chunk: many chunks, with a ragged last one
    _, _, _, _, _, _, _, chunked = _run_and_check(B, S, H, D, N, K, 77, workspace_bytes=int(one_row * 5),
                                                  label="chunked")
    _, _, _, _, _, _, _, whole = _run_and_check(B, S, H, D, N, K, 77, label="whole")
    assert torch.equal(chunked[0], whole[0])  # dq does not depend on the chunking
    with pytest.raises(ValueError):
        q, kv, sink, idx, do = _inputs(B, S, H, D, N, K, 77)
        o, lse = sparse_attn_fwd(q, kv, sink, idx)
        from streamindex_amd import _lib as L
        ws = torch.empty(16, dtype=torch.uint8, device="cuda")
        dq = torch.empty_like(q)
        dkv = torch.empty_like(kv)
        dsink = torch.empty_like(sink)
        rc = L.load().si_sparse_attn_bwd(
            q.data_ptr(), L.strides(q), kv.data_ptr(), L.strides(kv), sink.data_ptr(), idx.data_ptr(), 0,
            L.strides(idx), o.data_ptr(), L.strides(o), lse.data_ptr(), L.strides(lse), do.data_ptr(), L.strides(do),
            B, S, H, D, N, K, D ** -0.5, 0, dq.data_ptr(), L.strides(dq), dkv.data_ptr(), L.strides(dkv),
            dsink.data_ptr(), ws.data_ptr(), 16, L.stream_ptr(q.device))
        L.check(rc)


def test_bwd_empty_cases(cuda_device):
    H, D = 16, 64
    for (S, N, K) in [(8, 32, 0), (8, 0, 16)]:
        q, kv, sink, _, do = _inputs(1, S, H, D, max(N, 1), 1, 5)
        kv = kv[:, :N].contiguous()
        idx = torch.full((1, S, K), -1, dtype=torch.int32, device="cuda")
        o, lse = sparse_attn_fwd(q, kv, sink, idx)
        dq, dkv, ds = sparse_attn_bwd(q, kv, sink, idx, o, lse, do)
        torch.cuda.synchronize()
        assert dq.float().abs().max().item() == 0.0
        assert dkv.shape == (1, N, D) and (N == 0 or dkv.float().abs().max().item() == 0.0)
        assert ds.abs().max().item() == 0.0  # o = 0, so delta = 0
    # rows with every index masked contribute nothing to dq / dkv
    _run_and_check(1, 24, H, D, 64, 32, 6, masked_rows=True, label="half-masked")


def test_bwd_no_query_rows_zeroes_dkv(cuda_device):
    """S = 0 with keys and slots present: dkv must come back as zeros (the
    reference's fp32 accumulator starts at zero), not as whatever the output
    buffer held.  dkv is pre-filled with NaN and passed through the C ABI."""
    from streamindex_amd import _lib as L

    H, D, N, K = 16, 64, 32, 16
    q = torch.empty((1, 0, H, D), dtype=torch.bfloat16, device="cuda")
    kv = torch.randn((1, N, D), device="cuda").to(torch.bfloat16)
    sink = torch.zeros(H, dtype=torch.float32, device="cuda")
    idx = torch.empty((1, 0, K), dtype=torch.int32, device="cuda")
    o, do, dq = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    lse = torch.empty((1, 0, H), dtype=torch.float32, device="cuda")
    dkv = torch.full_like(kv, float("nan"))
    dsink = torch.full_like(sink, float("nan"))
    lib = L.load()
    need = lib.si_sparse_attn_bwd_workspace_bytes(1, 0, H, D, N, K, 1 << 30)
    ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device="cuda")
    rc = lib.si_sparse_attn_bwd(
        q.data_ptr(), L.strides(q), kv.data_ptr(), L.strides(kv), sink.data_ptr(), idx.data_ptr(), 0,
        L.strides(idx), o.data_ptr(), L.strides(o), lse.data_ptr(), L.strides(lse), do.data_ptr(), L.strides(do),
        1, 0, H, D, N, K, D ** -0.5, 0, dq.data_ptr(), L.strides(dq), dkv.data_ptr(), L.strides(dkv),
        dsink.data_ptr(), ws.data_ptr(), ws.numel(), L.stream_ptr(q.device))
    L.check(rc)
    torch.cuda.synchronize()
    assert torch.equal(dkv, torch.zeros_like(dkv))
    assert torch.equal(dsink, torch.zeros_like(dsink))
    # the Python wrapper returns the same
    _, dkv2, ds2 = sparse_attn_bwd(q, kv, sink, idx, o, lse, do)
    assert torch.equal(dkv2, torch.zeros_like(dkv2)) and torch.equal(ds2, torch.zeros_like(ds2))


def test_bwd_v4_shape_sampled(cuda_device):
    """D = 576, H = 64, K = 512 causal indices over N = S/4 keys: dq on
    sampled rows, dkv on sampled keys (every selecting row), dsink in full."""
    S, H, D, K = 2048, 64, 576, 512
    N = S // 4
    q, kv, sink = synth.sparse_attn_inputs(1, S, H, D, N, seed=2027)
    idx = synth.causal_random_topk(1, S, K, 4, seed=9)
    g = torch.Generator().manual_seed(9)
    do = torch.randn(1, S, H, D, generator=g).to(torch.bfloat16).cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx)
    dq, dkv, dsink = sparse_attn_bwd(q, kv, sink, idx, o, lse, do)
    torch.cuda.synchronize()
    rows = np.array([3, 400, 1025, 2047])
    keys = np.array([0, 7, 255, 511])
    rdq, rdkv, rds = _oracle(q, kv, sink, idx, o, lse, do, D ** -0.5, keys=keys, rows=rows)
    _close(dq[0, rows].float().cpu().numpy(), rdq[0], "v4 dq rows")
    _close(dkv[0, keys].float().cpu().numpy(), rdkv[0], "v4 dkv keys")
    assert np.all(np.abs(dsink.cpu().numpy() - rds) <= _dsink_bound(o, do, sink, lse))


def test_inverted_topk_correctness(cuda_device):
    # tests/test_inverted_topk.py:18-67 (distinct picks per query, every 4th slot masked)
    from streamindex_amd import build_inverted_topk

    B, S, K, N, K_MAX = 2, 32, 8, 64, 32
    g = torch.Generator().manual_seed(600)
    idx = torch.stack([torch.randperm(N, generator=g)[:K] for _ in range(B * S)]).reshape(B, S, K).int()
    idx[:, :, ::4] = -1
    idx[0, 3, 1] = N + 5   # out of range: ignored
    inv, cnt = build_inverted_topk(idx.cuda(), n_kv=N, k_max=K_MAX)
    inv, cnt = inv.cpu().numpy(), cnt.cpu().numpy()
    ic = idx.numpy()
    for b in range(B):
        for t in range(N):
            qs = [s for s in range(S) for j in range(K) if ic[b, s, j] == t]
            assert cnt[b, t] == len(qs)
            assert list(inv[b, t, :len(qs)]) == qs          # ascending (query, slot) order
            assert np.all(inv[b, t, len(qs):] == -1)


def test_inverted_topk_counts_overflow(cuda_device):
    # tests/test_inverted_topk.py:70-95: counts are not clamped to k_max
    from streamindex_amd import build_inverted_topk

    B, S, K, N, K_MAX = 1, 64, 4, 16, 8
    g = torch.Generator().manual_seed(601)
    idx = torch.zeros((B, S, K), dtype=torch.int32)
    idx[:, :, 1:] = torch.randint(1, N, (B, S, K - 1), generator=g, dtype=torch.int32)
    inv, cnt = build_inverted_topk(idx.cuda(), n_kv=N, k_max=K_MAX)
    assert cnt[0, 0].item() == 64
    assert list(inv[0, 0].cpu().numpy()) == list(range(K_MAX))


def test_bwd_v2_matches_v1(cuda_device):
    # tests/test_triton_sparse_attn_bwd_v2.py:46-100 (including H > 64)
    from streamindex_amd import sparse_attn_bwd_v2

    for (H, seed) in [(16, 700), (128, 702)]:
        q, kv, sink, idx, do = _inputs(1, 32, H, 64, 64, 16, seed)
        o, lse = sparse_attn_fwd(q, kv, sink, idx)
        a = sparse_attn_bwd(q, kv, sink, idx, o, lse, do)
        b = sparse_attn_bwd_v2(q, kv, sink, idx, o, lse, do, block_q=4, k_max=8)
        for x, y in zip(a, b):
            assert torch.equal(x, y)
        rdq, rdkv, _ = _oracle(q, kv, sink, idx, o, lse, do, 64 ** -0.5)
        _close(b[0][0].float().cpu().numpy(), rdq[0], f"v2 dq H{H}")
        _close(b[1][0].float().cpu().numpy(), rdkv[0], f"v2 dkv H{H}")
