"""The no-alloc backward (si_sparse_attn_bwd_noalloc) against the backward
with a caller-provided workspace (si_sparse_attn_bwd_ragged), through the C
ABI: bit-identical outputs on two calls in a row (the second smaller), a
problem that the static scratch has to process in row chunks, and the
rejection of a problem whose smallest workspace exceeds the scratch."""

from __future__ import annotations

import pytest
import torch

from streamindex_amd import _lib as L
from streamindex_amd import sparse_attn_fwd, synth

pytestmark = pytest.mark.gpu


def _problem(B, S, H, D, N, K, seed, ragged):
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=seed)
    idx = torch.stack([synth.causal_random_topk(1, S, K, 1, seed=seed + b)[0] for b in range(B)])
    idx = torch.where(idx >= 0, idx % N, idx)  # repeats allowed: keys selected by several slots
    idx[:, :, ::7] = -1
    g = torch.Generator().manual_seed(seed)
    do = torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).cuda()
    row_len = None
    if ragged:
        row_len = torch.randint(0, K + 1, (B, S), generator=g, dtype=torch.int32).cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, row_len=row_len)
    torch.cuda.synchronize()
    return q, kv, sink, idx, o, lse, do, row_len


def _outs(q, kv):
    B, S, H, D = q.shape
    dq = torch.full_like(q, float("nan"))
    dkv = torch.full_like(kv, float("nan"))
    dsink = torch.full((H,), float("nan"), dtype=torch.float32, device=q.device)
    return dq, dkv, dsink


def _args(p, outs):
    q, kv, sink, idx, o, lse, do, row_len = p
    dq, dkv, dsink = outs
    B, S, H, D = q.shape
    head = (q.data_ptr(), L.strides(q), kv.data_ptr(), L.strides(kv), sink.data_ptr(), idx.data_ptr(),
            1 if idx.dtype == torch.int64 else 0, L.strides(idx), o.data_ptr(), L.strides(o), lse.data_ptr(),
            L.strides(lse), do.data_ptr(), L.strides(do), B, S, H, D, kv.shape[1], idx.shape[2], D ** -0.5,
            1 if q.dtype == torch.float16 else 0, dq.data_ptr(), L.strides(dq), dkv.data_ptr(), L.strides(dkv),
            dsink.data_ptr())
    rl = (None, None) if row_len is None else (row_len.data_ptr(), L.strides(row_len))
    return head, rl


def _noalloc(p):
    outs = _outs(p[0], p[1])
    head, rl = _args(p, outs)
    lib = L.load()
    L.check(lib.si_sparse_attn_bwd_noalloc(*head, *rl, L.stream_ptr(p[0].device)))
    return outs


def _with_workspace(p, ws_bytes):
    outs = _outs(p[0], p[1])
    head, rl = _args(p, outs)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=p[0].device)
    lib = L.load()
    L.check(lib.si_sparse_attn_bwd_ragged(*head, ws.data_ptr(), ws.numel(), *rl, L.stream_ptr(p[0].device)))
    return outs


def test_noalloc_backward_matches_workspace_backward(cuda_device):
    lib = L.load()
    cap = int(lib.si_sparse_attn_bwd_noalloc_scratch_bytes())
    assert cap == 128 << 20
    # 1) V4 attention dims, more rows than one scratch-sized chunk holds:
    #    the same chunk plan as the caller-workspace entry given `cap` bytes
    big = _problem(1, 1024, 64, 576, 512, 512, 21, ragged=False)
    whole = lib.si_sparse_attn_bwd_workspace_bytes(1, 1024, 64, 576, 512, 512, 1 << 40)
    assert whole > cap, "the first problem must need row chunks within the scratch"
    got = _noalloc(big)
    ref = _with_workspace(big, cap)
    torch.cuda.synchronize()
    for g, r, name in zip(got, ref, ("dq", "dkv", "dsink")):
        assert torch.equal(g, r), f"first call: {name} differs"
    # 2) a smaller problem right after it (ragged rows, int64 indices, B = 2):
    #    the scratch still holds the first call's data, nothing may leak through
    small = _problem(2, 40, 16, 64, 96, 48, 22, ragged=True)
    small = small[:3] + (small[3].long(),) + small[4:]
    got = _noalloc(small)
    ref = _with_workspace(small, 1 << 24)
    torch.cuda.synchronize()
    for g, r, name in zip(got, ref, ("dq", "dkv", "dsink")):
        assert torch.equal(g, r), f"second call: {name} differs"


def test_noalloc_rejects_problems_beyond_the_scratch(cuda_device):
    # S = 1M rows need 4 * S * 64 bytes of per-row dsink terms (256 MiB) even
    # one row per chunk: rejected before anything is launched
    lib = L.load()
    B, S, H, D, N, K = 1, 1 << 20, 1, 32, 64, 8
    q = torch.zeros(B, S, H, D, dtype=torch.bfloat16, device="cuda")
    kv = torch.zeros(B, N, D, dtype=torch.bfloat16, device="cuda")
    sink = torch.zeros(H, dtype=torch.float32, device="cuda")
    idx = torch.full((B, S, K), -1, dtype=torch.int32, device="cuda")
    lse = torch.zeros(B, S, H, dtype=torch.float32, device="cuda")
    p = (q, kv, sink, idx, q, lse, q, None)
    outs = _outs(q, kv)
    head, rl = _args(p, outs)
    rc = lib.si_sparse_attn_bwd_noalloc(*head, *rl, L.stream_ptr(q.device))
    assert rc == L.SI_ERR_UNSUPPORTED
    assert "no-alloc" in lib.si_last_error().decode()
