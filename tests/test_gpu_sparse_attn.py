"""GPU parity of the sparse-attention forward kernel against the CPU oracle.

Cases mirror tests/test_triton_sparse_attn_fwd.py:70-129 and
tests/test_against_reference.py:109-177 (dense fall-through, random masking,
all-masked rows, masking == truncation) plus the V4 shape D=576, H=64.
Tolerance: |o - o_ref| <= 2e-2 (bf16 output), |lse - lse_ref| <= 2e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import sparse_attn, sparse_attn_fwd, synth
from tests.conftest import bf16_bits

pytestmark = pytest.mark.gpu

O_TOL = 2e-2
LSE_TOL = 2e-3


def _check(q, kv, sink, idx, scale, o, lse, label=""):
    B = q.shape[0]
    for b in range(B):
        ro, rl = O.sparse_attn_rows(bf16_bits(q[b]), bf16_bits(kv[b]), sink.cpu().numpy(),
                                    idx[b].cpu().numpy().astype(np.int64), scale)
        go = o[b].float().cpu().numpy()
        gl = lse[b].cpu().numpy()
        assert np.isfinite(go).all(), f"{label}: non-finite output"
        oe = np.abs(go - ro).max()
        le = np.abs(gl - rl).max()
        assert oe <= O_TOL, f"{label}[b={b}]: o error {oe:.3e}"
        assert le <= LSE_TOL * max(1.0, np.abs(rl).max()), f"{label}[b={b}]: lse error {le:.3e}"


def test_dense_fallthrough(cuda_device):
    # tests/test_triton_sparse_attn_fwd.py:70-86
    B, S, H, D, N = 1, 16, 16, 64, 64
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=100, q_scale=0.5, kv_scale=0.5)
    idx = torch.arange(N, device="cuda").view(1, 1, N).expand(B, S, N).contiguous().int()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, D ** -0.5, o, lse, "dense")
    # closed form: with every key selected this is softmax over (keys ∪ sink) in torch fp32
    s = torch.einsum("bshd,bnd->bshn", q.float(), kv.float()) * D ** -0.5
    full = torch.cat([s, sink.view(1, 1, H, 1).expand(B, S, H, 1)], dim=-1).softmax(-1)[..., :N]
    ref = torch.einsum("bshn,bnd->bshd", full, kv.float())
    assert (o.float() - ref).abs().max().item() <= O_TOL


def test_random_masked(cuda_device):
    # tests/test_triton_sparse_attn_fwd.py:90-106 (every 4th index masked)
    B, S, H, D, N, K = 2, 32, 16, 64, 256, 64
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=101, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(101)
    idx = torch.randint(0, N, (B, S, K), generator=g, dtype=torch.int32)
    idx[:, :, ::4] = -1
    idx = idx.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, D ** -0.5, o, lse, "masked")


def test_all_masked_row(cuda_device):
    # tests/test_triton_sparse_attn_fwd.py:110-129: zero output, lse = sink
    B, S, H, D, N, K = 1, 8, 16, 32, 64, 16
    q, kv, _ = synth.sparse_attn_inputs(B, S, H, D, N, seed=102)
    sink = torch.zeros(H, dtype=torch.float32, device="cuda")
    g = torch.Generator().manual_seed(102)
    idx = torch.randint(0, N, (B, S, K), generator=g, dtype=torch.int32)
    idx[:, 0, :] = -1
    idx = idx.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    assert o[:, 0].float().abs().max().item() == 0.0
    assert torch.allclose(lse[:, 0], sink.view(1, H).expand(B, H))
    _check(q, kv, sink, idx, D ** -0.5, o, lse, "all-masked")


def test_masking_equals_truncation(cuda_device):
    # tests/test_against_reference.py:139-161: trailing -1 == shorter index list
    B, S, H, D, N = 1, 12, 16, 128, 100
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=103)
    g = torch.Generator().manual_seed(103)
    idx = torch.randint(0, N, (B, S, 40), generator=g)
    padded = torch.cat([idx, torch.full((B, S, 24), -1, dtype=idx.dtype)], dim=-1).cuda()
    o1, l1 = sparse_attn_fwd(q, kv, sink, idx.cuda())
    o2, l2 = sparse_attn_fwd(q, kv, sink, padded)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


@pytest.mark.parametrize("D", [576, 128])
def test_reference_maximum_jumps(cuda_device, D):
    # Scores that rise by far more than the lazy threshold (2^64 in exp2 units)
    # in later tiles, twice: the softmax takes the path that reduces the tile
    # maximum over the lane groups, moves the reference and rescales the
    # accumulated output (alpha < 1) mid-row; the first tiles keep it fixed.
    B, S, H, N, K = 1, 6, 64, 320, 320
    g = torch.Generator().manual_seed(211 + D)
    u = torch.randn(D, generator=g) * 10.0
    q = (u + torch.randn(B, S, H, D, generator=g)).to(torch.bfloat16)
    kv = (torch.randn(B, N, D, generator=g) * 0.01)
    scale = D ** -0.5
    # key rows 256..287 score about 80 / scale (115 in exp2 units, past the
    # threshold of 64 over the cold keys' ~0), rows 288..319 about 200 / scale
    # (288: past it again); outputs stay below 8, where bf16 rounds by <= 2^-6
    kv[0, 256:288] = u * (80.0 / scale) / u.dot(u)
    kv[0, 288:320] = u * (200.0 / scale) / u.dot(u)
    kv = kv.to(torch.bfloat16)
    sink = torch.randn(H, generator=g)
    idx = torch.arange(K, dtype=torch.int32).repeat(B, S, 1)  # hot keys in tiles 8 and 9
    q, kv, sink, idx = q.cuda(), kv.cuda(), sink.cuda(), idx.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, scale)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, scale, o, lse, label=f"jumps D={D}")
    assert float(lse.min()) > 100.0  # the hot keys dominate every head


@pytest.mark.parametrize("D,i64", [(576, False), (128, True), (512, False)])
def test_fully_masked_tiles(cuda_device, D, i64):
    # Whole 32-key tiles of -1 (the first tile, tiles in the middle, the last
    # one, every tile of some rows) as HCA's causal tail produces them: the
    # result equals the oracle and, bit for bit, the same rows with those
    # tiles removed.
    B, S, H, N, K = 1, 16, 64, 400, 256
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=600 + D, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(D)
    dt = torch.int64 if i64 else torch.int32
    idx = torch.randint(0, N, (B, S, K), generator=g, dtype=dt)
    dead = [0, 3, 4, 7]
    for t in dead:
        idx[:, :, 32 * t:32 * t + 32] = -1
    idx[:, 5, :] = -1                  # every tile masked
    idx[:, 6, 32 * 5 + 7] = 17         # one valid key in an otherwise dead row
    idx[:, 6, :32 * 5 + 7] = -1
    idx[:, 6, 32 * 5 + 8:] = -1
    idx = idx.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, D ** -0.5, o, lse, f"dead tiles D={D}")
    assert o[:, 5].float().abs().max().item() == 0.0
    keep = torch.tensor([t for t in range(K // 32) if t not in dead])
    cols = (keep.view(-1, 1) * 32 + torch.arange(32)).flatten().cuda()
    rows = [r for r in range(S) if r not in (5, 6)]
    o2, l2 = sparse_attn_fwd(q[:, rows], kv, sink, idx[:, rows][:, :, cols].contiguous(), D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(o[:, rows], o2) and torch.equal(lse[:, rows], l2)


@pytest.mark.parametrize("D,H,B,S,K,i64", [(576, 64, 1, 700, 32, False), (576, 64, 2, 600, 96, True),
                                           (576, 80, 1, 400, 64, False), (128, 16, 1, 1000, 200, False),
                                           (512, 128, 1, 300, 160, True)])
def test_many_rows(cuda_device, D, H, B, S, K, i64):
    # More query rows than compute units, with 1, 3, 2, 7 and 5 key tiles per
    # row, two head groups (full and partial), H < 64, B = 2 and int64
    # indices.  Sampled rows (first, last and spread) against the oracle; some
    # rows fully masked.
    N = 300
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=700 + D + H, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(S + K)
    idx = torch.randint(-1, N, (B, S, K), generator=g, dtype=torch.int64 if i64 else torch.int32)
    idx[:, 3::17, :] = -1
    idx = idx.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, S, max(1, S // 23)), [0, 1, 3, S - 2, S - 1]]))
    rows = rows[rows < S]
    for b in range(B):
        sel = torch.from_numpy(rows).cuda()
        ro, rl = O.sparse_attn_rows(bf16_bits(q[b, sel]), bf16_bits(kv[b]), sink.cpu().numpy(),
                                    idx[b, sel].cpu().numpy().astype(np.int64), D ** -0.5)
        go = o[b, sel].float().cpu().numpy()
        gl = lse[b, sel].cpu().numpy()
        assert np.isfinite(go).all()
        assert np.abs(go - ro).max() <= O_TOL, f"b={b}: o error {np.abs(go - ro).max():.3e}"
        assert np.abs(gl - rl).max() <= LSE_TOL * max(1.0, np.abs(rl).max())
    # a slice of the rows launched on its own: identical bits (a row's result
    # does not depend on the other rows of the launch)
    lo = 256 if S >= 296 else S // 2
    hi = min(S, lo + 40)
    o2, l2 = sparse_attn_fwd(q[:, lo:hi].contiguous(), kv, sink, idx[:, lo:hi].contiguous(), D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(o[:, lo:hi], o2) and torch.equal(lse[:, lo:hi], l2)


@pytest.mark.parametrize("D,i64", [(576, False), (128, True)])
def test_row_len(cuda_device, D, i64):
    # Per-row column counts (0, inside a tile, on a tile edge, past K, random):
    # columns at or past row_len are masked and their tiles never run.  Equal
    # to the oracle over the tail-masked rows, and bit for bit to the plain
    # forward over those rows (whose dead tiles are skipped, not dropped).
    B, S, H, N, K = 2, 40, 64, 300, 200
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=800 + D, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(D)
    idx = torch.randint(-1, N, (B, S, K), generator=g, dtype=torch.int64 if i64 else torch.int32)
    rl = torch.randint(0, K + 40, (B, S), generator=g, dtype=torch.int32)
    rl[:, :6] = torch.tensor([0, 1, 31, 32, 33, K], dtype=torch.int32)
    rl[:, 6] = K + 7
    idx, rl = idx.cuda(), rl.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5, row_len=rl)
    col = torch.arange(K, device="cuda")
    masked = idx.masked_fill(col >= rl.unsqueeze(-1).long(), -1)
    o2, l2 = sparse_attn_fwd(q, kv, sink, masked, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, l2)
    _check(q, kv, sink, masked, D ** -0.5, o, lse, f"row_len D={D}")
    assert o[:, 0].float().abs().max().item() == 0.0  # row_len 0: nothing attended


@pytest.mark.parametrize("D", [576, 512])
def test_rows_per_workgroup(cuda_device, D):
    # At D >= 512 a workgroup runs 8 consecutive rows and copies each next row's
    # first index words during the current row.  Rows of every kind next to each
    # other in a group (no tile, one tile, five tiles -- the next row's words go
    # out at the first iteration --, long rows, lengths past K), S not a multiple
    # of 8, two batches and two head groups: bit for bit the same rows launched
    # one at a time, and the oracle over the tail-masked rows.
    B, S, H, N, K = 2, 37, 100, 400, 256
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=900 + D, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(900 + D)
    idx = torch.randint(-1, N, (B, S, K), generator=g, dtype=torch.int32)
    rl = torch.randint(0, K + 40, (B, S), generator=g, dtype=torch.int32)
    rl[:, :16] = torch.tensor([0, 0, 32, 160, 256, 1, 0, 300, 200, 33, 161, 0, 64, 256, 5, 129], dtype=torch.int32)
    idx, rl = idx.cuda(), rl.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5, row_len=rl)
    torch.cuda.synchronize()
    for s in range(S):
        o1, l1 = sparse_attn_fwd(q[:, s:s + 1].contiguous(), kv, sink, idx[:, s:s + 1].contiguous(), D ** -0.5,
                                 row_len=rl[:, s:s + 1].contiguous())
        assert torch.equal(o[:, s:s + 1], o1) and torch.equal(lse[:, s:s + 1], l1), f"D={D} row {s}"
    col = torch.arange(K, device="cuda")
    masked = idx.masked_fill(col >= rl.unsqueeze(-1).long(), -1)
    _check(q, kv, sink, masked, D ** -0.5, o, lse, f"rows per workgroup D={D}")


@pytest.mark.parametrize("D", [32, 64, 128, 256, 512, 576])
def test_head_dims(cuda_device, D):
    B, S, H, N, K = 1, 24, 64, 300, 96
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=200 + D)
    idx = synth.causal_random_topk(B, S, K, 1, seed=D)
    o, lse = sparse_attn_fwd(q, kv, sink, idx)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, D ** -0.5, o, lse, f"D={D}")


@pytest.mark.parametrize("D,K,i64", [(576, 160, False), (576, 256, True), (576, 512, False), (128, 192, True),
                                     (64, 256, False), (256, 224, False)])
def test_tile_pipeline_depths(cuda_device, D, K, i64):
    # 5..16 key tiles: the steady-state iteration, its three tail variants and
    # the index prefetch distance all run (up to 4 tiles only the tails run)
    B, S, H, N = 1, 16, 64, 512
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=500 + K, q_scale=0.5, kv_scale=0.5)
    g = torch.Generator().manual_seed(K)
    idx = torch.randint(0, N, (B, S, K), generator=g, dtype=torch.int64 if i64 else torch.int32)
    idx[:, :, ::5] = -1
    idx = idx.cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, D ** -0.5, o, lse, f"D={D} K={K}")


@pytest.mark.parametrize("H", [16, 24, 64, 128, 192, 256, 300])
def test_head_counts(cuda_device, H):
    # any H: one workgroup per 64-head group (the reference's cdiv(H, block_h)
    # grid, sparse_attn_fwd.py:258); 300 leaves a partial fifth group
    B, S, D, N, K = 2, 10, 128, 64, 50
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=300 + H)
    g = torch.Generator().manual_seed(H)
    idx = torch.randint(-1, N + 3, (B, S, K), generator=g).cuda()  # includes -1 and >= N (masked)
    o, lse = sparse_attn_fwd(q, kv, sink, idx, 0.1)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, 0.1, o, lse, f"H={H}")


@pytest.mark.parametrize("H", [192, 136])
def test_head_groups_v4_dim(cuda_device, H):
    # D = 576 with three head groups (eight rows per workgroup) and int64 indices
    B, S, D, N, K = 1, 40, 576, 300, 96
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=320 + H)
    g = torch.Generator().manual_seed(320 + H)
    idx = torch.randint(-1, N, (B, S, K), generator=g).cuda()
    o, lse = sparse_attn_fwd(q, kv, sink, idx)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, D ** -0.5, o, lse, f"D=576 H={H}")


def test_v4_shape_with_indexer_indices(cuda_device):
    # V4 CSA layout (64 heads, D=576, ratio 4) at small S: indices from the fused indexer.
    from streamindex_amd import chunked_indexer_topk

    S, T = 512, 128
    qi, ki, wi = synth.indexer_inputs(1, S, 64, 128, ratio=4, seed=2026)
    idx, _ = chunked_indexer_topk(qi, ki, wi, 64, causal_ratio=4)
    q, kv, sink = synth.sparse_attn_inputs(1, S, 64, 576, T, seed=2027)
    o, lse = sparse_attn_fwd(q, kv, sink, idx, 576 ** -0.5)
    torch.cuda.synchronize()
    _check(q, kv, sink, idx, 576 ** -0.5, o, lse, "v4")


def test_sparse_attn_matches_fwd(cuda_device):
    B, S, H, D, N, K = 1, 4, 16, 64, 32, 8
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N, seed=7)
    idx = synth.causal_random_topk(B, S, K, 1, seed=7)
    o = sparse_attn(q, kv, sink, idx)
    o2, _ = sparse_attn_fwd(q, kv, sink, idx)
    assert torch.equal(o, o2)


@pytest.mark.parametrize("D,H,f16", [(576, 64, False), (128, 16, True), (64, 80, False), (512, 130, False)])
def test_two_kv_tensors(cuda_device, D, H, f16):
    # [kv ; kv2] read in place (the CSA / HCA layout): bit-identical to the
    # forward over their concatenation, with per-row column counts, a strided
    # second tensor and indices past N (masked); gradients through the
    # two-tensor autograd equal those of the concatenated one.
    from streamindex_amd import sparse_attn_fwd_kv2, sparse_attn_kv2

    B, S, N1, N2, K = 2, 48, 100, 37, 96
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N1, seed=400 + D)
    _, big, _ = synth.sparse_attn_inputs(B, 1, 1, D, 2 * N2, seed=401 + D)
    kv2 = big[:, ::2]  # row stride 2 D
    if f16:
        q, kv, kv2 = q.half(), kv.half(), kv2.half()
    g = torch.Generator().manual_seed(D + H)
    idx = torch.randint(-1, N1 + N2 + 3, (B, S, K), generator=g, dtype=torch.int32).cuda()
    rl = torch.randint(0, K + 5, (B, S), generator=g, dtype=torch.int32).cuda()
    kv_cat = torch.cat([kv, kv2], dim=1)
    for row_len in (None, rl):
        o1, l1 = sparse_attn_fwd_kv2(q, kv, kv2, sink, idx, row_len=row_len)
        o2, l2 = sparse_attn_fwd(q, kv_cat, sink, idx, row_len=row_len)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
    if not f16:
        o1, l1 = sparse_attn_fwd_kv2(q, kv, kv2, sink, idx)
        _check(q, kv_cat, sink, idx, D ** -0.5, o1, l1, f"kv2 D={D}")
    leaves = [t.detach().requires_grad_() for t in (q, kv, kv2, sink)]
    o = sparse_attn_kv2(leaves[0], leaves[1], leaves[2], leaves[3], idx, row_len=rl)
    do = torch.randn(o.shape, generator=g).to(o.dtype).cuda()
    g1 = torch.autograd.grad(o, leaves, do)
    leaves2 = [t.detach().requires_grad_() for t in (q, kv_cat, sink)]
    o2 = sparse_attn(leaves2[0], leaves2[1], leaves2[2], idx, row_len=rl)
    g2 = torch.autograd.grad(o2, leaves2, do)
    assert torch.equal(o, o2)
    assert torch.equal(g1[0], g2[0]) and torch.equal(g1[3], g2[2])
    assert torch.equal(torch.cat([g1[1], g1[2]], dim=1), g2[1])


def test_two_kv_empty_first(cuda_device):
    # no rows in the first tensor (its data pointer may be null): every index
    # selects a row of the second one, masked keys must not read the first;
    # bit-identical to the one-tensor forward over the second tensor
    from streamindex_amd import sparse_attn_fwd_kv2

    B, S, H, D, N2, K = 2, 24, 64, 576, 45, 64
    q, kv2, sink = synth.sparse_attn_inputs(B, S, H, D, N2, seed=411)
    kv = torch.empty(B, 0, D, dtype=kv2.dtype, device=kv2.device)
    g = torch.Generator().manual_seed(2)
    idx = torch.randint(-1, N2 + 4, (B, S, K), generator=g, dtype=torch.int32).cuda()
    rl = torch.randint(0, K + 1, (B, S), generator=g, dtype=torch.int32).cuda()
    for row_len in (None, rl):
        o1, l1 = sparse_attn_fwd_kv2(q, kv, kv2, sink, idx, row_len=row_len)
        o2, l2 = sparse_attn_fwd(q, kv2, sink, idx, row_len=row_len)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_two_kv_empty_second(cuda_device):
    # no rows in the second tensor: the one-tensor path; indices past N1 masked
    from streamindex_amd import sparse_attn_fwd_kv2

    B, S, H, D, N1, K = 1, 16, 16, 64, 40, 32
    q, kv, sink = synth.sparse_attn_inputs(B, S, H, D, N1, seed=410)
    kv2 = torch.empty(B, 0, D, dtype=kv.dtype, device=kv.device)
    idx = torch.randint(-1, N1 + 4, (B, S, K), generator=torch.Generator().manual_seed(1), dtype=torch.int32).cuda()
    o1, l1 = sparse_attn_fwd_kv2(q, kv, kv2, sink, idx)
    o2, l2 = sparse_attn_fwd(q, kv, sink, idx)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
