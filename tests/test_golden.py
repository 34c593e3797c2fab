"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every stored output exactly (indices, index rows,
quantised values and scales) or to float32 rounding (scores, attention
outputs and gradients).
GPU: the HIP kernels reproduce the stored outputs — exact index lists for
the indexer (including the exact-tie case) and for the CSA / HCA index rows,
bit-exact quantisation, 2e-2 for attention outputs, 1e-2 relative
(Frobenius) and 2e-2 of max|ref| for the backward's dq and dkv.
"""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
INDEXER = sorted(glob.glob(os.path.join(HERE, "indexer_*.npz")))
ATTN = sorted(glob.glob(os.path.join(HERE, "attn_d*.npz")))
BWD = sorted(glob.glob(os.path.join(HERE, "attn_bwd_*.npz")))
QUANT = os.path.join(HERE, "quant_blocks.npz")
CSA = os.path.join(HERE, "csa_rows.npz")


def _ratio(z):
    r = int(z["ratio"])
    return None if r < 0 else r


@pytest.mark.parametrize("path", INDEXER, ids=os.path.basename)
def test_oracle_reproduces_indexer_fixture(path):
    z = np.load(path)
    idx, val, _ = O.indexer_topk_rows(z["q"], z["k"], z["w"], int(z["top_k"]), causal_ratio=_ratio(z))
    assert np.array_equal(idx, z["idx"])
    assert np.array_equal(val, z["score"])


@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_oracle_reproduces_attn_fixture(path):
    z = np.load(path)
    o, lse = O.sparse_attn_rows(z["q"], z["kv"], z["sink"], z["idx"], float(z["scale"]))
    assert np.array_equal(o.astype(np.float32), z["o"])
    assert np.array_equal(lse.astype(np.float32), z["lse"])


def _t(bits, dev):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("path", INDEXER, ids=os.path.basename)
def test_gpu_matches_indexer_fixture(cuda_device, path):
    from streamindex_amd import chunked_indexer_topk

    z = np.load(path)
    q = _t(z["q"], cuda_device).unsqueeze(0)
    k = _t(z["k"], cuda_device).unsqueeze(0)
    w = torch.from_numpy(z["w"]).to(cuda_device).unsqueeze(0)
    idx, sc = chunked_indexer_topk(q, k, w, int(z["top_k"]), causal_ratio=_ratio(z))
    torch.cuda.synchronize()
    assert np.array_equal(idx[0].cpu().numpy(), z["idx"])
    ref = z["score"]
    got = sc[0].cpu().numpy().astype(np.float64)
    fin = np.isfinite(ref)
    assert np.array_equal(fin, np.isfinite(got))
    assert np.abs(got[fin] - ref[fin]).max() <= 1e-4 * (np.abs(ref[fin]).max() + 1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ATTN, ids=os.path.basename)
def test_gpu_matches_attn_fixture(cuda_device, path):
    from streamindex_amd import sparse_attn_fwd

    z = np.load(path)
    q = _t(z["q"], cuda_device).unsqueeze(0)
    kv = _t(z["kv"], cuda_device).unsqueeze(0)
    sink = torch.from_numpy(z["sink"]).to(cuda_device)
    idx = torch.from_numpy(z["idx"]).to(cuda_device).unsqueeze(0)
    o, lse = sparse_attn_fwd(q, kv, sink, idx, float(z["scale"]))
    torch.cuda.synchronize()
    assert np.abs(o[0].float().cpu().numpy() - z["o"]).max() <= 2e-2
    assert np.abs(lse[0].cpu().numpy() - z["lse"]).max() <= 2e-3 * max(1.0, np.abs(z["lse"]).max())


@pytest.mark.parametrize("path", BWD, ids=os.path.basename)
def test_oracle_reproduces_bwd_fixture(path):
    z = np.load(path)
    dq, dkv, dsink = O.sparse_attn_bwd_rows(z["q"], z["kv"], z["o"], z["do"], z["sink"], z["lse"], z["idx"],
                                            float(z["scale"]))
    assert np.array_equal(dq.astype(np.float32), z["dq"])
    assert np.array_equal(dkv.astype(np.float32), z["dkv"])
    assert np.array_equal(dsink.astype(np.float32), z["dsink"])


def _quant_expect(z, tag):
    return {k[:-len(tag) - 1]: z[k] for k in z.files if k.endswith("_" + tag)}


def test_oracle_reproduces_quant_fixture():
    z = np.load(QUANT)
    for tag, x, dt in (("f32", z["x"], "float32"), ("bf16", z["xb"], "bfloat16")):
        e = _quant_expect(z, tag)
        assert np.array_equal(O.act_quant_simulate(x, dt, 128), e["sim8"])
        assert np.array_equal(O.fp4_act_quant_simulate(x, dt, 32), e["sim4"])
        v8, s8 = O.fp8_pack(x, 128)
        v8p, s8p = O.fp8_pack(x, 128, pow2=True)
        v4, s4 = O.fp4_pack(x, 32)
        for got, key in ((v8, "v8"), (s8, "s8"), (v8p, "v8p"), (s8p, "s8p"), (v4, "v4"), (s4, "s4")):
            assert np.array_equal(got, e[key]), key


def test_oracle_reproduces_csa_rows_fixture():
    z = np.load(CSA)
    S = z["scores"].shape[0]
    rows = np.arange(S)
    csa = O.csa_scores_topk_rows(z["scores"], rows, int(z["m"]), int(z["top_k"]), int(z["n_win"]), S)
    hca = O.hca_idx_rows(rows, int(z["n_win"]), int(z["n_comp_hca"]), int(z["m_prime"]), S)
    assert np.array_equal(csa.astype(np.int32), z["csa"])
    assert np.array_equal(hca.astype(np.int32), z["hca"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", BWD, ids=os.path.basename)
def test_gpu_matches_bwd_fixture(cuda_device, path):
    from streamindex_amd import sparse_attn_bwd

    z = np.load(path)
    q = _t(z["q"], cuda_device).unsqueeze(0)
    kv = _t(z["kv"], cuda_device).unsqueeze(0)
    o = _t(z["o"], cuda_device).unsqueeze(0)
    do = _t(z["do"], cuda_device).unsqueeze(0)
    sink = torch.from_numpy(z["sink"]).to(cuda_device)
    lse = torch.from_numpy(z["lse"]).to(cuda_device).unsqueeze(0)
    idx = torch.from_numpy(z["idx"]).to(cuda_device).unsqueeze(0)
    dq, dkv, dsink = sparse_attn_bwd(q, kv, sink, idx, o, lse, do, float(z["scale"]))
    torch.cuda.synchronize()
    for got, ref in ((dq[0].float().cpu().numpy(), z["dq"]), (dkv[0].float().cpu().numpy(), z["dkv"])):
        assert np.linalg.norm(got - ref) <= 1e-2 * np.linalg.norm(ref)
        assert np.abs(got - ref).max() <= 2e-2 * np.abs(ref).max()
    gs = dsink.float().cpu().numpy()
    assert np.abs(gs - z["dsink"]).max() <= 1e-3 * max(1.0, np.abs(z["dsink"]).max())


@pytest.mark.gpu
def test_gpu_matches_quant_fixture(cuda_device):
    from streamindex_amd import quant

    z = np.load(QUANT)
    for tag, x, dt in (("f32", z["x"], torch.float32), ("bf16", z["xb"], torch.bfloat16)):
        e = _quant_expect(z, tag)
        xt = torch.from_numpy(x).to(cuda_device).to(dt)
        assert np.array_equal(quant.act_quant_simulate(xt, 128).float().cpu().numpy(), e["sim8"])
        assert np.array_equal(quant.fp4_act_quant_simulate(xt, 32).float().cpu().numpy(), e["sim4"])
        v8, s8 = quant.act_quant(xt, 128)
        v8p, s8p = quant.act_quant(xt, 128, scale_fmt="ue8m0")
        p4, s4 = quant.fp4_act_quant(xt, 32)
        torch.cuda.synchronize()
        assert np.array_equal(v8.float().cpu().numpy(), e["v8"]) and np.array_equal(s8.cpu().numpy(), e["s8"])
        assert np.array_equal(v8p.float().cpu().numpy(), e["v8p"]) and np.array_equal(s8p.cpu().numpy(), e["s8p"])
        assert np.array_equal(O.fp4_unpack(p4.cpu().numpy()), e["v4"]) and np.array_equal(s4.cpu().numpy(), e["s4"])


@pytest.mark.gpu
def test_gpu_matches_csa_rows_fixture(cuda_device):
    from streamindex_amd import build_csa_topk_idxs, build_hca_topk_idxs

    z = np.load(CSA)
    S, T = z["scores"].shape
    sc = torch.from_numpy(z["scores"]).to(cuda_device).unsqueeze(0)
    csa = build_csa_topk_idxs(sc, int(z["n_win"]), int(z["top_k"]), seq_len=S, n_compressed=T, m=int(z["m"]),
                              device=cuda_device)
    hca = build_hca_topk_idxs(B=1, seq_len=S, n_win=int(z["n_win"]), n_compressed=int(z["n_comp_hca"]),
                              m_prime=int(z["m_prime"]), device=cuda_device)
    torch.cuda.synchronize()
    assert np.array_equal(csa[0].cpu().numpy(), z["csa"])
    assert np.array_equal(hca[0].cpu().numpy(), z["hca"])
