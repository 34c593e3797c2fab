"""Benchmark of the StreamIndex MI355X hot path.

Metric: V4-Flash indexer ms at S=64K and S=1M, MFMA utilisation, peak HBM.
Default workload: the V4-Flash indexer on one MI355X,
B=1, S=65,536, H_I=64, D_I=128, T=16,384, top_k=512, causal_ratio=4,
chunk_s=2048, chunk_t=8192, seeded bf16/fp32 synthetic inputs resident in HBM.
One "step" = one ``chunked_indexer_topk`` call (one launch of the fused
score + top-k kernel).

Printed (one JSON line, rank 0):
  value          ms per call at S=64K (lower is better)
  roofline       MFMA bound of the dominant kernel: algorithmic FLOPs
                 (2·H_I·D_I per causally legal (s,t) pair) / mean kernel time
                 from HIP events on the launch stream, vs 2516.6 TFLOP/s
  peak_hbm_gib   max_memory_allocated delta during one call (inputs excluded)
  parity         recall vs the CPU oracle on sampled rows
  cpu_baseline   the CPU oracle on a bounded row sample, extrapolated
  extra          S=1M indexer time (config[4] indexer stage), the indexer over
                 the production V4 dtypes (fp4 q, fp8 k) at S=64K and 1M vs the
                 fp8 MFMA peak with sampled-row recall, sparse-attn fwd
                 at config[3] with its HBM roofline, the sparse-attn backward
                 at config[3] (dq, dkv, dsink from the saved o / lse; sampled
                 dq rows and dkv keys against the oracle), and the end-to-end CSA
                 forward (flash_csa_forward: fused indexer -> int32 window +
                 compressed index rows -> sparse attention, 64 heads, d=576,
                 n_win=128) at S=64K and at S=1M (config[4]) with its stage
                 split, peak HBM and sampled-row recall against the oracle,
                 and at S=1M again with the fp4/fp8 indexer (the production
                 V4 indexer dtypes, quantised inside the timed call)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from streamindex_amd import (build_hca_topk_idxs, chunked_indexer_topk, csa_topk_idxs,  # noqa: E402
                             flash_csa_forward, flash_hca_forward, sparse_attn, sparse_attn_bwd, sparse_attn_fwd)
from streamindex_amd import synth  # noqa: E402
from streamindex_amd import _lib  # noqa: E402
from streamindex_amd.csa import csa_row_len  # noqa: E402
from streamindex_amd.hca import hca_row_len  # noqa: E402

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5033.2   # MI355X dense fp8 MFMA (the fp4 x fp8 product runs at the fp8 rate)
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
# Reference timings on one H200 (other hardware; context only):
# benchmarks/results/2026-04-27/scaling_v4_flash_indexer_final.log:10,14
REF_H200_MS = {65536: 122.2, 1048576: 30899.6}

TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def _events_time(fn, iters: int, stream: torch.cuda.Stream) -> float:
    """Mean ms per call, HIP events recorded on `stream` (the launch stream)."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    return float(np.mean([s.elapsed_time(e) for s, e in zip(starts, ends)]))


def _peak_gib(fn) -> float:
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    peak = max(0, torch.cuda.max_memory_allocated() - base) / 1024 ** 3
    del out
    return peak


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def indexer_parity_and_cpu(q, k, w, idx, sc, ratio, top_k, nrows, seed=0):
    """Oracle on `nrows` sampled rows: recall + CPU time (the cpu_baseline leg)."""
    from oracle import oracle as O

    S = q.shape[1]
    T = k.shape[1]
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(S, size=min(nrows, S), replace=False)).astype(np.int64)
    qb = _bits(q[0, torch.from_numpy(rows).to(q.device)])
    kb = _bits(k[0])
    wb = w[0, torch.from_numpy(rows).to(q.device)].float().cpu().numpy()
    local = np.arange(len(rows), dtype=np.int64)
    O.lib()
    t0 = time.perf_counter()
    lim = O.legal_limits(rows, T, ratio)
    scores = O.indexer_scores(qb, kb, wb, local, lim=lim)  # rows' own q/w are packed densely
    ref_idx, _ = O.topk(scores, lim, top_k)
    cpu_s = time.perf_counter() - t0
    got = idx[0].cpu().numpy()[rows]
    rec = O.set_overlap_recall(ref_idx, got)
    pairs_sample = float(np.minimum(lim, T).sum())
    return {
        "rows": int(len(rows)),
        "recall_mean": float(rec.mean()),
        "recall_min": float(rec.min()),
        "exact_rows_frac": float((rec == 1.0).mean()),
        "cpu_s": cpu_s,
        "pairs_sample": pairs_sample,
    }


def run_indexer(S, ratio, top_k, chunk_s, chunk_t, steps, warmup, H=64, D=128, seed=2026):
    dev = torch.device("cuda:0")
    q, k, w = synth.indexer_inputs(1, S, H, D, ratio=ratio, seed=seed, device=dev)
    T = k.shape[1]
    fn = lambda: chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio, chunk_s=chunk_s, chunk_t=chunk_t)  # noqa: E731
    for _ in range(max(1, warmup)):
        out = fn()
    torch.cuda.synchronize()
    peak = _peak_gib(fn)
    stream = torch.cuda.current_stream(dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = _events_time(fn, steps, stream)
    wall = (time.perf_counter() - t0) * 1e3 / steps
    flops = synth.indexer_flops(S, T, H, D, ratio)
    idx, sc = fn()
    torch.cuda.synchronize()
    return dict(q=q, k=k, w=w, T=T, ms=ms, wall_ms=wall, peak_gib=peak, flops=flops, idx=idx, sc=sc)


def run_indexer_q(S, ratio, top_k, steps, warmup, H=64, D=128, seed=2026, parity_rows=256):
    """The indexer over the production V4 dtypes: the same synthetic q / k as
    run_indexer, quantised (untimed) to fp4 (UE8M0 per 32 dims) and fp8 (one
    scale per key row); `indexer_topk_q` timed; sampled rows checked against the
    oracle on the dequantised inputs (exact scores, same gate as the tests)."""
    from oracle import oracle as O
    from streamindex_amd import indexer_topk_q, quant

    dev = torch.device("cuda:0")
    q, k, w = synth.indexer_inputs(1, S, H, D, ratio=ratio, seed=seed, device=dev)
    T = k.shape[1]
    q4, qs = quant.fp4_act_quant(q, 32)
    k8, ks = quant.act_quant(k, D)
    del q, k
    fn = lambda: indexer_topk_q(q4, qs, k8, ks, w, top_k, causal_ratio=ratio, check_scales=False)  # noqa: E731
    for _ in range(max(1, warmup)):
        fn()
    torch.cuda.synchronize()
    ms = _events_time(fn, steps, torch.cuda.current_stream(dev))
    idx, sc = fn()
    torch.cuda.synchronize()
    rng = np.random.default_rng(7)
    rows = np.sort(rng.choice(S, size=min(parity_rows, S), replace=False)).astype(np.int64)
    sel = torch.from_numpy(rows).to(dev)
    qv = O.fp4_unpack(q4[0, sel].cpu().numpy()) * np.repeat(qs[0, sel].cpu().numpy(), 32, axis=-1)
    kv = k8[0].float().cpu().numpy()
    lim = O.legal_limits(rows, T, ratio)
    ref = O.indexer_scores(O.f32_to_bf16_bits(qv.astype(np.float32)), O.f32_to_bf16_bits(kv),
                           w[0, sel].float().cpu().numpy(), np.arange(len(rows), dtype=np.int64), lim=lim)
    ref = ref * ks[0, :, 0].cpu().numpy().astype(np.float64)[None, :]
    ref_idx, _ = O.topk(ref, lim, top_k)
    rec = O.set_overlap_recall(ref_idx, idx[0, sel].cpu().numpy())
    flops = synth.indexer_flops(S, T, H, D, ratio)
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "fp8_mfma_frac": flops / (ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS,
            "parity_rows": int(len(rows)), "recall_mean": float(rec.mean()), "recall_min": float(rec.min())}


def run_sparse_attn(S, T, H, D, top_k, steps, warmup, idx=None, bwd=False, fwd=True):
    """Forward (and optionally backward) sparse attention at one shape.  The
    backward is timed from the forward's saved (o, lse) with dO ~ N(0,1)·0.5,
    including its key sort and reduction; its FLOPs count the five products
    per selected (row, key) pair (S and dP recomputed, dQ, dK, dV): 10 H D."""
    dev = torch.device("cuda:0")
    q, kv, sink = synth.sparse_attn_inputs(1, S, H, D, T, seed=2027, device=dev)
    if idx is None:
        idx = synth.causal_random_topk(1, S, top_k, 4, device=dev)
    fn = lambda: sparse_attn_fwd(q, kv, sink, idx, D ** -0.5)  # noqa: E731
    nvalid = float((idx >= 0).sum().item())
    res = dict(nvalid=nvalid)
    stream = torch.cuda.current_stream(dev)
    if fwd:
        for _ in range(max(1, warmup)):
            fn()
        torch.cuda.synchronize()
        res["ms"] = _events_time(fn, steps, stream)
        res["flops"] = 4.0 * H * D * nvalid
        res["unique_bytes"] = (q.numel() * 2 * 2 + idx.numel() * idx.element_size() + S * H * 4 + kv.numel() * 2)
    if bwd:
        o, lse = fn()
        g = torch.Generator(device=dev)
        g.manual_seed(2028)
        do = torch.randn(q.shape, generator=g, device=dev, dtype=torch.bfloat16).mul_(0.5)
        bfn = lambda: sparse_attn_bwd(q, kv, sink, idx, o, lse, do, D ** -0.5)  # noqa: E731
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        for _ in range(max(1, warmup)):
            grads = bfn()
        del grads
        torch.cuda.synchronize()
        res["bwd_ms"] = _events_time(bfn, steps, stream)
        res["bwd_flops"] = 10.0 * H * D * nvalid
        res["bwd_peak_extra_gib"] = (torch.cuda.max_memory_allocated(dev) - base) / 2 ** 30
        res["bwd_parity"] = attn_bwd_check(q, kv, sink, idx, o, lse, do, bfn())
    return res


def attn_bwd_check(q, kv, sink, idx, o, lse, do, grads, nrows=2, nkeys=2, seed=6):
    """dq on sampled rows and dkv on sampled late keys (few rows select them)
    against the oracle backward; relative Frobenius and max errors."""
    from oracle import oracle as O

    dq, dkv, _ = grads
    S, N, D = q.shape[1], kv.shape[1], q.shape[3]
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(S, size=nrows, replace=False))
    keys = np.sort(N - 1 - rng.choice(N // 16, size=nkeys, replace=False))
    sel = torch.from_numpy(rows).to(q.device)
    idx_c = idx[0].cpu().numpy().astype(np.int64)
    hit = np.nonzero(np.isin(idx_c, keys).any(axis=1))[0]
    ht = torch.from_numpy(hit).to(q.device)
    sk = sink.cpu().numpy()
    rdq, _, _ = O.sparse_attn_bwd_rows(_bits(q[0, sel]), _bits(kv[0]), _bits(o[0, sel]), _bits(do[0, sel]), sk,
                                       lse[0, sel].cpu().numpy(), idx_c[rows], D ** -0.5, want_dkv=False)
    _, rdkv, _ = O.sparse_attn_bwd_rows(_bits(q[0, ht]), _bits(kv[0]), _bits(o[0, ht]), _bits(do[0, ht]), sk,
                                        lse[0, ht].cpu().numpy(), idx_c[hit], D ** -0.5, keys=keys, want_dq=False)
    out = {"dq_rows": int(nrows), "dkv_keys": int(nkeys), "dkv_key_rows": int(len(hit))}
    for name, got, ref in (("dq", dq[0, sel].float().cpu().numpy(), rdq),
                           ("dkv", dkv[0, torch.from_numpy(keys).to(q.device)].float().cpu().numpy(), rdkv)):
        out[f"{name}_rel_fro"] = float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))
        out[f"{name}_max_rel"] = float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))
    return out


def csa_recall(qi, ki, w, rows_gpu, n_win, top_k, m, nrows, seed=3):
    """Recall of the compressed picks of `nrows` sampled rows against the oracle."""
    from oracle import oracle as O

    S = qi.shape[1]
    T = ki.shape[1]
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(S, size=min(nrows, S), replace=False)).astype(np.int64)
    sel = torch.from_numpy(rows).to(qi.device)
    lim = O.legal_limits(rows, T, m)
    sc = O.indexer_scores(_bits(qi[0, sel]), _bits(ki[0]), w[0, sel].float().cpu().numpy(),
                          np.arange(len(rows), dtype=np.int64), lim=lim)
    ref_idx, _ = O.topk(sc, lim, top_k)
    got = rows_gpu[0, sel, n_win:].long().cpu().numpy()
    got = np.where(got >= 0, got - S, -1)
    rec = O.set_overlap_recall(ref_idx, got)
    return {"rows": int(len(rows)), "recall_mean": float(rec.mean()), "recall_min": float(rec.min())}


def csa_attn_check(q, kv, kvc, sink, rows_gpu, nrows=8, seed=4):
    """Max |o - o_ref| of the attention output on `nrows` sampled rows (oracle over the GPU's index rows)."""
    from oracle import oracle as O

    S, H, D = q.shape[1], q.shape[2], q.shape[3]
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(S, size=min(nrows, S), replace=False)).astype(np.int64)
    sel = torch.from_numpy(rows).to(q.device)
    idx = rows_gpu[0, sel].long()
    kv_full = torch.cat([kv[0], kvc[0]], dim=0)
    uniq = torch.unique(idx[idx >= 0])
    remap = torch.where(idx >= 0, torch.searchsorted(uniq, idx.clamp(min=0)), torch.full_like(idx, -1))
    o = sparse_attn(q[:, sel], torch.cat([kv, kvc], dim=1), sink, rows_gpu[:, sel], None)
    ro, _ = O.sparse_attn_rows(_bits(q[0, sel]), _bits(kv_full[uniq]), sink.cpu().numpy(), remap.cpu().numpy(),
                               D ** -0.5)
    return float(np.abs(o[0].float().cpu().numpy() - ro).max())


def run_csa_e2e(S, steps, warmup, parity_rows, n_h=64, d=576, H_I=64, D_I=128, m=4, n_win=128, top_k=512,
                quantized=False, bwd=False):
    """flash_csa_forward at V4-Flash dims; returns timings, stage split, peak HBM and parity.  With
    ``quantized`` the indexer runs under the production dtypes (fp4 q, fp8 k, quantised inside the
    timed call); the recall is then that of the quantised selection against the bf16 oracle."""
    dev = torch.device("cuda:0")
    qi, ki, w = synth.indexer_inputs(1, S, H_I, D_I, ratio=m, seed=2026, device=dev)
    q, kv, kvc, sink = synth.csa_attn_inputs(1, S, n_h, d, S // m, seed=2027, device=dev)
    fn = lambda: flash_csa_forward(q, kv, kvc, qi, ki, w, sink, n_win=n_win, top_k=top_k, m=m,  # noqa: E731
                                   quantized_indexer=quantized)
    for _ in range(max(1, warmup)):
        fn()
    torch.cuda.synchronize()
    peak = _peak_gib(fn)
    stream = torch.cuda.current_stream(dev)
    ms = _events_time(fn, steps, stream)
    # stage split of one call (same three steps flash_csa_forward runs)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record(stream)
    rows_gpu = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m, seq_len=S, quantized=quantized)
    row_len = csa_row_len(1, S, n_win, top_k, S // m, m, dev)
    ev[1].record(stream)
    kv_full = torch.cat([kv, kvc], dim=1)
    ev[2].record(stream)
    o = sparse_attn(q, kv_full, sink, rows_gpu, None, row_len=row_len)
    ev[3].record(stream)
    torch.cuda.synchronize()
    del o, kv_full
    nvalid = float((rows_gpu >= 0).sum().item())
    res = {
        "S": S, "T": S // m, "n_h": n_h, "d": d, "n_win": n_win, "top_k": top_k,
        "ms": ms, "peak_hbm_gib": peak,
        "indexer_ms": ev[0].elapsed_time(ev[1]), "concat_ms": ev[1].elapsed_time(ev[2]),
        "attn_ms": ev[2].elapsed_time(ev[3]),
        "indexer_flops": synth.indexer_flops(S, S // m, H_I, D_I, m),
        "attn_flops": 4.0 * n_h * d * nvalid,
    }
    res["indexer_tflops"] = res["indexer_flops"] / (res["indexer_ms"] * 1e-3) / 1e12
    res["attn_tflops"] = res["attn_flops"] / (res["attn_ms"] * 1e-3) / 1e12
    if parity_rows > 0:
        res["recall_vs_bf16_oracle" if quantized else "parity"] = csa_recall(qi, ki, w, rows_gpu, n_win, top_k, m,
                                                                            parity_rows)
        res["attn_max_abs_err"] = csa_attn_check(q, kv, kvc, sink, rows_gpu)
    if bwd:
        # backward of the composition through autograd (the indexer's picks carry no gradient)
        qg, kvg, kvcg, sg = (t.detach().requires_grad_() for t in (q, kv, kvc, sink))
        og = flash_csa_forward(qg, kvg, kvcg, qi, ki, w, sg, n_win=n_win, top_k=top_k, m=m,
                               quantized_indexer=quantized)
        do = torch.randn_like(og)
        og.backward(do, retain_graph=True)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            og.backward(do, retain_graph=True)
        e1.record(stream)
        torch.cuda.synchronize()
        res["bwd_ms"] = e0.elapsed_time(e1) / steps
        res["bwd_tflops"] = 10.0 * n_h * d * nvalid / (res["bwd_ms"] * 1e-3) / 1e12
        del qg, kvg, kvcg, sg, og, do
    del q, kv, kvc, qi, ki, w, rows_gpu
    torch.cuda.empty_cache()
    return res


def run_hca_e2e(S, steps, warmup, check_rows, n_h=64, d=576, n_win=128, m_prime=128, bwd=False):
    """flash_hca_forward at V4-Flash attention dims (window n_win plus every causally legal
    compressed entry, ratio m_prime; ``hca.py:54-95``).  The index rows end in the masked
    compressed tail, on average half the row: whole 32-key tiles of it are skipped by the
    attention kernel.  Returns timings, stage split, useful FLOPs and parity on sampled rows."""
    dev = torch.device("cuda:0")
    T = S // m_prime
    q, kv, kvc, sink = synth.csa_attn_inputs(1, S, n_h, d, T, seed=2029, device=dev)
    fn = lambda: flash_hca_forward(q, kv, kvc, sink, n_win=n_win, m_prime=m_prime)  # noqa: E731
    for _ in range(max(1, warmup)):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ms = _events_time(fn, steps, stream)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record(stream)
    rows_gpu = build_hca_topk_idxs(B=1, seq_len=S, n_win=n_win, n_compressed=T, m_prime=m_prime, device=dev)
    row_len = hca_row_len(1, S, n_win, T, m_prime, dev)
    ev[1].record(stream)
    kv_full = torch.cat([kv, kvc], dim=1)
    ev[2].record(stream)
    o = sparse_attn(q, kv_full, sink, rows_gpu, None, row_len=row_len)
    ev[3].record(stream)
    torch.cuda.synchronize()
    del o, kv_full
    nvalid = float((rows_gpu >= 0).sum().item())
    K = n_win + T
    res = {
        "S": S, "T": T, "n_h": n_h, "d": d, "n_win": n_win, "m_prime": m_prime, "K": K, "ms": ms,
        "rows_ms": ev[0].elapsed_time(ev[1]), "concat_ms": ev[1].elapsed_time(ev[2]),
        "attn_ms": ev[2].elapsed_time(ev[3]),
        "valid_frac": nvalid / (S * K),
        "attn_flops": 4.0 * n_h * d * nvalid,
    }
    res["attn_tflops"] = res["attn_flops"] / (res["attn_ms"] * 1e-3) / 1e12
    if check_rows > 0:
        res["attn_max_abs_err"] = csa_attn_check(q, kv, kvc, sink, rows_gpu, nrows=check_rows)
    if bwd:
        # backward of the whole composition through autograd (the index rows carry no gradient)
        qg, kvg, kvcg, sg = (t.detach().requires_grad_() for t in (q, kv, kvc, sink))
        og = flash_hca_forward(qg, kvg, kvcg, sg, n_win=n_win, m_prime=m_prime)
        do = torch.randn_like(og)
        og.backward(do, retain_graph=True)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            og.backward(do, retain_graph=True)
        e1.record(stream)
        torch.cuda.synchronize()
        res["bwd_ms"] = e0.elapsed_time(e1) / steps
        res["bwd_tflops"] = 10.0 * n_h * d * nvalid / (res["bwd_ms"] * 1e-3) / 1e12
        del qg, kvg, kvcg, sg, og, do
    del q, kv, kvc, rows_gpu
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--seq", type=int, default=65536)
    ap.add_argument("--top-k", type=int, default=512)
    ap.add_argument("--ratio", type=int, default=4)
    ap.add_argument("--chunk-s", type=int, default=2048)
    ap.add_argument("--chunk-t", type=int, default=8192)
    ap.add_argument("--parity-rows", type=int, default=4096)
    ap.add_argument("--no-long", action="store_true", help="skip the S=1M indexer measurement")
    ap.add_argument("--no-attn", action="store_true", help="skip the sparse-attention measurement")
    ap.add_argument("--only-indexer", action="store_true", help="indexer timing only (for profilers)")
    ap.add_argument("--only-attn", action="store_true", help="sparse-attention timing only (for profilers)")
    ap.add_argument("--only-attn-bwd", action="store_true", help="sparse-attention backward timing only (for profilers)")
    ap.add_argument("--only-indexer-q", type=int, default=0, metavar="S",
                    help="fp4/fp8 indexer timing only at sequence length S (for profilers)")
    ap.add_argument("--no-indexer-q", action="store_true", help="skip the fp4/fp8 indexer measurements")
    ap.add_argument("--no-attn-bwd", action="store_true", help="skip the sparse-attention backward measurement")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end CSA forward measurements")
    ap.add_argument("--e2e-parity-rows", type=int, default=1024,
                    help="sampled rows for the S=1M end-to-end recall check (config[4] asks 1024)")
    ap.add_argument("--only-e2e", type=int, default=0, metavar="S",
                    help="end-to-end CSA forward timing at sequence length S only (for profilers)")
    ap.add_argument("--only-hca", type=int, default=0, metavar="S",
                    help="end-to-end HCA forward timing at sequence length S only (for profilers)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run 5 plain device copies of MIB MiB (scales HBM byte counters) and exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_mib": args.calibrate_copy, "launches": 5}), flush=True)
        return
    if args.only_hca:
        rh = run_hca_e2e(args.only_hca, args.steps, args.warmup, 0, bwd=not args.no_attn_bwd)
        print(json.dumps(rh), flush=True)
        return
    if args.only_e2e:
        re_ = run_csa_e2e(args.only_e2e, args.steps, args.warmup, 0)
        print(json.dumps({k: v for k, v in re_.items() if not isinstance(v, dict)}), flush=True)
        return
    if args.only_indexer_q:
        rq = run_indexer_q(args.only_indexer_q, args.ratio, args.top_k, args.steps, args.warmup)
        print(json.dumps(rq), flush=True)
        return
    if args.only_attn_bwd:
        ra = run_sparse_attn(65536, 16384, 64, 576, 512, args.steps, args.warmup, bwd=True, fwd=False)
        print(json.dumps({"sparse_attn_bwd_ms": ra["bwd_ms"], "tflops": ra["bwd_flops"] / ra["bwd_ms"] / 1e9,
                          "parity": ra["bwd_parity"]}), flush=True)
        return
    if args.only_attn:
        ra = run_sparse_attn(65536, 16384, 64, 576, 512, args.steps, args.warmup)
        print(json.dumps({"sparse_attn_ms": ra["ms"], "tflops": ra["flops"] / ra["ms"] / 1e9,
                          "unique_gbps": ra["unique_bytes"] / ra["ms"] / 1e6}), flush=True)
        return

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}), flush=True)
        sys.exit(1)
    _lib.load()

    print(f"[bench] indexer S={args.seq} warmup={args.warmup} steps={args.steps}", file=sys.stderr, flush=True)
    r = run_indexer(args.seq, args.ratio, args.top_k, args.chunk_s, args.chunk_t, args.steps, args.warmup)
    if args.only_indexer:
        print(json.dumps({"indexer_ms": r["ms"], "tflops": r["flops"] / r["ms"] / 1e9}), flush=True)
        return
    tflops = r["flops"] / (r["ms"] * 1e-3) / 1e12
    print(f"[bench] indexer {r['ms']:.3f} ms, {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)

    print(f"[bench] parity + cpu baseline on {args.parity_rows} sampled rows", file=sys.stderr, flush=True)
    par = indexer_parity_and_cpu(r["q"], r["k"], r["w"], r["idx"], r["sc"], args.ratio, args.top_k,
                                 args.parity_rows)
    total_pairs = synth.legal_pairs(args.seq, r["T"], args.ratio)
    cpu_ms_full = par["cpu_s"] * 1e3 * total_pairs / max(1.0, par["pairs_sample"])
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    del r["q"], r["k"], r["w"], r["idx"], r["sc"]
    torch.cuda.empty_cache()

    extra = {"indexer_wall_ms_per_call": r["wall_ms"], "reference_h200_ms_s64k": REF_H200_MS[65536]}
    if not args.no_long:
        print("[bench] indexer S=1M (config[4] indexer stage)", file=sys.stderr, flush=True)
        rl = run_indexer(1 << 20, args.ratio, args.top_k, args.chunk_s, args.chunk_t, 1, 1)
        extra["s1m_ms"] = rl["ms"]
        extra["s1m_tflops"] = rl["flops"] / (rl["ms"] * 1e-3) / 1e12
        extra["s1m_peak_hbm_gib"] = rl["peak_gib"]
        extra["reference_h200_ms_s1m"] = REF_H200_MS[1048576]
        del rl
        torch.cuda.empty_cache()
    if not args.no_indexer_q:
        print("[bench] fp4/fp8 indexer S=64K and S=1M", file=sys.stderr, flush=True)
        extra["indexer_q_s64k"] = run_indexer_q(65536, args.ratio, args.top_k, 5, 1)
        if not args.no_long:
            extra["indexer_q_s1m"] = run_indexer_q(1 << 20, args.ratio, args.top_k, 1, 1, parity_rows=64)
        torch.cuda.empty_cache()
    if not args.no_attn:
        print("[bench] sparse attention config[3]", file=sys.stderr, flush=True)
        ra = run_sparse_attn(65536, 16384, 64, 576, 512, 3, 1, bwd=not args.no_attn_bwd)
        extra["sparse_attn_ms"] = ra["ms"]
        if "bwd_ms" in ra:
            extra["sparse_attn_bwd_ms"] = ra["bwd_ms"]
            extra["sparse_attn_bwd_tflops"] = ra["bwd_flops"] / (ra["bwd_ms"] * 1e-3) / 1e12
            extra["sparse_attn_bwd_mfma_frac"] = extra["sparse_attn_bwd_tflops"] / PEAK_BF16_TFLOPS
            extra["sparse_attn_bwd_peak_extra_gib"] = ra["bwd_peak_extra_gib"]
            extra["sparse_attn_bwd_parity"] = ra["bwd_parity"]
        extra["sparse_attn_tflops"] = ra["flops"] / (ra["ms"] * 1e-3) / 1e12
        extra["sparse_attn_unique_gbps"] = ra["unique_bytes"] / (ra["ms"] * 1e-3) / 1e9
        extra["sparse_attn_hbm_frac"] = extra["sparse_attn_unique_gbps"] / PEAK_HBM_GBPS
        extra["sparse_attn_mfma_frac"] = extra["sparse_attn_tflops"] / PEAK_BF16_TFLOPS

    if not args.no_e2e:
        print("[bench] end-to-end CSA forward S=64K", file=sys.stderr, flush=True)
        extra["csa_e2e_s64k"] = run_csa_e2e(65536, 3, 1, 256, bwd=not args.no_attn_bwd)
        print("[bench] end-to-end CSA forward S=1M (config[4])", file=sys.stderr, flush=True)
        extra["csa_e2e_s1m"] = run_csa_e2e(1 << 20, 1, 1, args.e2e_parity_rows)
        print("[bench] end-to-end CSA forward S=1M with the fp4/fp8 indexer", file=sys.stderr, flush=True)
        extra["csa_e2e_s1m_quantized_indexer"] = run_csa_e2e(1 << 20, 1, 1, 256, quantized=True)
        print("[bench] end-to-end HCA forward S=64K", file=sys.stderr, flush=True)
        extra["hca_e2e_s64k"] = run_hca_e2e(65536, 3, 1, 8, bwd=not args.no_attn_bwd)

    traffic = None
    tfile = {}
    if os.path.exists(TRAFFIC_FILE):
        try:
            with open(TRAFFIC_FILE) as f:
                tfile = json.load(f)
            traffic = tfile.get("indexer_topk_c1_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    if "sparse_attn_ms" in extra and tfile.get("sparse_attn_c3_bytes_per_launch"):
        # fabric bytes per launch (HBM byte counters: L2-missing gathers, q, o, indices) over the
        # measured time: the bound of this kernel on random indices
        fab = tfile["sparse_attn_c3_bytes_per_launch"] / (extra["sparse_attn_ms"] * 1e-3) / 1e9
        extra["sparse_attn_fabric_gbps"] = fab
        extra["sparse_attn_fabric_frac"] = fab / PEAK_HBM_GBPS

    line = {
        "metric": "V4-Flash indexer ms @S=64K/1M, MFMA util %, peak HBM GB (1 GPU)",
        "value": round(r["ms"], 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)-scaled bf16 q/k_idx, N(0,1) fp32 weights)",
        "config": {"workload": "v4_flash_indexer_c1", "B": 1, "S": args.seq, "T": args.seq // args.ratio,
                   "H_I": 64, "D_I": 128, "top_k": args.top_k, "causal_ratio": args.ratio,
                   "chunk_s": args.chunk_s, "chunk_t": args.chunk_t},
        "mfma_util_pct": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "peak_hbm_gib": round(r["peak_gib"], 4),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "kernel": "indexer_topk_kernel", "flops_per_launch": r["flops"]},
        "parity": {k: par[k] for k in ("rows", "recall_mean", "recall_min", "exact_rows_frac")},
        "cpu_baseline": {"value": round(cpu_ms_full, 1), "unit": "ms (extrapolated to the full S=64K job)",
                         "cores": threads, "kind": "port",
                         "sample": f"{par['rows']} sampled query rows of config[1] through the C oracle "
                                   f"(scores in double + top-k), {par['cpu_s']:.2f} s measured, scaled by "
                                   f"legal (s,t) pairs"},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
