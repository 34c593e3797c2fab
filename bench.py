"""Benchmark of the StreamIndex MI355X hot path.

Metric: V4-Flash indexer ms at S=64K and S=1M, MFMA utilisation, peak HBM.
Default workload (config[1]): the V4-Flash indexer on one MI355X,
B=1, S=65,536, H_I=64, D_I=128, T=16,384, top_k=512, causal_ratio=4,
chunk_s=2048, chunk_t=8192, seeded bf16/fp32 synthetic inputs resident in HBM.
One "step" = one ``chunked_indexer_topk`` call (one launch of the fused
score + top-k kernel).

Printed (one JSON line, rank 0):
  value          ms per call at S=64K (lower is better)
  roofline       MFMA bound of the dominant kernel: algorithmic FLOPs
                 (2·H_I·D_I per causally legal (s,t) pair) / mean kernel time
                 from HIP events on the launch stream, vs 2516.6 TFLOP/s;
                 traffic = HBM bytes per launch from this run's FETCH_SIZE /
                 WRITE_SIZE counters (scaled by a plain copy's readings)
  counters       rocprofv3 passes run by this bench in a child process on the
                 same GPU: MFMA-busy fraction and shader clock of the indexer
                 at config[1], HBM bytes of the indexer and of config[3]
  peak_hbm_gib   max_memory_allocated delta during one call (inputs excluded)
  parity         config[1] against the CPU oracle on 4,096 sampled rows:
                 recall, exact sets where the k-th gap is wide, score error
  cpu_baseline   the reference's CPU path (fp32 torch materialise -> mask ->
                 topk -> post-mask, oracle/torch_materialize.py) run in full
                 at config[0] on this host, 1 warm-up + 3 timed, scaled to
                 the config[1] job by dense (s,t) pairs
  extra          config[0] on the GPU; config[2] (S=262,144) with its chunk
                 pairs and top_k sweep; S=1M (config[4] indexer stage) at
                 top_k 512 and 1024; the fp4/fp8 indexer; sparse attention at
                 config[3] on config[1]'s own indexer output with sampled
                 parity (and on random indices); its backward; the end-to-end
                 CSA forward at S=64K and S=1M (config[4]); the HCA forward
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
                             flash_csa_forward, flash_hca_forward, sparse_attn_bwd, sparse_attn_fwd,
                             sparse_attn_kv2)
from streamindex_amd import synth  # noqa: E402
from streamindex_amd import _lib  # noqa: E402
import importlib  # noqa: E402

# (the package re-exports the function sparse_attn under the module's name)
sparse_attn_mod = importlib.import_module("streamindex_amd.sparse_attn")
from streamindex_amd.csa import csa_row_len  # noqa: E402
from streamindex_amd.hca import hca_row_len  # noqa: E402

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5033.2   # MI355X dense fp8 MFMA (the fp4 x fp8 product runs at the fp8 rate)
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E
# Reference timings on one H200 (other hardware; context only):
# benchmarks/results/2026-04-27/scaling_v4_flash_indexer_final.log:10,12,14
REF_H200_MS = {65536: 122.2, 262144: 1935.3, 1048576: 30899.6}
REF_H200_GIB = {65536: 0.59, 262144: 1.71, 1048576: 6.21}
# top_k sweep at S=262,144: benchmarks/results/2026-05-01/RESULTS.md:35-42
REF_H200_TOPK_S256K_MS = {64: 1754, 256: 1881, 512: 1934, 1024: 1996, 2048: 2217}
# V4-Pro point, top_k=1024 at S=1M: RESULTS.md:86-96 (ms, GiB)
REF_H200_S1M_K1024 = (31973.3, 12.27)
# Backward workspace caps timed at config[3] (GiB)
BWD_SWEEP_GIB = (1, 2, 4, 8)



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
    """config[1] against the CPU oracle on `nrows` sampled rows: recall, the
    exact-set gate where the oracle's k-th gap is wide (1e-4 of the row scale),
    the score error at every returned index, and the C oracle's own time on
    those rows (a secondary, labelled CPU figure)."""
    from oracle import oracle as O

    S = q.shape[1]
    T = k.shape[1]
    rng = np.random.default_rng(seed)
    rows = np.sort(rng.choice(S, size=min(nrows, S), replace=False)).astype(np.int64)
    sel = torch.from_numpy(rows).to(q.device)
    qb = _bits(q[0, sel])
    kb = _bits(k[0])
    wb = w[0, sel].float().cpu().numpy()
    local = np.arange(len(rows), dtype=np.int64)
    O.lib()
    t0 = time.perf_counter()
    lim = O.legal_limits(rows, T, ratio)
    scores = O.indexer_scores(qb, kb, wb, local, lim=lim)  # rows' own q/w are packed densely
    ref_idx, ref_val = O.topk(scores, lim, top_k)
    cpu_s = time.perf_counter() - t0
    got = idx[0, sel].cpu().numpy()
    got_v = sc[0, sel].cpu().numpy().astype(np.float64)
    rec = O.set_overlap_recall(ref_idx, got)
    # score of every returned (row, index) against the oracle's fp64 score there
    valid = got >= 0
    rr, cc = np.nonzero(valid)
    ref_at = scores[rr, got[rr, cc]]
    row_scale = np.array([np.abs(scores[r, :max(1, int(lim[r]))]).mean() if lim[r] > 0 else 1.0
                          for r in range(len(rows))])
    rel = np.abs(got_v[rr, cc] - ref_at) / (np.abs(ref_at) + row_scale[rr])
    # exact index set wherever the k-th / (k+1)-th gap exceeds 1e-4 of the row scale
    wide = np.zeros(len(rows), dtype=bool)
    for r in range(len(rows)):
        n_leg = int(lim[r])
        if n_leg <= top_k:
            wide[r] = True  # every legal key is selected: the set is forced
            continue
        kth = ref_val[r, top_k - 1]
        legal = scores[r, :n_leg]
        below = legal[legal < kth]
        nxt = below.max() if below.size else -np.inf
        wide[r] = np.sum(legal >= kth) == top_k and (kth - nxt) > 1e-4 * row_scale[r]
    return {
        "rows": int(len(rows)),
        "recall_mean": float(rec.mean()),
        "recall_min": float(rec.min()),
        "exact_rows_frac": float((rec == 1.0).mean()),
        "wide_gap_rows": int(wide.sum()),
        "wide_gap_rows_exact": int((rec[wide] == 1.0).sum()),
        "max_score_rel_err": float(rel.max()) if rel.size else 0.0,
        "cpu_s": cpu_s,
        "pairs_sample": float(np.minimum(lim, T).sum()),
    }


def cpu_baseline_c0(ratio, top_k):
    """The reference's CPU path (oracle/torch_materialize.py: fp32 einsum ->
    ReLU -> weighted head sum -> mask -> topk -> post-mask) run in full at
    config[0] on this host: 1 warm-up + 3 timed runs."""
    from oracle.torch_materialize import time_materialize

    q, k, w = synth.indexer_inputs(1, 4096, 64, 128, ratio=ratio, seed=2026, device="cpu")
    res = time_materialize(q, k, w, top_k, ratio, warmup=1, repeats=3)
    res.pop("out")
    return res


def run_c0_gpu(ratio, top_k, steps):
    """config[0] (S=4,096) on the GPU, for the same-workload comparison with the CPU baseline."""
    dev = torch.device("cuda:0")
    q, k, w = synth.indexer_inputs(1, 4096, 64, 128, ratio=ratio, seed=2026, device=dev)
    fn = lambda: chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio)  # noqa: E731
    fn()
    torch.cuda.synchronize()
    return _events_time(fn, steps, torch.cuda.current_stream(dev))


def run_indexer(S, ratio, top_k, chunk_s, chunk_t, steps, warmup, H=64, D=128, seed=2026):
    dev = torch.device("cuda:0")
    q, k, w = synth.indexer_inputs(1, S, H, D, ratio=ratio, seed=seed, device=dev)
    T = k.shape[1]
    fn = lambda: chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio, chunk_s=chunk_s, chunk_t=chunk_t)  # noqa: E731
    # (the peak-memory probe empties the allocator cache and idles the GPU, so
    # it runs before the warm-up: the timed calls follow the warm-up directly)
    peak = _peak_gib(fn)
    for _ in range(max(1, warmup)):
        out = fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    t0 = time.perf_counter()
    ms = _events_time(fn, steps, stream)
    wall = (time.perf_counter() - t0) * 1e3 / steps
    flops = synth.indexer_flops(S, T, H, D, ratio)
    idx, sc = fn()
    torch.cuda.synchronize()
    return dict(q=q, k=k, w=w, T=T, ms=ms, wall_ms=wall, peak_gib=peak, flops=flops, idx=idx, sc=sc)


def run_indexer_sweep(q, k, w, ratio, top_ks, steps):
    """chunked_indexer_topk at each top_k on the same resident inputs: ms
    (HIP events), TFLOP/s and peak HBM (outputs; the kernel needs no workspace)."""
    dev = q.device
    S, T, H, D = q.shape[1], k.shape[1], q.shape[2], q.shape[3]
    flops = synth.indexer_flops(S, T, H, D, ratio)
    out = {}
    for kk in top_ks:
        fn = lambda: chunked_indexer_topk(q, k, w, kk, causal_ratio=ratio, chunk_s=2048, chunk_t=8192)  # noqa: E731
        peak = _peak_gib(fn)
        fn()
        torch.cuda.synchronize()
        ms = _events_time(fn, steps, torch.cuda.current_stream(dev))
        out[str(kk)] = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12,
                        "mfma_frac": flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "peak_hbm_gib": peak}
    return out


def run_c2(ratio, steps):
    """config[2]: S=262,144, T=65,536 — time, TFLOP/s and peak HBM at top_k=512;
    the reference's chunk pairs give bit-identical outputs; the top_k sweep of
    benchmarks/results/2026-05-01/RESULTS.md:35-42 (H200 figures beside)."""
    S = 262144
    r = run_indexer(S, ratio, 512, 2048, 8192, steps, 1)
    q, k, w = r["q"], r["k"], r["w"]
    res = {"S": S, "T": r["T"], "ms": r["ms"], "tflops": r["flops"] / (r["ms"] * 1e-3) / 1e12,
           "mfma_frac": r["flops"] / (r["ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "peak_hbm_gib": r["peak_gib"],
           "reference_h200_ms": REF_H200_MS[S], "reference_h200_gib": REF_H200_GIB[S]}
    same = True
    for cs, ct in ((1024, 4096), (8192, 32768)):
        i2, s2 = chunked_indexer_topk(q, k, w, 512, causal_ratio=ratio, chunk_s=cs, chunk_t=ct)
        same = same and bool(torch.equal(i2, r["idx"])) and bool(torch.equal(s2, r["sc"]))
        del i2, s2
    res["chunk_pairs_identical"] = same
    del r["idx"], r["sc"]
    sweep = run_indexer_sweep(q, k, w, ratio, (64, 256, 512, 1024, 2048), max(2, steps))
    for kk, v in sweep.items():
        v["reference_h200_ms"] = REF_H200_TOPK_S256K_MS[int(kk)]
    res["top_k_sweep"] = sweep
    del q, k, w, r
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# Hardware counters of this run (rocprofv3 in a child process, same GPU)
# ---------------------------------------------------------------------------
# One pass per counter group (rocprofv3 does not split counters over passes):
# the MFMA pass stays within 8 SQ and 2 GRBM counters, FETCH_SIZE takes 3 of
# the 4 TCC counters and WRITE_SIZE 2, so they run separately.
# The MFMA pass also runs the S = 1M indexer (the north-star shape); the byte
# passes do not need it.
COUNTER_PASSES = (
    ("mfma", ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "GRBM_GUI_ACTIVE", "GRBM_COUNT"), True),
    ("fetch", ("FETCH_SIZE",), False),
    ("write", ("WRITE_SIZE",), False),
)
N_SIMD = 1024           # 256 CUs x 4 SIMDs
N_XCD = 8               # GRBM_GUI_ACTIVE is summed over the XCDs
MFMA_FLOP = 32 * 32 * 16 * 2   # v_mfma_f32_32x32x16_bf16
COPY_MIB = 1024         # plain device copy used to scale the byte counters


S1M = 1 << 20


def counter_child(ratio=4, top_k=512, s1m=False):
    """The workload the counter passes profile: with `s1m` first the S = 1M
    indexer (1 warm-up + 2 launches), then config[1]'s indexer (1 warm-up + 3
    launches), sparse attention at config[3] on its output (1 + 2), and a
    plain 1 GiB device copy (x3) that calibrates the byte counters."""
    dev = torch.device("cuda:0")
    if s1m:
        q, k, w = synth.indexer_inputs(1, S1M, 64, 128, ratio=ratio, seed=2026, device=dev)
        for _ in range(3):
            idx, sc = chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio, chunk_s=2048, chunk_t=8192)
            del idx, sc
        torch.cuda.synchronize()
        del q, k, w
        torch.cuda.empty_cache()
    q, k, w = synth.indexer_inputs(1, 65536, 64, 128, ratio=ratio, seed=2026, device=dev)
    for _ in range(4):
        idx, _ = chunked_indexer_topk(q, k, w, top_k, causal_ratio=ratio, chunk_s=2048, chunk_t=8192)
    torch.cuda.synchronize()
    del q, k, w
    qa, kv, sink = synth.sparse_attn_inputs(1, 65536, 64, 576, 16384, seed=2027, device=dev)
    for _ in range(3):
        o, lse = sparse_attn_fwd(qa, kv, sink, idx, 576 ** -0.5)
    torch.cuda.synchronize()
    del qa, kv, o, lse, idx
    n = COPY_MIB * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def _read_counters(path):
    """rocprofv3 counter CSV -> {dispatch id: {"kernel", "ns", counter: value}}."""
    import csv

    out = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            d = out.setdefault(int(row["Dispatch_Id"]), {"kernel": row["Kernel_Name"],
                                                         "ns": int(row["End_Timestamp"]) - int(row["Start_Timestamp"])})
            d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    return out


def _pick(disp, name, last):
    rows = [v for _, v in sorted(disp.items()) if name in v["kernel"]]
    return rows[-last:]


def _pick_first(disp, name, skip, count):
    rows = [v for _, v in sorted(disp.items()) if name in v["kernel"]]
    return rows[skip:skip + count]


def _mfma_summary(rows, flops):
    """Clock, MFMA-busy fraction and counter-derived utilisation of dispatches
    from the MFMA pass (busy cycles over 1,024 SIMDs; GRBM_GUI_ACTIVE summed
    over 8 XCDs)."""
    ns = float(np.mean([v["ns"] for v in rows]))
    cyc = float(np.mean([v["GRBM_GUI_ACTIVE"] for v in rows])) / N_XCD
    busy = float(np.mean([v["SQ_VALU_MFMA_BUSY_CYCLES"] for v in rows]))
    insts = float(np.mean([v["SQ_INSTS_MFMA"] for v in rows]))
    return {
        "kernel": rows[0]["kernel"].split("(")[0],
        "dispatches": len(rows), "avg_ms": ns * 1e-6,
        "clock_ghz": cyc / ns,
        "mfma_busy_pct": 100.0 * busy / N_SIMD / cyc,
        "mfma_insts": insts,
        "executed_mfma_flops": insts * MFMA_FLOP,
        "algorithmic_flops": flops,
        "mfma_util_pct_from_counters": 100.0 * insts * MFMA_FLOP / (ns * 1e-9) / 1e12 / PEAK_BF16_TFLOPS,
        "mfma_util_pct_from_time": 100.0 * flops / (ns * 1e-9) / 1e12 / PEAK_BF16_TFLOPS,
        "valu_per_mfma": float(np.mean([v["SQ_INSTS_VALU"] for v in rows])) / max(insts, 1.0),
    }


def run_counters(timeout=240):
    """Runs the counter passes over `counter_child` under rocprofv3 and returns
    the indexer's MFMA-busy fraction, shader clock and counter-derived MFMA
    utilisation, and the HBM bytes per launch of the indexer and of config[3]'s
    attention (byte counters scaled by what they read for a plain copy)."""
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        return {"error": "rocprofv3 not found"}
    tmp = tempfile.mkdtemp(prefix="si_pmc_", dir="/tmp")
    env = dict(os.environ, TMPDIR="/tmp")
    passes = {}
    for name, ctrs, s1m in COUNTER_PASSES:
        d = os.path.join(tmp, name)
        cmd = [prof, "--pmc", *ctrs, "--output-format", "csv", "-d", d, "-o", "pmc", "--",
               sys.executable, os.path.abspath(__file__), "--counter-child"] + (["--counter-s1m"] if s1m else [])
        print(f"[bench] counter pass {name}: {' '.join(ctrs)}", file=sys.stderr, flush=True)
        p = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                             start_new_session=True)
        try:
            log, _ = p.communicate(timeout=timeout)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.wait()
            return {"error": f"counter pass {name} timed out after {timeout} s"}
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            return {"error": f"counter pass {name}: no counter file (rc {p.returncode})",
                    "log_tail": log.decode("utf-8", "replace")[-600:]}
        passes[name] = _read_counters(files[0])
    res = {"passes": [" ".join(c) for _, c, _ in COUNTER_PASSES],
           "cmd": "rocprofv3 --pmc <pass> --output-format csv -- python3 bench.py --counter-child "
                  "[--counter-s1m: MFMA pass]"}
    # The S = 1M launches come first in the MFMA pass: the first three
    # indexer dispatches, of which the first is the warm-up.  config[1]'s are
    # the last three (after its own warm-up).
    s1m = _pick_first(passes["mfma"], "indexer_topk", 1, 2)
    if len(s1m) == 2:
        res["indexer_s1m"] = _mfma_summary(s1m, synth.indexer_flops(S1M, S1M // 4, 64, 128, 4))
    idx = _pick(passes["mfma"], "indexer_topk", 3)
    if idx:
        res["indexer_c1"] = _mfma_summary(idx, synth.indexer_flops(65536, 16384, 64, 128, 4))
    copies = _pick(passes["fetch"], "copyBuffer", 3)
    wcopies = _pick(passes["write"], "copyBuffer", 3)
    if copies and wcopies:
        nbytes = COPY_MIB * (1 << 20)
        fscale = nbytes / (float(np.mean([v["FETCH_SIZE"] for v in copies])) * 1024.0)
        wscale = nbytes / (float(np.mean([v["WRITE_SIZE"] for v in wcopies])) * 1024.0)
        res["fetch_scale"], res["write_scale"] = fscale, wscale
        for key, kname, last in (("indexer_c1", "indexer_topk", 3), ("sparse_attn_c3", "sparse_attn_fwd_kernel", 2)):
            f = _pick(passes["fetch"], kname, last)
            wr = _pick(passes["write"], kname, last)
            if f and wr:
                fb = float(np.mean([v["FETCH_SIZE"] for v in f])) * 1024.0 * fscale
                wb = float(np.mean([v["WRITE_SIZE"] for v in wr])) * 1024.0 * wscale
                res.setdefault(key, {}).update({"hbm_read_bytes": fb, "hbm_write_bytes": wb,
                                                "hbm_bytes_per_launch": fb + wb})
    return res


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


def run_indexer_score(S, steps, warmup, ratio=4, H=64, D=128, seed=2026, parity_rows=16):
    """The materialised-score operator (`indexer_score`: every (s, t) pair, no
    mask, as the reference kernel) at config[1]'s shape: S x T fp32 scores
    (4 GiB at S = 64K).  Dense work 2*H*D per pair; its output writes bound it
    below the MFMA time only for much longer rows.  Sampled rows are checked
    against the oracle's float64 scores (the tests' 1e-4 relative gate)."""
    from oracle import oracle as O
    from streamindex_amd import indexer_score

    dev = torch.device("cuda:0")
    q, k, w = synth.indexer_inputs(1, S, H, D, ratio=ratio, seed=seed, device=dev)
    T = k.shape[1]
    fn = lambda: indexer_score(q, k, w)  # noqa: E731
    for _ in range(max(1, warmup)):
        out = fn()
    del out
    torch.cuda.synchronize()
    ms = _events_time(fn, steps, torch.cuda.current_stream(dev))
    sc = fn()
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(11).choice(S, size=min(parity_rows, S), replace=False)).astype(np.int64)
    ref = O.indexer_scores(_bits(q[0]), _bits(k[0]), w[0].float().cpu().numpy(), rows)
    got = sc[0, torch.from_numpy(rows).to(dev)].double().cpu().numpy()
    scale = np.abs(ref).mean(axis=1, keepdims=True)
    err = float((np.abs(got - ref) / (np.abs(ref) + scale)).max())
    flops = 2.0 * H * D * S * T
    out_bytes = 4.0 * S * T
    del sc, q, k, w
    torch.cuda.empty_cache()
    return {"S": S, "T": T, "ms": ms, "tflops": flops / (ms * 1e-3) / 1e12,
            "mfma_frac": flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
            "write_gbps": out_bytes / (ms * 1e-3) / 1e9, "output_gib": out_bytes / 2 ** 30,
            "parity_rows": int(len(rows)), "max_rel_err": err, "pass": err < 1e-4}


def attn_parity(q, kv, sink, idx, o, lse, nrows=64, seed=33):
    """Sampled rows of a sparse-attention output against the oracle over the
    same index rows: max |o - o_ref| (gate 2e-2) and max |lse - lse_ref|."""
    from oracle import oracle as O

    S, D = q.shape[1], q.shape[3]
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, 3, 4, S - 1], rng.choice(S, size=min(nrows, S), replace=False)]))
    sel = torch.from_numpy(rows).to(q.device)
    ir = idx[0, sel].long()
    uniq = torch.unique(ir[ir >= 0])
    remap = torch.where(ir >= 0, torch.searchsorted(uniq, ir.clamp(min=0)), torch.full_like(ir, -1))
    ro, rl = O.sparse_attn_rows(_bits(q[0, sel]), _bits(kv[0, uniq]), sink.cpu().numpy(), remap.cpu().numpy(),
                                D ** -0.5)
    oe = float(np.abs(o[0, sel].float().cpu().numpy() - ro).max())
    le = float(np.abs(lse[0, sel].cpu().numpy() - rl).max())
    return {"rows": int(len(rows)), "o_max_abs_err": oe, "lse_max_abs_err": le, "pass": bool(oe <= 2e-2 and le <= 2e-3)}


def run_sparse_attn(S, T, H, D, top_k, steps, warmup, idx=None, bwd=False, fwd=True, parity_rows=0, bwd_cap=None,
                    sweep=True):
    """Forward (and optionally backward) sparse attention at one shape, on the
    given indices (config[3]: config[1]'s indexer output) or on random distinct
    causal ones.  The backward is timed from the forward's saved (o, lse) with
    dO ~ N(0,1)·0.5, including its key sort and reduction; its FLOPs count the
    five products per selected (row, key) pair (S and dP recomputed, dQ, dK,
    dV): 10 H D."""
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
        if parity_rows:
            o, lse = fn()
            torch.cuda.synchronize()
            res["parity"] = attn_parity(q, kv, sink, idx, o, lse, parity_rows)
            del o, lse
    if bwd:
        o, lse = fn()
        g = torch.Generator(device=dev)
        g.manual_seed(2028)
        do = torch.randn(q.shape, generator=g, device=dev, dtype=torch.bfloat16).mul_(0.5)
        def bfn(cap=bwd_cap):
            return sparse_attn_bwd(q, kv, sink, idx, o, lse, do, D ** -0.5, workspace_bytes=cap)

        for _ in range(max(1, warmup)):
            bfn()  # (each call's gradients are freed before the next call)
        torch.cuda.synchronize()
        res["bwd_ms"] = _events_time(bfn, steps, stream)
        res["bwd_flops"] = 10.0 * H * D * nvalid
        # memory one call adds beyond its inputs: dq, dkv, dsink and the workspace
        res["bwd_peak_extra_gib"] = _peak_gib(bfn)
        res["bwd_workspace_cap_gib"] = sparse_attn_mod.BWD_WORKSPACE_CAP / 2 ** 30
        swept = []
        for cap_gib in (BWD_SWEEP_GIB if sweep else ()):
            f = lambda: bfn(cap_gib << 30)  # noqa: E731
            f()
            torch.cuda.synchronize()
            swept.append({"workspace_cap_gib": cap_gib, "ms": _events_time(f, max(3, steps // 2), stream),
                          "peak_extra_gib": _peak_gib(f)})
        res["bwd_workspace_sweep"] = swept
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
    o = sparse_attn_kv2(q[:, sel], kv, kvc, sink, rows_gpu[:, sel], None)
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
    peak = _peak_gib(fn)
    for _ in range(max(1, warmup)):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    ms = _events_time(fn, steps, stream)
    # stage split of one call (the two steps flash_csa_forward runs; the
    # attention reads kv and kv_compressed in place)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record(stream)
    rows_gpu = csa_topk_idxs(qi, ki, w, n_win=n_win, top_k=top_k, m=m, seq_len=S, quantized=quantized)
    row_len = csa_row_len(1, S, n_win, top_k, S // m, m, dev)
    ev[1].record(stream)
    o = sparse_attn_kv2(q, kv, kvc, sink, rows_gpu, None, row_len=row_len)
    ev[2].record(stream)
    torch.cuda.synchronize()
    del o
    nvalid = float((rows_gpu >= 0).sum().item())
    res = {
        "S": S, "T": S // m, "n_h": n_h, "d": d, "n_win": n_win, "top_k": top_k,
        "ms": ms, "peak_hbm_gib": peak,
        "indexer_ms": ev[0].elapsed_time(ev[1]), "attn_ms": ev[1].elapsed_time(ev[2]),
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
        leaves = (qg, kvg, kvcg, sg)
        # autograd.grad returns the gradients without accumulating into .grad
        grads = torch.autograd.grad(og, leaves, do, retain_graph=True)
        del grads
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            grads = torch.autograd.grad(og, leaves, do, retain_graph=True)
            del grads
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
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record(stream)
    rows_gpu = build_hca_topk_idxs(B=1, seq_len=S, n_win=n_win, n_compressed=T, m_prime=m_prime, device=dev)
    row_len = hca_row_len(1, S, n_win, T, m_prime, dev)
    ev[1].record(stream)
    o = sparse_attn_kv2(q, kv, kvc, sink, rows_gpu, None, row_len=row_len)
    ev[2].record(stream)
    torch.cuda.synchronize()
    del o
    nvalid = float((rows_gpu >= 0).sum().item())
    K = n_win + T
    res = {
        "S": S, "T": T, "n_h": n_h, "d": d, "n_win": n_win, "m_prime": m_prime, "K": K, "ms": ms,
        "rows_ms": ev[0].elapsed_time(ev[1]), "attn_ms": ev[1].elapsed_time(ev[2]),
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
        leaves = (qg, kvg, kvcg, sg)
        grads = torch.autograd.grad(og, leaves, do, retain_graph=True)
        del grads
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            grads = torch.autograd.grad(og, leaves, do, retain_graph=True)
            del grads
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
    # (ten warm-up calls: from idle the clock takes about that many config[1]
    # calls to ramp up, 8.7 -> 7.2 ms per call)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seq", type=int, default=65536)
    ap.add_argument("--top-k", type=int, default=512)
    ap.add_argument("--ratio", type=int, default=4)
    ap.add_argument("--chunk-s", type=int, default=2048)
    ap.add_argument("--chunk-t", type=int, default=8192)
    ap.add_argument("--parity-rows", type=int, default=4096)
    ap.add_argument("--no-long", action="store_true", help="skip the S=1M indexer measurements")
    ap.add_argument("--no-c2", action="store_true", help="skip the S=262,144 (config[2]) measurements")
    ap.add_argument("--no-attn", action="store_true", help="skip the sparse-attention measurement")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (config[0] on the host)")
    ap.add_argument("--no-counters", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--counter-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--counter-s1m", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--only-indexer", action="store_true", help="indexer timing only (for profilers)")
    ap.add_argument("--only-attn", action="store_true",
                    help="config[3] sparse-attention timing only, on config[1]'s indexer output (for profilers)")
    ap.add_argument("--only-attn-random", action="store_true",
                    help="sparse-attention timing on random causal indices only (for profilers)")
    ap.add_argument("--idx-order", choices=("given", "sorted"), default="given",
                    help="with --only-attn: the indexer's order (best score first) or each row sorted by key "
                         "(descending, -1 last)")
    ap.add_argument("--idx-int32", action="store_true", help="with --only-attn: int32 instead of int64 indices")
    ap.add_argument("--only-attn-bwd", action="store_true", help="sparse-attention backward timing only (for profilers)")
    ap.add_argument("--bwd-workspace-gib", type=float, default=0.0, metavar="GIB",
                    help="with --only-attn-bwd: cap the backward's workspace at GIB (default: the library's cap)")
    ap.add_argument("--only-indexer-q", type=int, default=0, metavar="S",
                    help="fp4/fp8 indexer timing only at sequence length S (for profilers)")
    ap.add_argument("--no-indexer-q", action="store_true", help="skip the fp4/fp8 indexer measurements")
    ap.add_argument("--no-score", action="store_true", help="skip the materialised-score (indexer_score) leg")
    ap.add_argument("--only-score", action="store_true", help="indexer_score timing only (for profilers)")
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
    if args.counter_child:
        counter_child(args.ratio, args.top_k, s1m=args.counter_s1m)
        return
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
    if args.only_score:
        print(json.dumps(run_indexer_score(65536, args.steps, args.warmup, args.ratio)), flush=True)
        return
    if args.only_attn_bwd:
        ri = run_indexer(65536, args.ratio, args.top_k, args.chunk_s, args.chunk_t, 1, 1)
        idx = ri["idx"]
        del ri
        cap = int(args.bwd_workspace_gib * (1 << 30)) if args.bwd_workspace_gib > 0 else None
        ra = run_sparse_attn(65536, 16384, 64, 576, 512, args.steps, args.warmup, idx=idx, bwd=True, fwd=False,
                             bwd_cap=cap, sweep=False)
        print(json.dumps({"sparse_attn_bwd_ms": ra["bwd_ms"], "tflops": ra["bwd_flops"] / ra["bwd_ms"] / 1e9,
                          "peak_extra_gib": ra["bwd_peak_extra_gib"], "parity": ra["bwd_parity"]}), flush=True)
        return
    if args.only_attn or args.only_attn_random:
        idx = None
        if args.only_attn:
            ri = run_indexer(65536, args.ratio, args.top_k, args.chunk_s, args.chunk_t, 1, 1)
            idx = ri["idx"]
            del ri
            if args.idx_order == "sorted":
                # the same keys per row (the result does not depend on their order)
                idx = torch.sort(idx, dim=-1, descending=True).values
            if args.idx_int32:
                idx = idx.to(torch.int32)
            torch.cuda.empty_cache()
        ra = run_sparse_attn(65536, 16384, 64, 576, 512, args.steps, args.warmup, idx=idx)
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

    def say(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    say(f"indexer S={args.seq} warmup={args.warmup} steps={args.steps}")
    r = run_indexer(args.seq, args.ratio, args.top_k, args.chunk_s, args.chunk_t, args.steps, args.warmup)
    if args.only_indexer:
        print(json.dumps({"indexer_ms": r["ms"], "tflops": r["flops"] / r["ms"] / 1e9}), flush=True)
        return
    tflops = r["flops"] / (r["ms"] * 1e-3) / 1e12
    say(f"indexer {r['ms']:.3f} ms, {tflops:.1f} TFLOP/s")

    say(f"parity on {args.parity_rows} sampled rows")
    par = indexer_parity_and_cpu(r["q"], r["k"], r["w"], r["idx"], r["sc"], args.ratio, args.top_k,
                                 args.parity_rows)
    total_pairs = synth.legal_pairs(args.seq, r["T"], args.ratio)
    port_ms_full = par["cpu_s"] * 1e3 * total_pairs / max(1.0, par["pairs_sample"])
    c1_idx = r["idx"]  # config[3]'s indices: config[1]'s own indexer output
    del r["q"], r["k"], r["w"], r["sc"], r["idx"]
    torch.cuda.empty_cache()

    extra = {"indexer_wall_ms_per_call": r["wall_ms"], "reference_h200_ms_s64k": REF_H200_MS[65536],
             "reference_h200_gib_s64k": REF_H200_GIB[65536]}
    extra["c0_gpu_ms"] = run_c0_gpu(args.ratio, args.top_k, max(5, args.steps))
    cpu = None
    if not args.no_cpu:
        say("cpu baseline: the reference's fp32 materialise path at config[0] on the host")
        cpu = cpu_baseline_c0(args.ratio, args.top_k)

    if not args.no_attn:
        say("sparse attention config[3] on config[1]'s indexer output")
        ra = run_sparse_attn(65536, 16384, 64, 576, 512, 10, 5, idx=c1_idx, bwd=not args.no_attn_bwd,
                             parity_rows=64)
        c3 = {"indices": "config[1] chunked_indexer_topk output (int64, -1 past the causal count)",
              "ms": ra["ms"], "tflops": ra["flops"] / (ra["ms"] * 1e-3) / 1e12,
              "mfma_frac": ra["flops"] / (ra["ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
              "unique_gbps": ra["unique_bytes"] / (ra["ms"] * 1e-3) / 1e9,
              "valid_keys": ra["nvalid"], "parity": ra["parity"]}
        c3["hbm_frac"] = c3["unique_gbps"] / PEAK_HBM_GBPS
        if "bwd_ms" in ra:
            c3["bwd"] = {"ms": ra["bwd_ms"], "tflops": ra["bwd_flops"] / (ra["bwd_ms"] * 1e-3) / 1e12,
                         "mfma_frac": ra["bwd_flops"] / (ra["bwd_ms"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         "peak_extra_gib": ra["bwd_peak_extra_gib"],
                         "default_workspace_cap_gib": ra["bwd_workspace_cap_gib"],
                         "workspace_sweep": ra["bwd_workspace_sweep"], "parity": ra["bwd_parity"]}
        extra["sparse_attn_c3"] = c3
        del ra
        torch.cuda.empty_cache()
        say("sparse attention on random causal indices (secondary)")
        rr = run_sparse_attn(65536, 16384, 64, 576, 512, 10, 5)
        extra["sparse_attn_random_idx"] = {"ms": rr["ms"], "tflops": rr["flops"] / (rr["ms"] * 1e-3) / 1e12,
                                           "unique_gbps": rr["unique_bytes"] / (rr["ms"] * 1e-3) / 1e9}
        del rr
    del c1_idx
    torch.cuda.empty_cache()

    if not args.no_c2:
        say("config[2]: indexer S=262144, chunk pairs, top_k sweep")
        extra["c2_s256k"] = run_c2(args.ratio, 2)

    if not args.no_long:
        say("indexer S=1M (config[4] indexer stage), top_k 512 and 1024")
        rl = run_indexer(1 << 20, args.ratio, args.top_k, args.chunk_s, args.chunk_t, 1, 1)
        extra["s1m_ms"] = rl["ms"]
        extra["s1m_tflops"] = rl["flops"] / (rl["ms"] * 1e-3) / 1e12
        extra["s1m_mfma_frac"] = extra["s1m_tflops"] / PEAK_BF16_TFLOPS
        extra["s1m_peak_hbm_gib"] = rl["peak_gib"]
        extra["reference_h200_ms_s1m"] = REF_H200_MS[1048576]
        extra["reference_h200_gib_s1m"] = REF_H200_GIB[1048576]
        k1024 = run_indexer_sweep(rl["q"], rl["k"], rl["w"], args.ratio, (1024,), 1)["1024"]
        k1024["reference_h200_ms"], k1024["reference_h200_gib"] = REF_H200_S1M_K1024
        extra["s1m_topk1024"] = k1024
        del rl
        torch.cuda.empty_cache()
    if not args.no_indexer_q:
        say("fp4/fp8 indexer S=64K and S=1M")
        extra["indexer_q_s64k"] = run_indexer_q(65536, args.ratio, args.top_k, 10, 5)
        if not args.no_long:
            extra["indexer_q_s1m"] = run_indexer_q(1 << 20, args.ratio, args.top_k, 1, 1, parity_rows=64)
        torch.cuda.empty_cache()

    if not args.no_score:
        say("indexer_score (materialised scores) at config[1]'s shape")
        extra["indexer_score_c1"] = run_indexer_score(65536, 5, 2, args.ratio)

    if not args.no_e2e:
        say("end-to-end CSA forward S=64K")
        extra["csa_e2e_s64k"] = run_csa_e2e(65536, 5, 3, 256, bwd=not args.no_attn_bwd)
        say("end-to-end CSA forward S=1M (config[4])")
        extra["csa_e2e_s1m"] = run_csa_e2e(1 << 20, 1, 1, args.e2e_parity_rows)
        say("end-to-end CSA forward S=1M with the fp4/fp8 indexer")
        extra["csa_e2e_s1m_quantized_indexer"] = run_csa_e2e(1 << 20, 1, 1, 256, quantized=True)
        say("end-to-end HCA forward S=64K")
        extra["hca_e2e_s64k"] = run_hca_e2e(65536, 10, 3, 8, bwd=not args.no_attn_bwd)
    torch.cuda.empty_cache()

    counters = None
    traffic = None
    if not args.no_counters:
        counters = run_counters()
        ic = counters.get("indexer_c1", {}) if isinstance(counters, dict) else {}
        traffic = ic.get("hbm_bytes_per_launch")
        ac = counters.get("sparse_attn_c3", {}) if isinstance(counters, dict) else {}
        if "sparse_attn_c3" in extra and ac.get("hbm_bytes_per_launch"):
            fab = ac["hbm_bytes_per_launch"] / (extra["sparse_attn_c3"]["ms"] * 1e-3) / 1e9
            extra["sparse_attn_c3"]["hbm_counter_gbps"] = fab
            extra["sparse_attn_c3"]["hbm_counter_frac"] = fab / PEAK_HBM_GBPS
            extra["sparse_attn_c3"]["hbm_bytes_per_launch"] = ac["hbm_bytes_per_launch"]

    cpu_baseline = None
    if cpu is not None:
        dense_scale = (args.seq * (args.seq // args.ratio)) / (4096.0 * 1024.0)
        cpu_baseline = {
            "value": round(cpu["ms"] * dense_scale, 1),
            "unit": f"ms (config[1] job, extrapolated x{dense_scale:.0f} by dense (s,t) pairs from the full "
                    f"config[0] run)",
            "cores": cpu["threads"], "kind": "port",
            "sample": "config[0] in full (B=1, S=4096, T=1024, H_I=64, D_I=128, k=512, seed 2026): the reference's "
                      "CPU path op for op in torch fp32 (einsum bshd,btd->bsht, relu, weighted head sum, -inf mask, "
                      "topk, -1 post-mask; oracle/torch_materialize.py), 1 warm-up + 3 timed, median",
            "config0_ms": round(cpu["ms"], 1), "config0_runs_ms": [round(x, 1) for x in cpu["runs_ms"]],
            "config0_gpu_ms": round(extra["c0_gpu_ms"], 4),
            "cpu_model": cpu["cpu_model"], "os_cpu_count": cpu["os_cpu_count"],
            "port_sampled_c1": {"value_ms": round(port_ms_full, 1), "cpu_s": round(par["cpu_s"], 3),
                                "note": f"C oracle (fp64, OpenMP) on the {par['rows']} parity rows of config[1], "
                                        f"scaled by causally legal (s,t) pairs"},
        }

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
        "parity": {k: par[k] for k in ("rows", "recall_mean", "recall_min", "exact_rows_frac", "wide_gap_rows",
                                       "wide_gap_rows_exact", "max_score_rel_err")},
        "cpu_baseline": cpu_baseline,
        "counters": counters,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
