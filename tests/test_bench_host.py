"""Host-side arithmetic of ``bench.py``: the counter-CSV reader, the
clock / MFMA-busy / utilisation figures of the ``counters`` object, the
peak constants the roofline divides by, and the one-GPU contract.

Runs without a GPU: the counter rows are synthetic, with values chosen so
that every derived figure has a hand-computed answer (a shader clock of
exactly 2.0 GHz, a pipe busy exactly half the time, ...), so a dropped
factor (the 8 XCDs, the 1,024 SIMDs, the 32,768 FLOP of one
v_mfma_f32_32x32x16_bf16) fails here.
"""
import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _write_counter_csv(path, rows):
    """rows: (dispatch id, kernel, start ns, end ns, counter, value), in the
    column layout rocprofv3 --output-format csv writes."""
    fields = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
              "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
              "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp",
              "End_Timestamp"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for did, kernel, t0, t1, name, value in rows:
            rec = {k: 0 for k in fields}
            rec.update({"Dispatch_Id": did, "Kernel_Name": kernel, "Start_Timestamp": t0, "End_Timestamp": t1,
                        "Counter_Name": name, "Counter_Value": value})
            w.writerow(rec)


def test_peak_constants_match_the_part():
    # 256 CUs x 4,096 dense bf16 FLOP per clock per CU at 2.4 GHz; fp8 twice that
    assert bench.PEAK_BF16_TFLOPS == pytest.approx(256 * 4096 * 2.4e9 / 1e12, rel=1e-4)
    assert bench.PEAK_FP8_TFLOPS == pytest.approx(2 * bench.PEAK_BF16_TFLOPS, rel=1e-4)
    assert bench.PEAK_HBM_GBPS == 8000.0
    assert bench.MFMA_FLOP == 2 * 32 * 32 * 16
    assert bench.N_SIMD == 256 * 4 and bench.N_XCD == 8


def test_read_counters_groups_by_dispatch_and_sums_repeats(tmp_path):
    p = tmp_path / "pmc_counter_collection.csv"
    _write_counter_csv(p, [
        (7, "void si::indexer_topk_kernel<2, 128, 1536, false>(si::IndexerArgs)", 1000, 5000, "FETCH_SIZE", 10.0),
        (7, "void si::indexer_topk_kernel<2, 128, 1536, false>(si::IndexerArgs)", 1000, 5000, "FETCH_SIZE", 2.5),
        (7, "void si::indexer_topk_kernel<2, 128, 1536, false>(si::IndexerArgs)", 1000, 5000, "WRITE_SIZE", 4.0),
        (3, "__amd_rocclr_copyBuffer", 0, 250, "FETCH_SIZE", 1.0),
    ])
    d = bench._read_counters(str(p))
    assert set(d) == {3, 7}
    assert d[7]["ns"] == 4000 and d[3]["ns"] == 250
    assert d[7]["FETCH_SIZE"] == 12.5 and d[7]["WRITE_SIZE"] == 4.0
    # dispatch order, kernel-name filter, last / first-after-skip selection
    d[9] = {"kernel": "void si::indexer_topk_kernel<2, 128, 1536, false>", "ns": 1}
    assert [r["ns"] for r in bench._pick(d, "indexer_topk", 1)] == [1]
    assert [r["ns"] for r in bench._pick_first(d, "indexer_topk", 1, 5)] == [1]
    assert bench._pick(d, "sparse_attn", 3) == []


def test_mfma_summary_closed_forms():
    ns = 1_000_000                      # 1 ms per dispatch
    cycles = 2_000_000                  # 2.0 GHz shader clock
    insts = 30_000_000
    row = {"kernel": "void si::indexer_topk_kernel<2, 128, 1536, false>(si::IndexerArgs)", "ns": ns,
           "GRBM_GUI_ACTIVE": 8.0 * cycles,                           # summed over the 8 XCDs
           "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * 1024 * cycles,           # summed over 1,024 SIMDs: half busy
           "SQ_INSTS_MFMA": float(insts),
           "SQ_INSTS_VALU": 6.0 * insts}
    flops = 9.8e11
    s = bench._mfma_summary([row, dict(row)], flops)
    assert s["kernel"] == "void si::indexer_topk_kernel<2, 128, 1536, false>"
    assert s["dispatches"] == 2
    assert s["avg_ms"] == pytest.approx(1.0)
    assert s["clock_ghz"] == pytest.approx(2.0)
    assert s["mfma_busy_pct"] == pytest.approx(50.0)
    assert s["executed_mfma_flops"] == pytest.approx(insts * 32768.0)
    # 30e6 x 32,768 FLOP in 1 ms = 983.04 TFLOP/s
    assert s["mfma_util_pct_from_counters"] == pytest.approx(100.0 * 983.04 / 2516.6, rel=1e-6)
    assert s["mfma_util_pct_from_time"] == pytest.approx(100.0 * 980.0 / 2516.6, rel=1e-6)
    assert s["valu_per_mfma"] == pytest.approx(6.0)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
