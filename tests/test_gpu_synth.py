"""The device generator behind the benchmark configs' inputs (si_fill_normal,
streamindex_amd/csrc/synth.hip) against its CPU restatement in the oracle,
bit for bit, and against the committed whole-tensor digests of every config
tensor (tests/golden/synth_digests.json), so the full-size inputs are the
same on every box."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "synth_digests.json")


def _words(t: torch.Tensor) -> torch.Tensor:
    """The little-endian 16-bit words of a contiguous tensor, as int64."""
    return t.contiguous().view(-1).view(torch.int16).to(torch.int64) & 0xFFFF


def _digest(t: torch.Tensor):
    d1 = d2 = 0
    flat = t.contiguous().view(-1).view(torch.int16)
    n = flat.numel()
    chunk = 1 << 25
    for j0 in range(0, n, chunk):
        w = flat[j0:j0 + chunk].to(torch.int64) & 0xFFFF
        j = torch.arange(j0, j0 + w.numel(), device=w.device, dtype=torch.int64)
        d1 += int(w.sum())
        d2 += int((w * (j % 65521 + 1)).sum())
    return d1 % (1 << 64), d2 % (1 << 64)


@pytest.mark.parametrize("n,bf16,seed,stream,scale", [(1 << 20, True, 2026, 1, 128 ** -0.5), (12345, False, 9, 4, 1.0),
                                                      (7, True, 3, 2, 2.5), (4 * 100001 + 3, False, 2027, 13, 0.25)])
def test_device_matches_cpu_restatement(cuda_device, n, bf16, seed, stream, scale):
    t = synth.device_normal((n,), torch.bfloat16 if bf16 else torch.float32, seed=seed, stream=stream, scale=scale)
    torch.cuda.synchronize()
    ref = O.synth_normal(0, n, seed, stream, scale, bf16=bf16)
    got = t.cpu().view(torch.int16).numpy().view(np.uint16) if bf16 else t.cpu().numpy()
    if bf16:
        assert np.array_equal(got, ref)
    else:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_config_digests(cuda_device):
    with open(GOLDEN) as f:
        rows = json.load(f)["tensors"]
    rng = np.random.default_rng(0)
    for r in rows:
        bf16 = r["dtype"] == "bf16"
        print(f"[test] synth {r['config']} {r['name']} {r['shape']}", flush=True)
        t = synth.device_normal(tuple(r["shape"]), torch.bfloat16 if bf16 else torch.float32, seed=r["seed"],
                                stream=r["stream"], scale=r["scale"])
        torch.cuda.synchronize()
        assert _digest(t) == (r["d1"], r["d2"]), f"{r['config']} {r['name']}: digest differs from the fixture"
        n = t.numel()
        idx = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, 4096)]))
        got = t.view(-1)[torch.from_numpy(idx).cuda()].cpu()
        ref = O.synth_normal_at(idx, r["seed"], r["stream"], r["scale"], bf16=bf16)
        if bf16:
            assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), ref)
        else:
            assert np.array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))
        del t
        torch.cuda.empty_cache()


def test_synth_inputs_use_the_config_streams(cuda_device):
    """indexer_inputs / sparse_attn_inputs / csa_attn_inputs at a config size
    return exactly the fixture's tensors (spot-checked heads)."""
    with open(GOLDEN) as f:
        rows = {(r["config"], r["name"]): r for r in json.load(f)["tensors"]}
    q, k, w = synth.indexer_inputs(1, 65536, 64, 128, ratio=4, seed=2026)
    for t, name in ((q, "indexer.q"), (k, "indexer.k")):
        head = _words(t.view(-1)[:16]).cpu().numpy().tolist()
        assert head == rows[("config1", name)]["head_bits"], name
    assert w.view(-1)[:16].cpu().numpy().view(np.uint32).tolist() == rows[("config1", "indexer.w")]["head_bits"]
    del q, k, w
    qa, kv, sink = synth.sparse_attn_inputs(1, 65536, 64, 576, 16384, seed=2027)
    assert _words(qa.view(-1)[:16]).cpu().numpy().tolist() == rows[("config3", "attn.q")]["head_bits"]
    assert sink[:16].cpu().numpy().view(np.uint32).tolist() == rows[("config3", "attn.sink")]["head_bits"]
    del qa, kv, sink
    torch.cuda.empty_cache()
