"""Writes tests/golden/synth_digests.json: for every tensor the benchmark
configs draw with the counter-based generator (streamindex_amd.synth,
si_fill_normal), its shape, dtype, seed, stream and scale, the digests
(d1, d2) of the whole tensor and its first 16 values (bit patterns), all
computed on the CPU by the oracle's restatement of the generator.

The GPU test (tests/test_gpu_synth.py) draws the same tensors on the device
and must reproduce every digest; the CPU test (tests/test_synth.py) checks the
heads and the digests of the small tensors against the oracle.

    python tests/golden/make_synth_digests.py      # a few minutes on 8 cores
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

STREAMS = {"indexer.q": 1, "indexer.k": 2, "indexer.w": 3, "attn.q": 11, "attn.kv": 12, "attn.sink": 13,
           "csa.q": 21, "csa.kv": 22, "csa.kvc": 23, "csa.sink": 24}


def tensors():
    """(config, name, shape, bf16, seed, stream, scale) for every synthetic tensor of the configs."""
    out = []
    for cfg, S in (("config1", 65536), ("config2", 262144), ("config4", 1 << 20)):
        T = S // 4
        out += [(cfg, "indexer.q", (1, S, 64, 128), True, 2026, 128 ** -0.5),
                (cfg, "indexer.k", (1, T, 128), True, 2026, 128 ** -0.5),
                (cfg, "indexer.w", (1, S, 64), False, 2026, 1.0)]
    out += [("config3", "attn.q", (1, 65536, 64, 576), True, 2027, 1.0),
            ("config3", "attn.kv", (1, 16384, 576), True, 2027, 1.0),
            ("config3", "attn.sink", (64,), False, 2027, 1.0)]
    S = 1 << 20
    out += [("config4", "csa.q", (1, S, 64, 576), True, 2027, 1.0),
            ("config4", "csa.kv", (1, S, 576), True, 2027, 1.0),
            ("config4", "csa.kvc", (1, S // 4, 576), True, 2027, 1.0),
            ("config4", "csa.sink", (64,), False, 2027, 1.0)]
    return [(c, n, shp, bf, seed, STREAMS[n], sc) for (c, n, shp, bf, seed, sc) in out]


def main():
    rows = []
    for cfg, name, shape, bf16, seed, stream, scale in tensors():
        n = int(np.prod(shape))
        d1, d2 = O.synth_digest(n, seed, stream, scale, bf16=bf16)
        head = O.synth_normal(0, 16, seed, stream, scale, bf16=bf16)
        head_bits = head.tolist() if bf16 else head.view(np.uint32).tolist()
        rows.append({"config": cfg, "name": name, "shape": list(shape), "dtype": "bf16" if bf16 else "fp32",
                     "seed": seed, "stream": stream, "scale": scale, "d1": d1, "d2": d2, "head_bits": head_bits})
        print(f"{cfg} {name} {shape} d1={d1} d2={d2}", flush=True)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "synth_digests.json")
    with open(path, "w") as f:
        json.dump({"generator": "Philox4x32-10 + Box-Muller (streamindex_amd/csrc/synth.hip)", "tensors": rows}, f,
                  indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
