"""The counter-based synthetic-input generator, on the CPU (the oracle's C
restatement of streamindex_amd/csrc/synth.hip).

Pinned by: the published Philox4x32-10 known-answer vectors (Salmon et al.,
SC 2011; the Random123 distribution's kat_vectors for philox4x32 with 10
rounds); the committed fixture tests/golden/synth_digests.json (first values
and whole-tensor digests, written by tests/golden/make_synth_digests.py);
the ln / sin / cos polynomials against numpy's library functions; and the
N(0,1) moments and a Kolmogorov-Smirnov test.  A planted mistake (the pair's
sine and cosine swapped) changes the values the fixture holds.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "synth_digests.json")


def test_philox_known_answers():
    kat = [([0, 0, 0, 0], [0, 0], (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
           ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
           ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
            (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1))]
    for ctr, key, want in kat:
        assert O.philox4x32_10(ctr, key) == want


def _fixture():
    with open(GOLDEN) as f:
        return json.load(f)["tensors"]


def test_fixture_heads_and_small_digests():
    rows = _fixture()
    assert {r["config"] for r in rows} == {"config1", "config2", "config3", "config4"}
    for r in rows:
        bf16 = r["dtype"] == "bf16"
        head = O.synth_normal(0, 16, r["seed"], r["stream"], r["scale"], bf16=bf16)
        bits = head.tolist() if bf16 else head.view(np.uint32).tolist()
        assert bits == r["head_bits"], f"{r['config']} {r['name']} head"
        n = int(np.prod(r["shape"]))
        if n <= 1 << 24:  # whole-tensor digests of the small tensors; the GPU test checks every one
            assert O.synth_digest(n, r["seed"], r["stream"], r["scale"], bf16=bf16) == (r["d1"], r["d2"]), \
                f"{r['config']} {r['name']} digest"


def test_slices_and_indices_agree():
    full = O.synth_normal(0, 4099, 7, 3, 0.5)
    assert np.array_equal(O.synth_normal(1001, 2000, 7, 3, 0.5), full[1001:3001])
    idx = np.array([4098, 0, 5, 2048, 3, 3], dtype=np.int64)
    assert np.array_equal(O.synth_normal_at(idx, 7, 3, 0.5), full[idx])
    # bf16: the fp32 value rounded once, to nearest even
    b = O.synth_normal(0, 4099, 7, 3, 0.5, bf16=True)
    assert np.array_equal(b, O.f32_to_bf16_bits(full))
    # element i depends on (seed, stream, i) only: other streams and seeds differ
    assert not np.array_equal(O.synth_normal(0, 64, 7, 4, 0.5), full[:64])
    assert not np.array_equal(O.synth_normal(0, 64, 8, 3, 0.5), full[:64])


def test_moments_and_normality():
    from scipy import stats

    x = O.synth_normal(0, 1 << 22, 2026, 1).astype(np.float64)
    assert abs(x.mean()) < 3e-3 and abs(x.var() - 1.0) < 3e-3
    assert abs(((x - x.mean()) ** 4).mean() / x.var() ** 2 - 3.0) < 0.03
    assert stats.kstest(x[:200000], "norm").pvalue > 1e-3
    assert abs(np.corrcoef(x[0::2], x[1::2])[0, 1]) < 3e-3  # the two normals of a pair
    assert abs(np.corrcoef(x[:-4], x[4:])[0, 1]) < 3e-3     # neighbouring counters


def test_polynomials_against_numpy():
    """Inverting the generator's first stage recovers r and the angle: for
    each pair, n0^2 + n1^2 = -2 ln u1 and atan2(n1, n0) = 2 pi u2 to within
    fp32 rounding of the polynomials."""
    rng = np.random.default_rng(1)
    n = 1 << 14
    x = O.synth_normal(0, 4 * n, 11, 5).astype(np.float64).reshape(n, 4)
    r2 = x[:, 0] ** 2 + x[:, 1] ** 2
    assert np.all(r2 <= -2.0 * np.log(2.0 ** -24) * (1 + 1e-5))  # u1 >= 2^-24
    # the words themselves are not exposed: check against a direct fp64 Box-Muller of the same Philox words
    words = np.array([O.philox4x32_10([q, 0, 5, 0], [11, 0]) for q in range(256)], dtype=np.uint64)
    u1 = ((words[:, 0] >> 8) + 1).astype(np.float64) * 2.0 ** -24
    u2 = (words[:, 1] >> 8).astype(np.float64) * 2.0 ** -24
    r = np.sqrt(-2.0 * np.log(u1))
    ref = np.stack([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)], axis=1)
    got = x[:256, :2]
    assert np.abs(got - ref).max() < 2e-5 * max(1.0, np.abs(ref).max())
    del rng


def test_planted_swap_is_caught():
    rows = _fixture()
    r = next(t for t in rows if t["name"] == "indexer.w" and t["config"] == "config1")
    head = O.synth_normal(0, 16, r["seed"], r["stream"], r["scale"])
    swapped = head.reshape(-1, 2)[:, ::-1].reshape(-1)  # sine and cosine of each pair exchanged
    assert swapped.view(np.uint32).tolist() != r["head_bits"]
    assert head.view(np.uint32).tolist() == r["head_bits"]
