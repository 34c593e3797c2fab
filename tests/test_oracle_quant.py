"""Pins the quantisation and token-compressor oracle (CPU only).

* The numpy simulations against the reference formulas
  (flash_sparse/utils/quantization.py:19-65, with ``.abs()`` called as the
  formula intends) run by torch on the CPU — torch's float8_e4m3fn conversion,
  bf16/fp16 arithmetic and argmin are an independent implementation — in
  fp32, bf16 and fp16, over normal, tiny (amax below the clamp), exact-grid
  and tie inputs.
* e4m3 rounding against torch's float8 conversion on every representable
  value and every midpoint between neighbours; e2m1 rounding against the grid
  (fixed points, ties to the even code).
* The packed formats: dequantised error bounds, power-of-two scales, nibble
  order of the packing.
* The token compressor against the reference formula restated in torch
  (float64), a planted mistake (the b stream not shifted by one block), and
  closed forms (equal scores -> mean; one dominant score -> that token).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

DTYPES = ["float32", "bfloat16", "float16"]


def _torch_fp8_sim(t, bs):
    blocks = t.reshape(*t.shape[:-1], -1, bs)
    amax = blocks.abs().amax(dim=-1, keepdim=True).clamp_min(1e-4)
    scale = amax / 448.0
    q = (blocks / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return (q.float() * scale).reshape(t.shape).to(t.dtype)


def _torch_fp4_sim(t, bs):
    blocks = t.reshape(*t.shape[:-1], -1, bs)
    amax = blocks.abs().amax(dim=-1, keepdim=True).clamp_min(6 * 2.0 ** -126)
    scale = amax / 6.0
    grid = torch.tensor([-6, -4, -3, -2, -1.5, -1, -0.5, 0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=t.dtype)
    scaled = (blocks / scale).clamp(-6.0, 6.0)
    idx = (scaled.unsqueeze(-1) - grid).abs().argmin(dim=-1)
    return (grid[idx] * scale).reshape(t.shape).to(t.dtype)


def _inputs(seed, shape=(6, 256)):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32) * np.exp2(rng.integers(-8, 8, (shape[0], 1))).astype(np.float32)
    x[0, :64] = 1e-6 * rng.standard_normal(64)           # blocks below the amax clamp
    x[1, :32] = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6] * 4) * 0.75   # exact grid multiples
    x[2, :128] = np.linspace(-448, 448, 128)              # spans the whole fp8 range
    return x


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("seed", [0, 1])
def test_fp8_simulate_matches_reference_formula(dt, seed):
    x = O.round_to(_inputs(seed), dt)
    ref = _torch_fp8_sim(torch.from_numpy(x).to(getattr(torch, dt)), 128).float().numpy()
    assert np.array_equal(O.act_quant_simulate(x, dt, 128), ref)
    ref64 = _torch_fp8_sim(torch.from_numpy(x).to(getattr(torch, dt)), 64).float().numpy()
    assert np.array_equal(O.act_quant_simulate(x, dt, 64), ref64)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("seed", [0, 1])
def test_fp4_simulate_matches_reference_formula(dt, seed):
    x = O.round_to(_inputs(seed), dt)
    ref = _torch_fp4_sim(torch.from_numpy(x).to(getattr(torch, dt)), 32).float().numpy()
    assert np.array_equal(O.fp4_act_quant_simulate(x, dt, 32), ref)
    ref16 = _torch_fp4_sim(torch.from_numpy(x).to(getattr(torch, dt)), 16).float().numpy()
    assert np.array_equal(O.fp4_act_quant_simulate(x, dt, 16), ref16)


def test_fp4_simulate_ties_take_the_first_grid_value():
    # scaled values halfway between grid points: argmin keeps the lower (earlier) one
    x = np.zeros((1, 32), np.float32)
    x[0, :8] = [6, 0.25, 0.75, 1.25, 2.5, 3.5, 5, -0.25]
    got = O.fp4_act_quant_simulate(x, "float32", 32)[0, :8]
    assert list(got) == [6, 0, 0.5, 1, 2, 3, 4, -0.5]


def test_e4m3_round_matches_torch_on_values_and_midpoints():
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    vals = np.unique(vals[np.isfinite(vals)])
    assert np.array_equal(O.e4m3_round(vals), vals)                   # fixed points
    mids = (vals[1:] + vals[:-1]) / 2                                  # every tie
    pts = np.concatenate([mids, mids * (1 + 1e-6), mids * (1 - 1e-6)])
    pts = pts[np.abs(pts) <= 448]
    ref = torch.from_numpy(pts.astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(O.e4m3_round(pts.astype(np.float32)), ref)


def test_e2m1_round_grid_and_ties():
    mags = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    assert np.array_equal(O.e2m1_round(mags), mags)
    assert np.array_equal(O.e2m1_round(-mags[1:]), -mags[1:])
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    assert list(O.e2m1_round(ties)) == [0, 1, 1, 2, 2, 4, 4]             # even codes: 0, 2, 4, 6
    assert list(O.e2m1_round(ties + 1e-3)) == [0.5, 1, 1.5, 2, 3, 4, 6]


def test_packed_formats_bounds_and_scales():
    x = _inputs(3)
    v8, s8 = O.fp8_pack(x, 128)
    deq = (v8.reshape(6, 2, 128) * s8[..., None]).reshape(6, 256)
    # e4m3: relative error <= 2^-4 for normal values, absolute <= 2^-10 scale below
    err = np.abs(deq - x)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, np.repeat(s8, 128, -1) * 2.0 ** -10)
    assert np.all(err <= bound * (1 + 1e-6))
    v8p, s8p = O.fp8_pack(x, 128, pow2=True)
    assert np.all(np.exp2(np.round(np.log2(s8p))) == s8p)
    assert np.all(np.abs(v8p) <= 448)
    v4, s4 = O.fp4_pack(x, 32)
    assert np.all(np.exp2(np.round(np.log2(s4))) == s4)               # powers of two
    assert np.all(np.abs(v4) <= 6)
    deq4 = (v4.reshape(6, 8, 32) * s4[..., None]).reshape(6, 256)
    assert np.all(np.abs(deq4 - x) <= np.repeat(s4, 32, -1) * 1.0 + 1e-30)   # half the widest e2m1 step


def test_fp4_unpack_nibble_order():
    packed = np.array([[0x21, 0xF7]], np.uint8)   # low nibble first: 1 (0.5), 2 (1.0), 7 (6.0), 15 (-6.0)
    assert list(O.fp4_unpack(packed)[0]) == [0.5, 1.0, 6.0, -6.0]


def _torch_compressor(c_a, z_a, b_a, m, c_b, z_b, b_b, overlap):
    # reference.py:230-270 with the overlap path at function level (as its docstring states)
    B, S, c = c_a.shape
    n = S // m
    ca = c_a[:, :n * m].reshape(B, n, m, c)
    za = z_a[:, :n * m].reshape(B, n, m, c) + b_a
    if not overlap:
        return (ca * za.softmax(dim=2)).sum(dim=2)
    cb = c_b[:, :n * m].reshape(B, n, m, c)
    zb = z_b[:, :n * m].reshape(B, n, m, c) + b_b
    cbs = torch.zeros_like(cb)
    cbs[:, 1:] = cb[:, :-1]
    zbs = torch.full_like(zb, float("-inf"))
    zbs[:, 1:] = zb[:, :-1]
    return (torch.cat([ca, cbs], 2) * torch.cat([za, zbs], 2).softmax(dim=2)).sum(dim=2)


@pytest.mark.parametrize("overlap,m", [(True, 4), (False, 8), (False, 128)])
def test_token_compressor_matches_reference_formula(overlap, m):
    rng = np.random.default_rng(m)
    B, S, C = 2, 3 * m + 1, 16   # trailing token dropped
    arr = [rng.standard_normal((B, S, C)) for _ in range(4)]
    ba, bb = rng.standard_normal((m, C)), rng.standard_normal((m, C))
    got = O.token_compressor(arr[0], arr[1], ba, m, arr[2], arr[3], bb, overlap)
    t = [torch.from_numpy(a) for a in arr]
    ref = _torch_compressor(t[0], t[1], torch.from_numpy(ba), m, t[2], t[3], torch.from_numpy(bb), overlap).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    if overlap:   # planted mistake: b stream not shifted by one block
        wrong = O.token_compressor(arr[0], arr[1], ba, m, np.roll(arr[2], m, 1), np.roll(arr[3], m, 1), bb, overlap)
        assert np.abs(wrong - ref).max() > 1e-3


def test_token_compressor_closed_forms():
    rng = np.random.default_rng(5)
    c = rng.standard_normal((1, 8, 3))
    z = np.zeros((1, 8, 3))
    out = O.token_compressor(c, z, np.zeros((4, 3)), 4)
    np.testing.assert_allclose(out[0], c[0].reshape(2, 4, 3).mean(1), rtol=1e-12)
    z[0, 2] = 80.0   # one dominant score in block 0
    out = O.token_compressor(c, z, np.zeros((4, 3)), 4)
    np.testing.assert_allclose(out[0, 0], c[0, 2], rtol=1e-9)
