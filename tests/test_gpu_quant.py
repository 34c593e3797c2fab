"""GPU parity of the quantisation and token-compressor kernels.

Bit-exact against the oracle (which tests/test_oracle_quant.py pins to the
reference formulas run by torch on the CPU): the fp8 / fp4 simulations in
fp32, bf16 and fp16 (flash_sparse/utils/quantization.py:19-65), and the packed
production formats (fp8 bytes, fp4 nibbles, scales).  The compressor and the
gated pool compute in fp32 and round once, so they are checked against the
float64 oracle within 2e-2 relative to max|ref| for bf16 inputs and 1e-5 for
fp32 inputs.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from streamindex_amd import compressor, quant

pytestmark = pytest.mark.gpu

TD = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def _x(seed, shape, dt):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(shape) * np.exp2(rng.integers(-6, 6, shape[:-1] + (1,)))).astype(np.float32)
    x.reshape(-1, shape[-1])[0, :64] = 1e-6   # a block below the amax clamp
    return O.round_to(x, dt)


@pytest.mark.parametrize("dt", ["float32", "bfloat16", "float16"])
def test_simulations_bit_exact(cuda_device, dt):
    x = _x(1, (3, 7, 256), dt)
    t = torch.from_numpy(x).to(TD[dt]).cuda()
    for bs in (128, 64):
        got = quant.act_quant_simulate(t, bs).float().cpu().numpy()
        assert np.array_equal(got, O.act_quant_simulate(x, dt, bs)), f"fp8 {dt} bs={bs}"
    for bs in (32, 16):
        got = quant.fp4_act_quant_simulate(t, bs).float().cpu().numpy()
        assert np.array_equal(got, O.fp4_act_quant_simulate(x, dt, bs)), f"fp4 {dt} bs={bs}"
    with pytest.raises(AssertionError):
        quant.act_quant_simulate(t[..., :200], 128)


@pytest.mark.parametrize("dt", ["float32", "bfloat16"])
def test_packed_formats_bit_exact(cuda_device, dt):
    x = _x(2, (5, 512), dt)
    t = torch.from_numpy(x).to(TD[dt]).cuda()
    for fmt in (None, "ue8m0"):
        v, s = quant.act_quant(t, 128, fmt)
        rv, rs = O.fp8_pack(x, 128, pow2=fmt == "ue8m0")
        assert v.dtype == torch.float8_e4m3fn and s.shape == (5, 4)
        assert np.array_equal(s.cpu().numpy(), rs)
        assert np.array_equal(v.float().cpu().numpy(), rv.astype(np.float32))
    p, s4 = quant.fp4_act_quant(t, 32)
    rv4, rs4 = O.fp4_pack(x, 32)
    assert p.dtype == torch.uint8 and p.shape == (5, 256)
    assert np.array_equal(s4.cpu().numpy(), rs4)
    assert np.array_equal(O.fp4_unpack(p.cpu().numpy()), rv4)


@pytest.mark.parametrize("dt,tol", [("float32", 1e-5), ("bfloat16", 2e-2)])
@pytest.mark.parametrize("overlap,m", [(True, 4), (False, 128), (False, 8)])
def test_token_compressor(cuda_device, dt, tol, overlap, m):
    rng = np.random.default_rng(m + overlap)
    B, S, C = 2, 5 * m + 3, 96
    arr = [O.round_to(rng.standard_normal((B, S, C)).astype(np.float32), dt) for _ in range(4)]
    ba, bb = rng.standard_normal((m, C)).astype(np.float32), rng.standard_normal((m, C)).astype(np.float32)
    t = [torch.from_numpy(a).to(TD[dt]).cuda() for a in arr]
    kw = dict(c_b=t[2], z_b=t[3], b_b=torch.from_numpy(bb).cuda()) if overlap else {}
    got = compressor.token_compressor(t[0], t[1], torch.from_numpy(ba).cuda(), m, overlap=overlap, **kw)
    ref = O.token_compressor(arr[0], arr[1], ba, m, arr[2], arr[3], bb, overlap)
    assert got.shape == (B, S // m, C) and got.dtype == TD[dt]
    assert np.abs(got.float().cpu().numpy() - ref).max() <= tol * np.abs(ref).max()


def test_gated_pool(cuda_device):
    rng = np.random.default_rng(9)
    kv = rng.standard_normal((3, 5, 7, 4)).astype(np.float32)
    sc = rng.standard_normal((3, 5, 7, 4)).astype(np.float32)
    for dim in (-2, 1, 0):
        got = compressor.softmax_gated_pool(torch.from_numpy(kv).cuda(), torch.from_numpy(sc).cuda(), dim=dim)
        w = np.exp(sc - sc.max(dim, keepdims=True))
        ref = (kv * w).sum(dim) / w.sum(dim)
        assert np.abs(got.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
