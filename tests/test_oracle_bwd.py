"""Pins the sparse-attention backward oracle (CPU only).

* np_sparse_attn_bwd against central finite differences of the fp64 forward
  np_sparse_attn (itself pinned by tests/test_oracle.py): with the exact saved
  (o, lse) the formulas of sparse_attn_bwd.py:1-26 must be the gradient of
  sum(o * do) with respect to q, kv and the sink.
* Planted mistakes (no delta term, p in place of ds for dkv, a sign flip of
  dsink) must fail the same check.
* Closed form: a row with every key masked has dq = 0, no dkv contribution
  and dsink = -delta (its lse is the sink).
* The C oracle against the numpy restatement on bf16-representable inputs,
  with duplicated and out-of-range keys, key subsets and the dsink-only mode.
"""

import numpy as np
import pytest

from oracle import oracle as O


def _problem(seed, n=3, H=2, D=8, N=6, K=5):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, H, D)) * 0.7
    kv = rng.standard_normal((N, D)) * 0.7
    sink = rng.standard_normal(H)
    idx = rng.integers(0, N, (n, K))
    idx[0, 1] = -1
    idx[1, 2] = N + 3          # out of range: masked like -1
    idx[2, 3] = idx[2, 0]      # duplicate key: counted twice
    g = rng.standard_normal((n, H, D))
    return q, kv, sink, idx, g


def _loss(q, kv, sink, idx, g, scale):
    o, _ = O.np_sparse_attn(q, kv, sink, idx, scale)
    return float((o * g).sum())


def _fd(fun, x, eps=1e-6):
    out = np.zeros_like(x)
    flat = x.reshape(-1)
    for i in range(flat.size):
        keep = flat[i]
        flat[i] = keep + eps
        up = fun()
        flat[i] = keep - eps
        dn = fun()
        flat[i] = keep
        out.reshape(-1)[i] = (up - dn) / (2 * eps)
    return out


def _grads(q, kv, sink, idx, g, scale, bwd=O.np_sparse_attn_bwd):
    o, lse = O.np_sparse_attn(q, kv, sink, idx, scale)
    return bwd(q, kv, o, g, sink, lse, idx, scale)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_bwd_formulas_are_the_gradient(seed):
    q, kv, sink, idx, g = _problem(seed)
    scale = 0.8
    dq, dkv, dsink = _grads(q, kv, sink, idx, g, scale)
    f = lambda: _loss(q, kv, sink, idx, g, scale)  # noqa: E731
    np.testing.assert_allclose(dq, _fd(f, q), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dkv, _fd(f, kv), rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(dsink, _fd(f, sink), rtol=1e-6, atol=1e-8)


def _no_delta(qf, kvf, of, dof, sink, lse, idx, scale):
    return O.np_sparse_attn_bwd(qf, kvf, of * 0.0, dof, sink, lse, idx, scale)


def _p_for_ds(qf, kvf, of, dof, sink, lse, idx, scale):
    dq, _, dsink = O.np_sparse_attn_bwd(qf, kvf, of, dof, sink, lse, idx, scale)
    # dkv built with p in place of ds on the score path
    _, dkv_v, _ = O.np_sparse_attn_bwd(qf * 0.0, kvf, of, dof, sink, lse, idx, scale)
    return dq, dkv_v, dsink


def _sink_sign(qf, kvf, of, dof, sink, lse, idx, scale):
    dq, dkv, dsink = O.np_sparse_attn_bwd(qf, kvf, of, dof, sink, lse, idx, scale)
    return dq, dkv, -dsink


@pytest.mark.parametrize("planted,which", [(_no_delta, 0), (_p_for_ds, 1), (_sink_sign, 2)])
def test_planted_mistakes_fail_the_gradient_check(planted, which):
    q, kv, sink, idx, g = _problem(5)
    scale = 0.8
    got = _grads(q, kv, sink, idx, g, scale, bwd=planted)[which]
    f = lambda: _loss(q, kv, sink, idx, g, scale)  # noqa: E731
    ref = _fd(f, (q, kv, sink)[which])
    assert np.abs(got - ref).max() > 1e-3


def test_all_masked_row_closed_form():
    q, kv, sink, idx, g = _problem(7)
    idx[1, :] = -1
    scale = 0.8
    o, lse = O.np_sparse_attn(q, kv, sink, idx, scale)
    np.testing.assert_allclose(lse[1], sink, rtol=0, atol=1e-12)
    np.testing.assert_allclose(o[1], 0.0, atol=0)
    dq, dkv, dsink = O.np_sparse_attn_bwd(q, kv, o, g, sink, lse, idx, scale)
    np.testing.assert_allclose(dq[1], 0.0, atol=0)
    # the masked row adds nothing to dkv: dropping it leaves dkv unchanged
    keep = np.array([0, 2])
    _, dkv2, dsink2 = O.np_sparse_attn_bwd(q[keep], kv, o[keep], g[keep], sink, lse[keep], idx[keep], scale)
    np.testing.assert_allclose(dkv, dkv2, atol=1e-15)
    # its sink term: p_sink = 1, delta = o.g = 0 -> no dsink either
    np.testing.assert_allclose(dsink, dsink2, atol=1e-15)


def test_single_valid_key_closed_form():
    """One valid key per row: p = sigmoid(z - sink), o = p v, and
    dq = scale p (1 - p) (g.v) v."""
    rng = np.random.default_rng(11)
    H, D, N = 2, 4, 3
    q = rng.standard_normal((1, H, D))
    kv = rng.standard_normal((N, D))
    sink = rng.standard_normal(H)
    idx = np.array([[-1, 2, -1]])
    g = rng.standard_normal((1, H, D))
    scale = 0.5
    o, lse = O.np_sparse_attn(q, kv, sink, idx, scale)
    dq, dkv, _ = O.np_sparse_attn_bwd(q, kv, o, g, sink, lse, idx, scale)
    v = kv[2]
    for h in range(H):
        z = scale * q[0, h] @ v
        p = 1.0 / (1.0 + np.exp(sink[h] - z))
        np.testing.assert_allclose(o[0, h], p * v, rtol=1e-12)
        np.testing.assert_allclose(dq[0, h], scale * p * (1 - p) * (g[0, h] @ v) * v, rtol=1e-10)
    np.testing.assert_allclose(dkv[[0, 1]], 0.0, atol=0)


@pytest.mark.parametrize("seed", [0, 3])
def test_c_oracle_matches_numpy(seed):
    rng = np.random.default_rng(seed)
    n, H, D, N, K = 9, 4, 24, 13, 10
    bits = lambda x: O.f32_to_bf16_bits(x.astype(np.float32))  # noqa: E731
    qb = bits(rng.standard_normal((n, H, D)) * 0.5)
    kb = bits(rng.standard_normal((N, D)) * 0.5)
    idx = rng.integers(-2, N + 2, (n, K))
    idx[3] = -1
    sink = rng.standard_normal(H).astype(np.float32)
    o, lse = O.sparse_attn_rows(qb, kb, sink, np.where((idx >= 0) & (idx < N), idx, -1), 0.3)
    ob = bits(o)
    db = bits(rng.standard_normal((n, H, D)))
    lse32 = lse.astype(np.float32)
    f = O.bf16_bits_to_f64
    dq_n, dkv_n, ds_n = O.np_sparse_attn_bwd(f(qb), f(kb), f(ob), f(db), sink.astype(np.float64),
                                             lse32.astype(np.float64), idx, 0.3)
    dq, dkv, ds = O.sparse_attn_bwd_rows(qb, kb, ob, db, sink, lse32, idx, 0.3)
    np.testing.assert_allclose(dq, dq_n, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(dkv, dkv_n, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ds, ds_n, rtol=1e-12, atol=1e-14)
    keys = np.array([5, 0, 12])
    none, dk_sub, ds_sub = O.sparse_attn_bwd_rows(qb, kb, ob, db, sink, lse32, idx, 0.3, keys=keys, want_dq=False)
    assert none is None
    np.testing.assert_allclose(dk_sub, dkv_n[keys], rtol=1e-12, atol=1e-14)
    _, no_dkv, ds_only = O.sparse_attn_bwd_rows(qb, kb, ob, db, sink, lse32, idx, 0.3, want_dq=False, want_dkv=False)
    assert no_dkv is None
    np.testing.assert_allclose(ds_only, ds_n, rtol=1e-12, atol=1e-14)
