"""CPU oracle for the StreamIndex CSA hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker.  The product
(``streamindex_amd``) never imports, loads or calls anything here.

Two independent restatements of the reference's materialise-then-topk path
live here:

* the C oracle in ``si_oracle.c`` (double accumulation, OpenMP), used for
  anything larger than a toy, bound through ctypes below;
* small numpy versions (``np_*``) used to cross-check the C code on tiny
  shapes, together with brute-force and closed-form checks in
  ``tests/test_oracle.py``.

Reference semantics followed (file:line in the reference tree):

* score: ``flash_sparse/reference.py:138-168`` (eq. 16);
* mask / topk / post-mask: ``eval/test_v4_indexer_parity.py:111-137``;
* chunked output width ``top_k`` with ``-1`` / ``-inf`` padding:
  ``flash_sparse/triton/chunked_indexer.py:89-110,154-158``;
* tie order (score desc, index asc): ``docs/streaming_topk.md:46-60``;
* set-overlap recall: ``eval/test_v4_indexer_parity.py:164-199``;
* sparse attention with sink: ``flash_sparse/reference.py:44-130``;
  LSE: ``flash_sparse/triton/sparse_attn_fwd.py:148-177``;
* sparse-attention backward from the saved (o, lse):
  ``flash_sparse/triton/sparse_attn_bwd.py:1-26,93-97,224-283``;
* fp8 / fp4 quantisation: ``flash_sparse/utils/quantization.py:19-65`` (the
  simulations, with the rounding of every torch op to the input dtype) and the
  packed production formats its docstring names (``quantization.py:3-9``);
  the token compressor: ``flash_sparse/reference.py:176-272``;
* CSA / HCA attention index rows: ``flash_sparse/csa.py:30-83,176-179``,
  ``flash_sparse/hca.py:24-51``, window ``flash_sparse/reference.py:460-475``.

Parity status: every function here is pinned by ``tests/test_oracle.py``
(brute force on tiny inputs, closed forms, invariants, and torch's own CPU
``einsum``/``topk``/``softmax`` as an independent library implementation).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compiles ``liboracle.so`` with the committed Makefile (gcc, OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        L.oracle_indexer_scores.argtypes = [P, P, P, I, I, I, I, P, I, P]
        L.oracle_indexer_scores.restype = None
        L.oracle_indexer_scores_lim.argtypes = [P, P, P, I, I, I, I, P, I, P, P]
        L.oracle_indexer_scores_lim.restype = None
        L.oracle_indexer_scores_f32.argtypes = [P, P, P, I, I, I, I, P, I, P]
        L.oracle_indexer_scores_f32.restype = None
        L.oracle_topk.argtypes = [P, I, I, P, P, I, P, P]
        L.oracle_topk.restype = None
        L.oracle_sparse_attn.argtypes = [P, P, P, P, I, I, I, I, I, ctypes.c_double, P, P]
        L.oracle_sparse_attn_bwd.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, ctypes.c_double, P, I, P, P, P]
        L.oracle_sparse_attn.restype = None
        L.oracle_sparse_attn_t.argtypes = [P, P, P, P, I, I, I, I, I, ctypes.c_double, ctypes.c_int, P, P]
        L.oracle_sparse_attn_t.restype = None
        L.oracle_sparse_attn_bwd_t.argtypes = [P, P, P, P, P, P, P, I, I, I, I, I, ctypes.c_double, P, I,
                                               ctypes.c_int, P, P, P]
        L.oracle_sparse_attn_bwd_t.restype = None
        L.oracle_f16_to_f32.argtypes = [P, I, P]
        L.oracle_f16_to_f32.restype = None
        L.oracle_fill_normal.argtypes = [I, I, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float, P, P]
        L.oracle_fill_normal.restype = None
        L.oracle_normal_digest.argtypes = [ctypes.c_int, I, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float, P, P]
        L.oracle_normal_digest.restype = None
        L.oracle_philox4x32_10.argtypes = [P, P, P]
        L.oracle_philox4x32_10.restype = None
        L.oracle_fill_normal_at.argtypes = [P, I, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float, P, P]
        L.oracle_fill_normal_at.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------------------------------------------------------------------
# bf16 helpers (inputs are carried as raw uint16 bit patterns)
# ---------------------------------------------------------------------------
def bf16_bits_to_f64(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


# ---------------------------------------------------------------------------
# Indexer (C oracle)
# ---------------------------------------------------------------------------
def indexer_scores(q_bits: np.ndarray, k_bits: np.ndarray, w: np.ndarray, rows: Optional[np.ndarray] = None,
                   precision: str = "f64", lim: Optional[np.ndarray] = None) -> np.ndarray:
    """Scores ``I(s, t)`` for the selected query rows of ONE batch.

    q_bits [S,H,D] uint16 (bf16 bits), k_bits [T,D] uint16, w [S,H] float32.
    Returns [len(rows), T] float64 (or float32 with ``precision='f32'``).
    With ``lim`` (f64 only), row r is scored for keys t < lim[r] only and holds
    NaN beyond (those keys are illegal and never read by the top-k).
    """
    S, H, D = q_bits.shape
    T = k_bits.shape[0]
    q_bits = np.ascontiguousarray(q_bits, dtype=np.uint16)
    k_bits = np.ascontiguousarray(k_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows = np.arange(S, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, dtype=np.int64)
    if precision == "f64":
        out = np.empty((len(rows), T), dtype=np.float64)
        if lim is None:
            lib().oracle_indexer_scores(_ptr(q_bits), _ptr(k_bits), _ptr(w), S, T, H, D, _ptr(rows), len(rows),
                                        _ptr(out))
        else:
            lim = np.ascontiguousarray(lim, dtype=np.int64)
            assert lim.shape == rows.shape
            lib().oracle_indexer_scores_lim(_ptr(q_bits), _ptr(k_bits), _ptr(w), S, T, H, D, _ptr(rows),
                                            len(rows), _ptr(lim), _ptr(out))
    else:
        out = np.empty((len(rows), T), dtype=np.float32)
        lib().oracle_indexer_scores_f32(_ptr(q_bits), _ptr(k_bits), _ptr(w), S, T, H, D, _ptr(rows), len(rows),
                                        _ptr(out))
    return out


def legal_limits(rows: np.ndarray, T: int, causal_ratio: Optional[int]) -> np.ndarray:
    """Number of legal leading keys per row: ``min(T, (s+1)//ratio)`` or ``T``."""
    rows = np.asarray(rows, dtype=np.int64)
    if causal_ratio is None:
        return np.full(rows.shape, T, dtype=np.int64)
    return np.minimum(T, (rows + 1) // int(causal_ratio)).astype(np.int64)


def topk(scores: np.ndarray, lim: np.ndarray, top_k: int, mask: Optional[np.ndarray] = None):
    """Per-row top-k (score desc, index asc) over legal keys, width ``top_k``."""
    scores = np.ascontiguousarray(scores, dtype=np.float64)
    n, T = scores.shape
    lim = np.ascontiguousarray(lim, dtype=np.int64)
    idx = np.empty((n, top_k), dtype=np.int64)
    val = np.empty((n, top_k), dtype=np.float64)
    mptr = None
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.uint8)
        mptr = _ptr(mask)
    lib().oracle_topk(_ptr(scores), n, T, _ptr(lim), mptr, top_k, _ptr(idx), _ptr(val))
    return idx, val


def indexer_topk_rows(q_bits, k_bits, w, top_k: int, *, rows=None, causal_ratio=None, mask_rows=None):
    """Materialise-then-topk for the selected rows of one batch.

    Returns (idx [n,top_k] int64, score [n,top_k] float64, scores [n,T] float64).
    """
    S = q_bits.shape[0]
    T = k_bits.shape[0]
    rows = np.arange(S, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
    sc = indexer_scores(q_bits, k_bits, w, rows)
    lim = legal_limits(rows, T, causal_ratio)
    idx, val = topk(sc, lim, top_k, mask_rows)
    return idx, val, sc


# ---------------------------------------------------------------------------
# Sparse attention (C oracle)
# ---------------------------------------------------------------------------
def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """IEEE binary16 bit patterns -> float32 through the C oracle's decoder."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_f16_to_f32(_ptr(b), b.size, _ptr(out))
    return out


def synth_normal(start: int, n: int, seed: int, stream: int, scale: float = 1.0, bf16: bool = False) -> np.ndarray:
    """Elements [start, start + n) of the counter-based synthetic tensor
    (seed, stream) times ``scale``: float32, or bf16 bit patterns (uint16).
    Restates ``streamindex_amd/csrc/synth.hip`` (``si_fill_normal``)."""
    if bf16:
        out = np.empty(n, dtype=np.uint16)
        lib().oracle_fill_normal(start, n, seed, stream, scale, None, _ptr(out))
    else:
        out = np.empty(n, dtype=np.float32)
        lib().oracle_fill_normal(start, n, seed, stream, scale, _ptr(out), None)
    return out


def synth_normal_at(idx: np.ndarray, seed: int, stream: int, scale: float = 1.0, bf16: bool = False) -> np.ndarray:
    """The synthetic tensor (seed, stream) at the flat indices ``idx``."""
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    if bf16:
        out = np.empty(idx.shape, dtype=np.uint16)
        lib().oracle_fill_normal_at(_ptr(idx), idx.size, seed, stream, scale, None, _ptr(out))
    else:
        out = np.empty(idx.shape, dtype=np.float32)
        lib().oracle_fill_normal_at(_ptr(idx), idx.size, seed, stream, scale, _ptr(out), None)
    return out


def philox4x32_10(ctr, key) -> tuple:
    """One Philox4x32-10 block: 4 counter words, 2 key words -> 4 words."""
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.empty(4, dtype=np.uint32)
    lib().oracle_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return tuple(int(x) for x in out)


def synth_digest(n: int, seed: int, stream: int, scale: float = 1.0, bf16: bool = False):
    """(d1, d2) over the little-endian 16-bit words w_j of the whole tensor:
    d1 = sum w_j, d2 = sum w_j (j mod 65521 + 1), both mod 2^64."""
    d1 = np.zeros(1, dtype=np.uint64)
    d2 = np.zeros(1, dtype=np.uint64)
    lib().oracle_normal_digest(1 if bf16 else 0, n, seed, stream, scale, _ptr(d1), _ptr(d2))
    return int(d1[0]), int(d2[0])


def sparse_attn_rows(q_bits: np.ndarray, kv_bits: np.ndarray, sink: np.ndarray, idx: np.ndarray, scale: float,
                     f16: bool = False):
    """Reference sparse attention for ``n`` rows of one batch.

    q_bits [n,H,D] uint16, kv_bits [N,D] uint16 (bf16 bits, or fp16 bits with
    ``f16``), sink [H] f32, idx [n,K] int.
    Returns (o [n,H,D] float64, lse [n,H] float64).
    """
    n, H, D = q_bits.shape
    N = kv_bits.shape[0]
    K = idx.shape[1]
    q_bits = np.ascontiguousarray(q_bits, dtype=np.uint16)
    kv_bits = np.ascontiguousarray(kv_bits, dtype=np.uint16)
    sink = np.ascontiguousarray(sink, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    o = np.empty((n, H, D), dtype=np.float64)
    lse = np.empty((n, H), dtype=np.float64)
    lib().oracle_sparse_attn_t(_ptr(q_bits), _ptr(kv_bits), _ptr(sink), _ptr(idx), n, H, D, N, K, float(scale),
                               1 if f16 else 0, _ptr(o), _ptr(lse))
    return o, lse


def sparse_attn_bwd_rows(q_bits, kv_bits, o_bits, do_bits, sink, lse, idx, scale: float, *, want_dq: bool = True,
                         keys: Optional[np.ndarray] = None, want_dkv: bool = True, f16: bool = False):
    """Reference sparse-attention backward for ``n`` rows of one batch.

    q_bits, o_bits, do_bits [n,H,D] uint16; kv_bits [N,D] uint16 (bf16 bits,
    or fp16 bits with ``f16``); sink [H] f32;
    lse [n,H] f32; idx [n,K] int.  Returns (dq [n,H,D] or None, dkv, dsink [H]),
    all float64.  dkv is [N,D] over every key, or [len(keys),D] for the listed
    keys only (the contributions of these ``n`` rows; a sampled check passes
    every row that selects a listed key).  dsink sums over the ``n`` rows.
    """
    n, H, D = q_bits.shape
    N = kv_bits.shape[0]
    K = idx.shape[1]
    arrs = [np.ascontiguousarray(x, dtype=np.uint16) for x in (q_bits, kv_bits, o_bits, do_bits)]
    sink = np.ascontiguousarray(sink, dtype=np.float32)
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    dq = np.empty((n, H, D), dtype=np.float64) if want_dq else None
    key_slot = None
    nslot = N
    if keys is not None:
        keys = np.asarray(keys, dtype=np.int64)
        key_slot = np.full(N, -1, dtype=np.int64)
        key_slot[keys] = np.arange(len(keys))
        nslot = len(keys)
    dkv = np.zeros((nslot, D), dtype=np.float64) if want_dkv else None
    dsink = np.zeros(H, dtype=np.float64)
    lib().oracle_sparse_attn_bwd_t(_ptr(arrs[0]), _ptr(arrs[1]), _ptr(arrs[2]), _ptr(arrs[3]), _ptr(sink), _ptr(lse),
                                   _ptr(idx), n, H, D, N, K, float(scale),
                                   None if key_slot is None else _ptr(key_slot), nslot if want_dkv else 0,
                                   1 if f16 else 0, None if dq is None else _ptr(dq),
                                   None if dkv is None else _ptr(dkv), _ptr(dsink))
    return dq, dkv, dsink


# ---------------------------------------------------------------------------
# numpy restatements (tiny shapes only; cross-checks of the C oracle)
# ---------------------------------------------------------------------------
def np_indexer_scores(qf: np.ndarray, kf: np.ndarray, w: np.ndarray) -> np.ndarray:
    """qf [S,H,D], kf [T,D], w [S,H] (float64) -> [S,T]; reference.py:165-168."""
    qk = np.einsum("shd,td->sht", qf, kf)
    return (np.maximum(qk, 0.0) * w[:, :, None]).sum(axis=1)


def np_topk(scores: np.ndarray, lim: np.ndarray, top_k: int) -> tuple:
    """Lexicographic (score desc, index asc) selection with -1/-inf padding."""
    n, T = scores.shape
    idx = np.full((n, top_k), -1, dtype=np.int64)
    val = np.full((n, top_k), -np.inf)
    for r in range(n):
        L = int(min(T, lim[r]))
        t = np.arange(L)
        order = np.lexsort((t, -scores[r, :L]))[:top_k]
        idx[r, : len(order)] = t[order]
        val[r, : len(order)] = scores[r, order]
    return idx, val


def np_chunked_topk(scores: np.ndarray, lim: np.ndarray, top_k: int, chunk_t: int) -> tuple:
    """Partition-merge restatement of chunked_indexer.py:112-155 on a score row
    block: per-chunk top-min(k,cT) then merge into a running top-k."""
    n, T = scores.shape
    run_i = np.full((n, top_k), -1, dtype=np.int64)
    run_v = np.full((n, top_k), -np.inf)
    for t0 in range(0, T, chunk_t):
        t1 = min(t0 + chunk_t, T)
        blk = scores[:, t0:t1].copy()
        tt = np.arange(t0, t1)
        blk[tt[None, :] >= lim[:, None]] = -np.inf
        kc = min(top_k, t1 - t0)
        ci = np.empty((n, kc), dtype=np.int64)
        cv = np.empty((n, kc))
        for r in range(n):
            o = np.lexsort((tt, -blk[r]))[:kc]
            ci[r] = tt[o]
            cv[r] = blk[r, o]
        ci = np.where(np.isinf(cv), -1, ci)
        allv = np.concatenate([run_v, cv], axis=1)
        alli = np.concatenate([run_i, ci], axis=1)
        for r in range(n):
            # -1 sorts after every real index among -inf ties
            key_i = np.where(alli[r] < 0, np.iinfo(np.int64).max, alli[r])
            o = np.lexsort((key_i, -allv[r]))[:top_k]
            run_v[r] = allv[r, o]
            run_i[r] = alli[r, o]
        run_i = np.where(np.isinf(run_v), -1, run_i)
    return run_i, run_v


def np_sparse_attn(qf: np.ndarray, kvf: np.ndarray, sink: np.ndarray, idx: np.ndarray, scale: float):
    """qf [n,H,D], kvf [N,D], sink [H], idx [n,K] -> (o [n,H,D], lse [n,H]); reference.py:93-130."""
    n, H, D = qf.shape
    valid = (idx >= 0) & (idx < kvf.shape[0])                     # out of range: masked, as -1
    g = kvf[np.where(valid, idx, 0)] * valid[..., None]           # [n,K,D]
    sc = np.einsum("nhd,nkd->nhk", qf, g) * scale
    sc = np.where(valid[:, None, :], sc, -np.inf)
    mx = np.maximum(sc.max(axis=-1), sink[None, :])                 # [n,H]
    p = np.exp(sc - mx[..., None])
    den = p.sum(-1) + np.exp(sink[None, :] - mx)
    o = np.einsum("nhk,nkd->nhd", p, g) / den[..., None]
    lse = np.log(den) + mx
    return o, lse


def np_sparse_attn_bwd(qf, kvf, of, dof, sink, lse, idx, scale: float):
    """Backward of np_sparse_attn from its saved (o, lse), as
    sparse_attn_bwd.py:1-26 states it: p = e^{scale q.k - lse},
    ds = p (do.k - sum_d o do) scale, dq = sum_j ds k_j,
    dkv[idx_j] += ds q + p do, dsink = -sum_rows e^{sink - lse} (o.do).
    All float64; returns (dq [n,H,D], dkv [N,D], dsink [H])."""
    n, H, D = qf.shape
    N = kvf.shape[0]
    valid = (idx >= 0) & (idx < N)
    safe = np.where(valid, idx, 0)
    g = kvf[safe] * valid[..., None]                                  # [n,K,D]
    z = np.einsum("nhd,nkd->nhk", qf, g) * scale
    p = np.where(valid[:, None, :], np.exp(z - lse[..., None]), 0.0)  # [n,H,K]
    delta = (of * dof).sum(-1)                                        # [n,H]
    dp = np.einsum("nhd,nkd->nhk", dof, g)
    ds = p * (dp - delta[..., None]) * scale
    dq = np.einsum("nhk,nkd->nhd", ds, g)
    contrib = np.einsum("nhk,nhd->nkd", ds, qf) + np.einsum("nhk,nhd->nkd", p, dof)
    dkv = np.zeros((N, D))
    np.add.at(dkv, safe[valid], contrib[valid])
    dsink = -(np.exp(sink[None, :] - lse) * delta).sum(0)
    return dq, dkv, dsink


# ---------------------------------------------------------------------------
# FP8 / FP4 quantisation (utils/quantization.py) and the token compressor
# ---------------------------------------------------------------------------
FP4_GRID = np.array([-6, -4, -3, -2, -1.5, -1, -0.5, 0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=np.float64)
FP4_CODES = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, 0, -0.5, -1, -1.5, -2, -3, -4, -6], dtype=np.float64)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to bf16 / fp16 (nearest, ties to even) or keep fp32;
    returns float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float32":
        return x
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def e4m3_round(x: np.ndarray) -> np.ndarray:
    """Nearest OCP fp8 e4m3 value (bias 7, 3 mantissa bits, subnormal step
    2^-9, max 448), ties to even; |x| <= 448 expected."""
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    with np.errstate(divide="ignore"):
        ex = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    ex = np.maximum(ex, -6)
    q = np.exp2(ex - 3)
    r = np.minimum(np.round(a / q) * q, 448.0)  # np.round: ties to even
    return np.where(a > 0, np.copysign(r, x), x)


def act_quant_simulate(x: np.ndarray, dtype: str, block_size: int = 128) -> np.ndarray:
    """quantization.py:19-37 with every torch op rounded to ``dtype``."""
    x = np.asarray(x, dtype=np.float32)
    blk = x.reshape(*x.shape[:-1], -1, block_size)
    amax = round_to(np.maximum(np.abs(blk).max(-1, keepdims=True), np.float32(1e-4)), dtype)
    scale = round_to(amax / np.float32(448.0), dtype)
    y = np.clip(round_to(blk / scale, dtype), -448.0, 448.0)
    q = e4m3_round(y).astype(np.float32)
    return round_to(q * scale, dtype).reshape(x.shape)


def fp4_act_quant_simulate(x: np.ndarray, dtype: str, block_size: int = 32) -> np.ndarray:
    """quantization.py:40-65 with every torch op rounded to ``dtype`` (argmin
    over the diffs rounded to ``dtype``; first minimum wins)."""
    x = np.asarray(x, dtype=np.float32)
    blk = x.reshape(*x.shape[:-1], -1, block_size)
    amax = round_to(np.maximum(np.abs(blk).max(-1, keepdims=True), np.float32(6 * 2.0 ** -126)), dtype)
    scale = round_to(amax / np.float32(6.0), dtype)
    y = np.clip(round_to(blk / scale, dtype), -6.0, 6.0)
    diffs = np.abs(round_to(y[..., None] - FP4_GRID.astype(np.float32), dtype))
    q = FP4_GRID.astype(np.float32)[np.argmin(diffs, axis=-1)]
    return round_to(q * scale, dtype).reshape(x.shape)


def fp8_pack(x: np.ndarray, block_size: int = 128, pow2: bool = False):
    """Production fp8: (e4m3 values as float64, fp32 scale per block)."""
    x = np.asarray(x, dtype=np.float32)
    blk = x.reshape(*x.shape[:-1], -1, block_size)
    amax = np.maximum(np.abs(blk).max(-1, keepdims=True), np.float32(1e-4))
    scale = (amax / np.float32(448.0)).astype(np.float32)
    if pow2:
        scale = np.exp2(np.ceil(np.log2(scale.astype(np.float64)))).astype(np.float32)
    y = np.clip((blk / scale).astype(np.float32), -448.0, 448.0)
    return e4m3_round(y).reshape(x.shape), scale[..., 0]


def e2m1_round(y: np.ndarray) -> np.ndarray:
    """Nearest e2m1 value, ties to the even code (0, 1, 2, 4 have even codes)."""
    a = np.abs(np.asarray(y, dtype=np.float64))
    mags = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])
    d = np.abs(a[..., None] - mags)
    best = d.min(-1, keepdims=True)
    tie_ok = (d == best) & ((np.arange(8) % 2) == 0)      # prefer an even code among ties
    idx = np.where(tie_ok.any(-1), np.argmax(tie_ok, -1), np.argmin(d, -1))
    return np.copysign(mags[idx], y) * (mags[idx] > 0)


def fp4_pack(x: np.ndarray, block_size: int = 32):
    """Production fp4: (e2m1 values as float64, power-of-two fp32 scale per block)."""
    x = np.asarray(x, dtype=np.float32)
    blk = x.reshape(*x.shape[:-1], -1, block_size)
    amax = np.maximum(np.abs(blk).max(-1, keepdims=True), np.float32(6 * 2.0 ** -126))
    ratio = (amax / np.float32(6.0)).astype(np.float32).astype(np.float64)
    scale = np.exp2(np.ceil(np.log2(ratio))).astype(np.float32)
    return e2m1_round((blk / scale).astype(np.float32)).reshape(x.shape), scale[..., 0]


def fp4_unpack(packed: np.ndarray) -> np.ndarray:
    """uint8 [..., n/2] (element 2i in the low nibble) -> e2m1 values [..., n]."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,))
    out[..., 0::2] = FP4_CODES[p & 15]
    out[..., 1::2] = FP4_CODES[p >> 4]
    return out


def token_compressor(c_a, z_a, b_a, m, c_b=None, z_b=None, b_b=None, overlap=False):
    """reference.py:176-272 in float64 (overlap: block i pools [block i of a ;
    block i-1 of b], block 0's b half empty)."""
    c_a, z_a, b_a = (np.asarray(t, dtype=np.float64) for t in (c_a, z_a, b_a))
    B, S, C = c_a.shape
    n = S // m
    ca = c_a[:, :n * m].reshape(B, n, m, C)
    za = z_a[:, :n * m].reshape(B, n, m, C) + b_a
    if not overlap:
        w = np.exp(za - za.max(2, keepdims=True))
        return (ca * w).sum(2) / w.sum(2)
    cb = np.asarray(c_b, dtype=np.float64)[:, :n * m].reshape(B, n, m, C)
    zb = np.asarray(z_b, dtype=np.float64)[:, :n * m].reshape(B, n, m, C) + np.asarray(b_b, dtype=np.float64)
    cbs = np.zeros_like(cb)
    cbs[:, 1:] = cb[:, :-1]
    zbs = np.full_like(zb, -np.inf)
    zbs[:, 1:] = zb[:, :-1]
    cj = np.concatenate([ca, cbs], 2)
    zj = np.concatenate([za, zbs], 2)
    w = np.exp(zj - zj.max(2, keepdims=True))
    return (cj * w).sum(2) / w.sum(2)


# ---------------------------------------------------------------------------
# CSA / HCA attention index rows (integer work: numpy)
# ---------------------------------------------------------------------------
def window_idxs(rows: np.ndarray, n_win: int) -> np.ndarray:
    """Sliding-window columns ``[n, n_win]`` (``flash_sparse/reference.py:460-475``):
    column j of query s is ``s - n_win + 1 + j`` when that lies in ``[0, s]``, else -1."""
    s = np.asarray(rows, dtype=np.int64)[:, None]
    t = s - n_win + 1 + np.arange(n_win, dtype=np.int64)[None, :]
    return np.where((t >= 0) & (t <= s), t, -1)


def csa_idx_rows(comp_idx: np.ndarray, rows: np.ndarray, n_win: int, offset: int) -> np.ndarray:
    """CSA attention index rows ``[n, n_win + K]`` from per-row compressed picks
    (``flash_sparse/csa.py:76-83``, and ``:176-179`` for the chunked path):
    window columns, then each pick ``+ offset`` (-1 stays -1)."""
    comp = np.asarray(comp_idx, dtype=np.int64)
    comp = np.where(comp >= 0, comp + offset, -1)
    return np.concatenate([window_idxs(rows, n_win), comp], axis=1)


def csa_scores_topk_rows(scores: np.ndarray, rows: np.ndarray, m: int, top_k: int, n_win: int,
                         offset: int) -> np.ndarray:
    """``build_csa_topk_idxs`` (``flash_sparse/csa.py:59-83``) for the given rows of one
    batch: causal mask ``m(i+1)-1 <= s``, top-min(k,T) with ties by smaller index,
    selected ``-inf`` -> -1, padding to ``top_k``, window + offset."""
    rows = np.asarray(rows, dtype=np.int64)
    lim = legal_limits(rows, scores.shape[1], m)
    idx, val = topk(scores, lim, top_k)
    idx = np.where(np.isneginf(val), -1, idx)
    return csa_idx_rows(idx, rows, n_win, offset)


def hca_idx_rows(rows: np.ndarray, n_win: int, n_comp: int, m_prime: int, offset: int) -> np.ndarray:
    """HCA attention index rows ``[n, n_win + n_comp]`` (``flash_sparse/hca.py:40-51``):
    window columns, then compressed entry i as ``i + offset`` where
    ``m_prime·(i+1) - 1 <= s``, else -1."""
    s = np.asarray(rows, dtype=np.int64)[:, None]
    i = np.arange(n_comp, dtype=np.int64)[None, :]
    comp = np.where(m_prime * (i + 1) - 1 <= s, i + offset, -1)
    return np.concatenate([window_idxs(rows, n_win), comp], axis=1)


# ---------------------------------------------------------------------------
# Metrics
# ---------------------------------------------------------------------------
def set_overlap_recall(idx_a: np.ndarray, idx_b: np.ndarray) -> np.ndarray:
    """Per-row |valid_a ∩ valid_b| / |valid_a| (eval/test_v4_indexer_parity.py:164-199).

    Negative entries are padding.  Both empty -> 1; a empty, b non-empty -> 0.
    Accepts [..., K] arrays; returns [...] float64.
    """
    a = np.asarray(idx_a, dtype=np.int64)
    b = np.asarray(idx_b, dtype=np.int64)
    lead = a.shape[:-1]
    a2 = a.reshape(-1, a.shape[-1])
    b2 = b.reshape(-1, b.shape[-1])
    out = np.empty(a2.shape[0])
    for r in range(a2.shape[0]):
        va = set(int(x) for x in a2[r] if x >= 0)
        vb = set(int(x) for x in b2[r] if x >= 0)
        if not va:
            out[r] = 1.0 if not vb else 0.0
        else:
            out[r] = len(va & vb) / len(va)
    return out.reshape(lead)

