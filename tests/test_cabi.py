"""CPU-only checks of the C ABI boundary (no kernel is launched).

* libstreamindex.so exists, loads, and exports every entry point declared in
  include/streamindex.h; the ctypes binding covers exactly those entries.
* Host-side argument validation returns the documented status codes before
  any HIP call, and the Python layer maps them to the reference's exception
  types (AssertionError for device/shape, ValueError for unsupported dims,
  as flash_sparse/triton/indexer_score.py:138-150 and sparse_attn_fwd.py:205-218).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from streamindex_amd import _lib
from streamindex_amd.build import LIB_PATH

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "streamindex.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(si_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB_PATH):
        pytest.skip("libstreamindex.so not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_expected_entries():
    names = _declared()
    for n in ("si_indexer_topk", "si_indexer_score", "si_sparse_attn_fwd", "si_last_error", "si_abi_version",
              "si_csa_indexer_topk", "si_csa_scores_topk", "si_hca_topk_idxs"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (si_[a-z0-9_]+)\b", out))
    declared = set(_declared())
    assert declared <= exported, f"missing exports: {declared - exported}"
    for n in declared:
        assert hasattr(lib, n)
    assert set(_lib.SIGNATURES) == declared


def test_version_and_workspace(lib):
    assert lib.si_abi_version() == 8
    # the top-k kernel knob: previous mode returned, out-of-range rejected
    assert lib.si_indexer_set_topk_kernel(2) == 0
    assert lib.si_indexer_set_topk_kernel(1) == 2
    assert lib.si_indexer_set_topk_kernel(7) == -1
    assert lib.si_indexer_set_topk_kernel(0) == 1
    assert lib.si_indexer_topk_workspace_bytes(1, 1 << 20, 1 << 18, 64, 128, 512) == 0


def _i64(*v):
    return (ctypes.c_int64 * len(v))(*v)


def test_c_validation_codes_without_gpu(lib):
    qs, ks, ws = _i64(8 * 64 * 128, 64 * 128, 128, 1), _i64(4 * 128, 128, 1), _i64(8 * 64, 64, 1)
    fake = 0x1000  # never dereferenced: every call below fails validation first
    # null strides
    rc = lib.si_indexer_topk(fake, None, fake, ks, fake, 0, ws, None, None, 1, 8, 4, 64, 128, 4, 4, fake, fake, None)
    assert rc == _lib.SI_ERR_INVALID and b"stride" in lib.si_last_error()
    # top_k = 0
    rc = lib.si_indexer_topk(fake, qs, fake, ks, fake, 0, ws, None, None, 1, 8, 4, 64, 128, 0, 4, fake, fake, None)
    assert rc == _lib.SI_ERR_INVALID and b"top_k" in lib.si_last_error()
    # mask and ratio together
    rc = lib.si_indexer_topk(fake, qs, fake, ks, fake, 0, ws, fake, _i64(32, 4, 1), 1, 8, 4, 64, 128, 4, 4,
                             fake, fake, None)
    assert rc == _lib.SI_ERR_INVALID and b"either" in lib.si_last_error()
    # non-contiguous head dim
    rc = lib.si_indexer_topk(fake, _i64(8 * 64 * 128, 64 * 128, 128, 2), fake, ks, fake, 0, ws, None, None,
                             1, 8, 4, 64, 128, 4, 4, fake, fake, None)
    assert rc == _lib.SI_ERR_INVALID
    # unsupported shape (D=48) is reported as such
    rc = lib.si_indexer_topk(fake, _i64(8 * 64 * 48, 64 * 48, 48, 1), fake, _i64(4 * 48, 48, 1), fake, 0, ws,
                             None, None, 1, 8, 4, 64, 48, 4, 4, fake, fake, None)
    assert rc == _lib.SI_ERR_UNSUPPORTED and b"D_I=48" in lib.si_last_error()
    # top_k beyond the kernel limit
    rc = lib.si_indexer_topk(fake, qs, fake, ks, fake, 0, ws, None, None, 1, 8, 4, 64, 128, 4097, 4, fake, fake,
                             None)
    assert rc == _lib.SI_ERR_UNSUPPORTED and b"4096" in lib.si_last_error()
    # H_I beyond the kernel limit
    qs257 = _i64(8 * 257 * 128, 257 * 128, 128, 1)
    rc = lib.si_indexer_topk(fake, qs257, fake, ks, fake, 0, _i64(8 * 257, 257, 1), None, None, 1, 8, 4, 257, 128,
                             4, 4, fake, fake, None)
    assert rc == _lib.SI_ERR_UNSUPPORTED and b"256" in lib.si_last_error()
    # sparse attention: unsupported head dim
    o4 = _i64(64 * 100, 64 * 100, 100, 1)
    rc = lib.si_sparse_attn_fwd(fake, o4, fake, _i64(100 * 16, 100, 1), fake, fake, 1, _i64(32, 8, 1),
                                1, 4, 64, 100, 16, 8, 0.1, 0, fake, o4, fake, _i64(256, 64, 1), None)
    assert rc == _lib.SI_ERR_INVALID or rc == _lib.SI_ERR_UNSUPPORTED
    # sparse attention: element types other than bf16 (0) and fp16 (1)
    q4 = _i64(64 * 128, 64 * 128, 128, 1)
    rc = lib.si_sparse_attn_fwd(fake, q4, fake, _i64(100 * 128, 128, 1), fake, fake, 1, _i64(32, 8, 1),
                                1, 4, 64, 128, 16, 8, 0.1, 2, fake, q4, fake, _i64(256, 64, 1), None)
    assert rc == _lib.SI_ERR_INVALID and b"qkv_dtype" in lib.si_last_error()
    # empty problems succeed without touching memory
    rc = lib.si_indexer_topk(None, qs, fake, ks, None, 0, ws, None, None, 1, 0, 4, 64, 128, 4, 4, None, None, None)
    assert rc == _lib.SI_OK
    # ... but a non-empty key set still needs its pointer
    rc = lib.si_indexer_topk(None, qs, None, ks, None, 0, ws, None, None, 1, 0, 4, 64, 128, 4, 4, None, None, None)
    assert rc == _lib.SI_ERR_INVALID


def _plan(lib, S, T, H, D, top_k, ratio=0):
    kern, cap = ctypes.c_int32(-1), ctypes.c_int32(-1)
    rc = lib.si_indexer_topk_plan(S, T, H, D, top_k, ratio, ctypes.byref(kern), ctypes.byref(cap))
    return rc, kern.value, cap.value


NARROW_K, WIDE_K, SPLIT_K = 1, 2, 3


def test_topk_dispatch_plan_without_gpu(lib):
    """The dispatch of si_indexer_topk, read through si_indexer_topk_plan (no launch)."""
    S = 1 << 16
    # config[1]: two-workgroup kernel with the 1536-key buffer; S = 1M rows reach 64K legal keys: four-M-block
    assert _plan(lib, S, S // 4, 64, 128, 512, 4) == (0, NARROW_K, 1536)
    assert _plan(lib, 1 << 20, 1 << 18, 64, 128, 512, 4) == (0, WIDE_K, 1536)
    # 128 heads at D = 128: four-M-block kernel, but never with fewer than 64 keys (its tile copies
    # would re-read rows past T), whatever the forced mode
    assert _plan(lib, 96, 300, 128, 128, 40)[:2] == (0, WIDE_K)
    for T in (1, 37, 63):
        assert _plan(lib, 96, T, 128, 128, 40)[:2] == (0, NARROW_K)
    prev = lib.si_indexer_set_topk_kernel(2)
    try:
        assert _plan(lib, 96, 63, 64, 128, 40)[:2] == (0, NARROW_K)
        assert _plan(lib, 96, 64, 64, 128, 40)[:2] == (0, WIDE_K)
    finally:
        lib.si_indexer_set_topk_kernel(prev)
    # capacities of the two-workgroup kernel per top_k
    for k, cap in ((32, 256), (33, 512), (192, 512), (193, 1536), (1152, 1536), (1153, 2048), (1536, 2048),
                   (1537, 4096), (2048, 4096)):
        assert _plan(lib, 96, 3000, 64, 128, k) == (0, NARROW_K, cap), k
    # past what one wave holds: the head-split kernel
    assert _plan(lib, 96, 3000, 192, 128, 512) == (0, SPLIT_K, 1536)
    assert _plan(lib, 96, 3000, 256, 64, 2000) == (0, SPLIT_K, 4608)
    assert _plan(lib, 96, 3000, 64, 128, 2049) == (0, SPLIT_K, 4608)
    assert _plan(lib, 96, 3000, 64, 128, 4096) == (0, SPLIT_K, 4608)
    assert _plan(lib, 96, 3000, 96, 256, 512) == (0, SPLIT_K, 1536)
    assert _plan(lib, 96, 3000, 64, 256, 1537) == (0, SPLIT_K, 4608)
    assert _plan(lib, 96, 3000, 256, 256, 4096) == (0, SPLIT_K, 4608)
    # limits
    assert _plan(lib, 96, 3000, 257, 128, 8)[0] == _lib.SI_ERR_UNSUPPORTED
    assert _plan(lib, 96, 3000, 64, 128, 4097)[0] == _lib.SI_ERR_UNSUPPORTED
    assert _plan(lib, 96, 3000, 64, 48, 8)[0] == _lib.SI_ERR_UNSUPPORTED
    assert _plan(lib, 96, 3000, 64, 128, 0)[0] == _lib.SI_ERR_INVALID


def test_csa_hca_validation_codes_without_gpu(lib):
    qs, ks, ws = _i64(8 * 64 * 128, 64 * 128, 128, 1), _i64(4 * 128, 128, 1), _i64(8 * 64, 64, 1)
    os_ = _i64(8 * 24, 24, 1)
    fake = 0x1000  # never dereferenced: every call below fails validation first
    # fused CSA rows: the +S offset must keep indices inside int32
    rc = lib.si_csa_indexer_topk(fake, qs, fake, ks, fake, 0, ws, 1, 8, 4, 64, 128, 16, 4, 8, (1 << 31) - 2,
                                 fake, os_, None, None)
    assert rc == _lib.SI_ERR_UNSUPPORTED and b"int32" in lib.si_last_error()
    rc = lib.si_csa_indexer_topk(fake, qs, fake, ks, fake, 0, ws, 1, 8, 4, 64, 128, 16, 4, -1, 8, fake, os_,
                                 None, None)
    assert rc == _lib.SI_ERR_INVALID and b"n_win" in lib.si_last_error()
    rc = lib.si_csa_indexer_topk(fake, qs, fake, ks, fake, 0, ws, 1, 8, 4, 64, 128, 16, 4, 8, 8, fake,
                                 _i64(8 * 24, 24, 2), None, None)
    assert rc == _lib.SI_ERR_INVALID and b"contiguous" in lib.si_last_error()
    # materialised-score CSA rows
    ss = _i64(8 * 4, 4, 1)
    rc = lib.si_csa_scores_topk(fake, ss, 1, 8, 4, 0, 4, 8, 8, fake, os_, None)
    assert rc == _lib.SI_ERR_INVALID and b"top_k" in lib.si_last_error()
    rc = lib.si_csa_scores_topk(fake, ss, 1, 8, 4, 4097, 4, 8, 8, fake, os_, None)
    assert rc == _lib.SI_ERR_UNSUPPORTED
    rc = lib.si_csa_scores_topk(fake, ss, 1, 0, 4, 16, 4, 8, 8, None, os_, None)  # empty: no launch
    assert rc == _lib.SI_OK
    # HCA rows
    rc = lib.si_hca_topk_idxs(1, 8, 4, 2, 0, 8, fake, os_, None)
    assert rc == _lib.SI_ERR_INVALID and b"m_prime" in lib.si_last_error()
    rc = lib.si_hca_topk_idxs(1, 0, 4, 2, 4, 0, None, os_, None)
    assert rc == _lib.SI_OK


def test_backward_and_inverted_index_limits_without_gpu(lib):
    # sizes whose (query, slot) pair positions would not fit the int32 segment bounds
    assert lib.si_build_inverted_topk_workspace_bytes(1, 1 << 21, 1 << 10, 4096) == -1
    assert b"too large" in lib.si_last_error()
    assert lib.si_sparse_attn_bwd_workspace_bytes(1, 1 << 31, 64, 576, 4096, 512, 1 << 30) == -1
    assert b"int32" in lib.si_last_error()
    assert lib.si_sparse_attn_bwd_workspace_bytes(1, 16, 64, 100, 64, 8, 1 << 30) == -1
    assert b"D=100" in lib.si_last_error()


def test_python_layer_errors_on_cpu_tensors():
    from streamindex_amd import chunked_indexer_topk, indexer_score, sparse_attn_fwd

    q = torch.zeros(1, 8, 16, 32, dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 32, dtype=torch.bfloat16)
    w = torch.zeros(1, 8, 16)
    with pytest.raises(AssertionError):
        chunked_indexer_topk(q, k, w, 4, causal_ratio=4)
    with pytest.raises(AssertionError):
        indexer_score(q, k, w)
    with pytest.raises(AssertionError):
        sparse_attn_fwd(torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16), torch.zeros(1, 4, 64, dtype=torch.bfloat16),
                        torch.zeros(16), torch.zeros(1, 2, 4, dtype=torch.int64))
    from streamindex_amd import build_csa_topk_idxs, flash_csa_forward, flash_hca_forward

    with pytest.raises(AssertionError):  # T != n_compressed (csa.py:56)
        build_csa_topk_idxs(torch.zeros(1, 8, 2), 4, 2, seq_len=8, n_compressed=3, m=4, device="cpu")
    with pytest.raises(AssertionError):  # CPU scores
        build_csa_topk_idxs(torch.zeros(1, 8, 2), 4, 2, seq_len=8, n_compressed=2, m=4, device="cpu")
    with pytest.raises(AssertionError):  # kv shape (csa.py:128)
        flash_csa_forward(torch.zeros(1, 8, 4, 32, dtype=torch.bfloat16), torch.zeros(1, 7, 32, dtype=torch.bfloat16),
                          torch.zeros(1, 2, 32, dtype=torch.bfloat16), q, k, w, torch.zeros(4), n_win=4, top_k=2)
    with pytest.raises(AssertionError):
        flash_hca_forward(torch.zeros(1, 8, 4, 32, dtype=torch.bfloat16), torch.zeros(1, 8, 32, dtype=torch.bfloat16),
                          torch.zeros(1, 2, 32, dtype=torch.bfloat16), torch.zeros(4), n_win=4, m_prime=4)


def test_error_mapping():
    _lib.check(_lib.SI_OK)
    if os.path.exists(LIB_PATH):
        with pytest.raises(ValueError):
            _lib.check(_lib.SI_ERR_INVALID)
        with pytest.raises(ValueError):
            _lib.check(_lib.SI_ERR_UNSUPPORTED)
        with pytest.raises(RuntimeError):
            _lib.check(_lib.SI_ERR_LAUNCH)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.ExtensionNotBuilt):
        _lib.load()


def test_reference_import_paths():
    import flash_sparse.triton as ft
    from flash_sparse.triton.chunked_indexer import chunked_indexer_topk
    from flash_sparse.triton.indexer_score import indexer_score, indexer_score_topk
    from flash_sparse.triton.sparse_attn_fwd import sparse_attn_fwd
    from flash_sparse.csa import build_csa_topk_idxs, flash_csa_forward
    from flash_sparse.hca import build_hca_topk_idxs, flash_hca_forward

    import streamindex_amd as si

    assert flash_csa_forward is si.flash_csa_forward and build_csa_topk_idxs is si.build_csa_topk_idxs
    assert flash_hca_forward is si.flash_hca_forward and build_hca_topk_idxs is si.build_hca_topk_idxs
    assert chunked_indexer_topk is si.chunked_indexer_topk
    assert indexer_score is si.indexer_score and indexer_score_topk is si.indexer_score_topk
    assert sparse_attn_fwd is si.sparse_attn_fwd and ft.sparse_attn is si.sparse_attn
    assert ft.sparse_attn_fwd is si.sparse_attn_fwd   # still the function after the submodule import

    from flash_sparse.triton.sparse_attn_bwd import sparse_attn_bwd
    from flash_sparse.triton.sparse_attn_bwd_v2 import sparse_attn_bwd_v2
    from flash_sparse.triton.inverted_topk import build_inverted_topk
    from flash_sparse.triton.indexer_streaming_topk import streaming_indexer_topk
    from flash_sparse.utils.quantization import act_quant_simulate, fp4_act_quant_simulate
    from flash_sparse.utils.compression import softmax_gated_pool

    assert ft.sparse_attn_bwd is sparse_attn_bwd is si.sparse_attn_bwd
    assert sparse_attn_bwd_v2 is si.sparse_attn_bwd_v2 and build_inverted_topk is si.build_inverted_topk
    from streamindex_amd import compressor, quant

    assert act_quant_simulate is quant.act_quant_simulate and fp4_act_quant_simulate is quant.fp4_act_quant_simulate
    assert softmax_gated_pool is compressor.softmax_gated_pool
    assert callable(streaming_indexer_topk)


def test_synth_legal_pairs_closed_form():
    from streamindex_amd import synth

    for S in (1, 3, 4, 5, 17, 64, 1000):
        for T in (0, 1, 3, 16, 100, 5000):
            for r in (1, 2, 4, 7):
                assert synth.legal_pairs(S, T, r) == sum(min(T, (s + 1) // r) for s in range(S))
    S = 1 << 16
    assert synth.legal_pairs(S, S // 4, 4) == S * S // 8 - S // 4
    assert synth.indexer_flops(S, S // 4, 64, 128, 4) == 2.0 * 64 * 128 * (S * S // 8 - S // 4)
