"""C-ABI checks that need no GPU: the library loads, exports every function
include/dsa_hip.h declares with the ctypes signatures the host uses, and its
argument validation returns the documented status codes before any device
work (so no call below touches a GPU)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from cppmega_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from cppmega_amd import build_lib
        build_lib.build()
    return _lib.load()


def test_header_and_binding_agree():
    declared = _declared_functions()
    assert declared == sorted(_lib.EXPORTED_SYMBOLS)
    assert set(_lib._SIGNATURES) == set(declared)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_functions():
        assert hasattr(raw, name), f"{name} missing from libdsa_hip.so"


def test_abi_version_and_status_codes(lib):
    assert lib.dsa_abi_version() == 201
    text = open(HEADER).read()
    for name, val in (("DSA_OK", 0), ("DSA_ERR_INVALID_ARG", -1), ("DSA_ERR_UNSUPPORTED", -2),
                      ("DSA_ERR_HIP", -3), ("DSA_ERR_WORKSPACE", -4)):
        assert re.search(rf"\b{name}\s*=\s*{val}\b", text), name
        assert getattr(_lib, name) == val


def _err(lib):
    return lib.dsa_last_error().decode()


def test_fwd_rejects_bad_arguments(lib):
    # (B, S, S_kv, H, G, D_qk, D_v, topk, dtype)
    bad = [
        (1, 4, 0, 16, 1, 128, 64, 32, 0),     # S_kv = 0
        (1, 4, 8, 16, 3, 128, 64, 32, 0),     # H not divisible by G
        (1, 4, 8, 16, 1, 128, 256, 32, 0),    # d_v > d_qk
        (1, 4, 8, 16, 1, 128, 64, 32, 7),     # unknown dtype
        (1, 4, 8, 16, 1, 128, 64, 0, 0),      # topk = 0
        (1, 4, 8, 16, 1, 128, 64, 32, 0),     # null pointers
        (1, 4, 8, 16, 1, 128, 64, 32, 1),     # e4m3 without scales (and null pointers)
    ]
    for B, S, Skv, H, G, D, dv, k, dt in bad:
        rc = lib.dsa_sparse_mla_fwd(None, None, None, None, None, B, S, Skv, H, G, D, dv, k,
                                    0.1, dt, None, None, None)
        assert rc == _lib.DSA_ERR_INVALID_ARG, (B, S, Skv, H, G, D, dv, k, dt)
        assert "dsa_sparse_mla_fwd" in _err(lib)
    # empty problems are a no-op success
    assert lib.dsa_sparse_mla_fwd(None, None, None, None, None, 0, 4, 8, 16, 1, 128, 64, 32,
                                  0.1, 0, None, None, None) == _lib.DSA_OK


def test_bwd_workspace_and_validation(lib):
    ws = lib.dsa_sparse_mla_bwd_workspace_size
    a = ws(2, 4096, 4096, 32, 1, 128, 64, 256, 0, 0)
    b = ws(2, 4096, 4096, 32, 1, 128, 64, 256, _lib.BWD_FP32_PARTIALS, 0)
    c = ws(1, 4096, 4096, 32, 1, 128, 64, 256, 0, 0)
    # fp16 partial rows: 2 * 4096 * 256 entries x 256 B, fp32 doubles them
    assert a >= 2 * 4096 * 256 * 128 * 2 and b > a and c < a
    assert ws(2, 4096, 4096, 32, 1, 128, 64, 256, 0, 0) == a      # deterministic
    rc = lib.dsa_sparse_mla_bwd(*([None] * 10), 0, 1, 4, 8, 16, 1, 128, 64, 32, 0.1, 0, None, None, 8, 0, None)
    assert rc == _lib.DSA_ERR_INVALID_ARG and "flags" in _err(lib)
    rc = lib.dsa_sparse_mla_bwd(*([None] * 10), 0, 1, 4, 70000, 16, 1, 128, 64, 32, 0.1, 0, None, None, 0, 0, None)
    assert rc == _lib.DSA_ERR_INVALID_ARG


def test_indexer_and_topk_validation(lib):
    rc = lib.dsa_indexer_scores(None, None, None, None, 1, 8, 8, 16, 64, 0, 2, None, None, 0, 1, None)
    assert rc == _lib.DSA_ERR_INVALID_ARG
    rc = lib.dsa_indexer_scores(None, None, None, None, 1, 8, 8, 16, 64, 0, 2, None, None, 5, 1, None)
    assert rc == _lib.DSA_ERR_INVALID_ARG
    # row_stride < row_len
    rc = lib.dsa_topk(None, 4, 100, 50, 4, 0, 0, None, None, 8, None, None)
    assert rc == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_topk(None, 0, 100, 100, 4, 0, 0, None, None, 8, None, None) == _lib.DSA_OK


def test_fp8_quantize_validation(lib):
    assert lib.dsa_fp8_quantize_workspace_size() >= 4 * 1024
    rc = lib.dsa_fp8_tensorwise_quantize(None, 16, 9, None, None, None, 0, None)
    assert rc == _lib.DSA_ERR_INVALID_ARG


def test_bwd_workspace_bounded_by_pass_cap(lib):
    """The backward runs in passes sized to a per-call cap on its partial dKV
    rows (the pass_bytes argument, 0 = 4 GiB), so its workspace is bounded: at
    cfg5 (s = 16384, h = 128, d_qk = 576, topk = 2048) one pass would hold
    ~155 GB of fp16 rows; with the default cap the workspace stays under 5 GiB,
    and a smaller cap shrinks it further (down to one 32-token chunk per pass,
    ~302 MB of rows at cfg5).  The cap is an argument, not process state: two
    queries with different caps do not affect each other."""
    wsz = lib.dsa_sparse_mla_bwd_workspace_size
    ws = int(wsz(1, 16384, 16384, 128, 1, 576, 512, 2048, 0, 0))
    assert 0 < ws < 5 * (1 << 30), ws
    assert int(wsz(1, 16384, 16384, 128, 1, 576, 512, 2048, 0, 4 << 30)) == ws
    ws_small = int(wsz(1, 16384, 16384, 128, 1, 576, 512, 2048, 0, 256 << 20))
    assert ws_small < ws and ws_small < 512 << 20, ws_small
    assert int(wsz(1, 16384, 16384, 128, 1, 576, 512, 2048, 0, 0)) == ws      # no state left behind
    # cfg2 fits one pass: its size does not depend on the cap while the cap covers it
    one = int(wsz(2, 4096, 4096, 32, 1, 128, 64, 256, 0, 0))
    assert one > 2 * 4096 * 256 * 257
    # the index is prebuilt only for a one-pass plan; its size follows the cap
    assert int(lib.dsa_sparse_mla_bwd_index_size(2, 4096, 4096, 32, 1, 128, 64, 256, 0, 0)) > 0
    assert int(lib.dsa_sparse_mla_bwd_index_size(2, 4096, 4096, 32, 1, 128, 64, 256, 0, 64 << 20)) == 0
    assert int(lib.dsa_sparse_mla_bwd_indexed_workspace_size(2, 4096, 4096, 32, 1, 128, 64, 256, 0, 0)) < one


def test_fused_indexer_topk_limits(lib):
    """The fused indexer + top-k's top-k bound per shape, and its refusals
    (unsupported shape, top-k past the bound, bad flags, null pointers)
    before any device work."""
    assert lib.dsa_indexer_topk_fused_max_topk(16, 64) == 832
    assert lib.dsa_indexer_topk_fused_max_topk(32, 128) == 1728
    assert lib.dsa_indexer_topk_fused_max_topk(64, 128) == 3520
    assert lib.dsa_indexer_topk_fused_max_topk(48, 64) == 0
    assert lib.dsa_indexer_topk_fused_max_topk(16, 96) == 0
    args = lambda H, D, k, causal=1, dt=_lib.DTYPE_BF16: (None, None, None, None, None, 2, 8, 8, H, D, dt,
                                                          _lib.DTYPE_F32, None, None, k, causal, 1, None)
    assert lib.dsa_indexer_topk_fused(*args(16, 64, 833)) == _lib.DSA_ERR_UNSUPPORTED
    assert "at most 832" in _err(lib)
    assert lib.dsa_indexer_topk_fused(*args(48, 64, 8)) == _lib.DSA_ERR_UNSUPPORTED
    assert lib.dsa_indexer_topk_fused(*args(16, 64, 8, causal=2)) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_indexer_topk_fused(*args(16, 64, 8, dt=7)) == _lib.DSA_ERR_INVALID_ARG
    assert lib.dsa_indexer_topk_fused(*args(16, 64, 8)) == _lib.DSA_ERR_INVALID_ARG  # null pointers
    assert "null tensor pointer" in _err(lib)
