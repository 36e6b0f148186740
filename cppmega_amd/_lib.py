"""ctypes binding of libdsa_hip.so (the C-ABI declared in include/dsa_hip.h).

The product path has exactly one implementation: these HIP kernels.  If the
library is missing or the device is not a gfx950 GPU every entry point
raises; nothing falls back to a CPU or PyTorch implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libdsa_hip.so")

DSA_OK = 0
DSA_ERR_INVALID_ARG = -1
DSA_ERR_UNSUPPORTED = -2
DSA_ERR_HIP = -3
DSA_ERR_WORKSPACE = -4

DTYPE_BF16 = 0
DTYPE_E4M3 = 1
DTYPE_F32 = 2
DTYPE_I32 = 3
DTYPE_I64 = 4
DTYPE_MXFP8 = 5

BWD_FP32_PARTIALS = 1

# Every symbol include/dsa_hip.h declares (checked by the CPU test suite).
EXPORTED_SYMBOLS = (
    "dsa_last_error",
    "dsa_abi_version",
    "dsa_device_check",
    "dsa_sparse_mla_fwd",
    "dsa_sparse_mla_fwd_workspace_size",
    "dsa_sparse_mla_fwd_ws",
    "dsa_sparse_mla_bwd_workspace_size",
    "dsa_sparse_mla_bwd_index_size",
    "dsa_sparse_mla_bwd_indexed_workspace_size",
    "dsa_sparse_mla_bwd_build_index",
    "dsa_sparse_mla_bwd_indexed",
    "dsa_sparse_mla_bwd",
    "dsa_indexer_scores",
    "dsa_indexer_scores_masked",
    "dsa_mask_windows",
    "dsa_topk_finalize",
    "dsa_indexer_scores_backward_workspace_size",
    "dsa_indexer_scores_backward",
    "dsa_indexer_topk_streaming_workspace_size",
    "dsa_indexer_topk_streaming",
    "dsa_indexer_topk_fused_max_topk",
    "dsa_indexer_topk_fused",
    "dsa_topk",
    "dsa_topk_workspace_size",
    "dsa_topk_ws",
    "dsa_fp8_quantize_workspace_size",
    "dsa_fp8_tensorwise_quantize",
    "dsa_fp8_tensorwise_quantize_noalloc",
    "dsa_fp8_dequantize",
    "dsa_fp8_dequantize_blockwise",
    "dsa_indexer_kl_loss_workspace_size",
    "dsa_indexer_kl_loss",
    "dsa_indexer_kl_loss_backward",
    "dsa_topk_index_mask",
    "dsa_stage_timing",
    "dsa_stage_times",
)

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_size_t = ctypes.c_size_t
_u64 = ctypes.c_uint64

_SIGNATURES = {
    "dsa_last_error": (ctypes.c_char_p, []),
    "dsa_abi_version": (_i32, []),
    "dsa_device_check": (_i32, [_i32]),
    "dsa_sparse_mla_fwd": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _f32, _i32, _c_void_p, _c_void_p, _c_void_p]),
    "dsa_sparse_mla_fwd_workspace_size": (_size_t, [_i64] * 5 + [_i32]),
    "dsa_sparse_mla_fwd_ws": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _f32, _i32, _c_void_p, _c_void_p, _c_void_p, _size_t, _c_void_p]),
    "dsa_sparse_mla_bwd_workspace_size": (_size_t, [_i64] * 8 + [_i32, _u64]),
    "dsa_sparse_mla_bwd_index_size": (_size_t, [_i64] * 8 + [_i32, _u64]),
    "dsa_sparse_mla_bwd_indexed_workspace_size": (_size_t, [_i64] * 8 + [_i32, _u64]),
    "dsa_sparse_mla_bwd_build_index": (_i32, [_c_void_p] + [_i64] * 8 + [_i32, _u64, _c_void_p, _size_t,
                                                                          _c_void_p]),
    "dsa_sparse_mla_bwd_indexed": (_i32, [_c_void_p] * 9 + [_c_void_p, _size_t, _c_void_p, _size_t] + [_i64] * 8
                                   + [_f32, _i32, _c_void_p, _c_void_p, _i32, _u64, _c_void_p]),
    "dsa_sparse_mla_bwd": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                  _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _size_t,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _f32, _i32, _c_void_p, _c_void_p, _i32, _u64, _c_void_p]),
    "dsa_indexer_scores": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                  _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                                  _c_void_p, _c_void_p, _i32, _i32, _c_void_p]),
    "dsa_indexer_scores_masked": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                         _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                                         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                         _c_void_p, _i32, _c_void_p]),
    "dsa_mask_windows": (_i32, [_c_void_p, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "dsa_topk_finalize": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p]),
    "dsa_indexer_scores_backward_workspace_size": (_size_t, [_i64] * 5),
    "dsa_indexer_scores_backward": (_i32, [_c_void_p] * 7 + [_i64] * 5 + [_i32] * 4
                                    + [_c_void_p, _c_void_p, _c_void_p, _size_t, _c_void_p]),
    "dsa_indexer_topk_streaming_workspace_size": (_size_t, [_i64] * 4),
    "dsa_indexer_topk_streaming": (_i32, [_c_void_p] * 5 + [_i64] * 5 + [_i32, _i32, _c_void_p, _c_void_p, _i64,
                                                                         _i32, _i32, _c_void_p, _size_t, _c_void_p]),
    "dsa_indexer_topk_fused_max_topk": (_i64, [_i64, _i64]),
    "dsa_indexer_topk_fused": (_i32, [_c_void_p] * 5 + [_i64] * 5 + [_i32, _i32, _c_void_p, _c_void_p, _i64,
                                                                     _i32, _i32, _c_void_p]),
    "dsa_topk": (_i32, [_c_void_p, _i64, _i64, _i64, _i64, _i32, _i64,
                        _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p]),
    "dsa_topk_workspace_size": (_size_t, [_i64, _i64, _i64]),
    "dsa_topk_ws": (_i32, [_c_void_p, _i64, _i64, _i64, _i64, _i32, _i64,
                           _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _size_t, _c_void_p]),
    "dsa_fp8_quantize_workspace_size": (_size_t, []),
    "dsa_fp8_tensorwise_quantize": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p,
                                           _c_void_p, _size_t, _c_void_p]),
    "dsa_fp8_tensorwise_quantize_noalloc": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p]),
    "dsa_fp8_dequantize": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i32, _c_void_p]),
    "dsa_fp8_dequantize_blockwise": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _c_void_p]),
    "dsa_indexer_kl_loss_workspace_size": (_size_t, [_i64] * 5 + [_i32]),
    "dsa_indexer_kl_loss": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32,
                                   _c_void_p, _size_t, _c_void_p]),
    "dsa_indexer_kl_loss_backward": (_i32, [_c_void_p, _c_void_p, _i32, _i64, _c_void_p, _c_void_p, _c_void_p,
                                            _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32,
                                            _c_void_p, _size_t, _c_void_p]),
    "dsa_topk_index_mask": (_i32, [_c_void_p, _i32, _i64, _c_void_p, _i64, _i64, _i64, _i64, _i64,
                                   _f32, _f32, _i32, _c_void_p]),
    "dsa_stage_timing": (_i32, [_i32]),
    "dsa_stage_times": (_i32, [_i32, ctypes.POINTER(ctypes.c_float), _i32]),
}

_lock = threading.Lock()
_lib = None
_checked_devices: set[int] = set()


class DSAError(RuntimeError):
    """A non-zero status returned by libdsa_hip.so."""

    def __init__(self, what: str, code: int, message: str):
        super().__init__(f"{what} failed (status {code}): {message}")
        self.code = code


def load():
    """Load libdsa_hip.so (raises RuntimeError when it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m cppmega_amd.build_lib` "
                    "(or __graft_entry__.build()); there is no fallback implementation")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != DSA_OK:
        msg = load().dsa_last_error().decode(errors="replace")
        raise DSAError(what, rc, msg)


def ensure_device(t: torch.Tensor) -> int:
    """Fail closed unless `t` lives on a gfx950 GPU; returns the device index."""
    if not t.is_cuda:
        raise RuntimeError(
            f"cppmega_amd kernels need tensors on a gfx950 GPU (got device {t.device}); "
            "there is no CPU path")
    dev = t.device.index if t.device.index is not None else torch.cuda.current_device()
    if dev not in _checked_devices:
        check(load().dsa_device_check(dev), "dsa_device_check")
        _checked_devices.add(dev)
    return dev


def stream_ptr(device: int) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


BWD_STAGES = ("csr", "main", "reduce")


def stage_timing(enable: bool) -> None:
    """Turn per-stage HIP-event timing of dsa_sparse_mla_bwd on or off for this thread."""
    load().dsa_stage_timing(1 if enable else 0)


def stage_times(back: int = 0, max_stages: int = 8) -> list[float]:
    """Elapsed ms per stage of the timed call `back` calls ago (waits for its events)."""
    buf = (ctypes.c_float * max_stages)()
    n = load().dsa_stage_times(int(back), buf, max_stages)
    if n < 0:
        check(n, "dsa_stage_times")
    return [float(buf[i]) for i in range(n)]
