"""Shared host-side helpers of the SparseMLA entry points."""
from __future__ import annotations

import torch

from .. import _lib


def normalize_sm_scale(sm_scale, d_qk: int) -> float:
    """None -> d_qk^-0.5; a tensor is read once on the host (as the reference
    does, cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:74-82)."""
    if sm_scale is None:
        return float(d_qk) ** -0.5
    if isinstance(sm_scale, torch.Tensor):
        return float(sm_scale.detach().item())
    return float(sm_scale)


_NOT_LOOKED_UP = object()
_QUANTIZED_TENSOR = _NOT_LOOKED_UP


def _quantized_tensor_type():
    """Transformer Engine's QuantizedTensor class, or None without TE.  Looked up
    once per process: a failed import is not cached by Python, and this runs
    several times per SparseMLA call."""
    global _QUANTIZED_TENSOR
    if _QUANTIZED_TENSOR is _NOT_LOOKED_UP:
        try:
            from transformer_engine.pytorch.tensor import QuantizedTensor  # type: ignore
        except ImportError:
            QuantizedTensor = None
        _QUANTIZED_TENSOR = QuantizedTensor
    return _QUANTIZED_TENSOR


def unwrap_quantized(t):
    """Dequantise a Transformer-Engine QuantizedTensor if one is passed (TE is
    optional; plain tensors are returned unchanged)."""
    if isinstance(t, torch.Tensor) and type(t) is torch.Tensor:
        return t
    qt = _quantized_tensor_type()
    if qt is not None and isinstance(t, qt):
        return t.dequantize()
    return t


def stream_of(t: torch.Tensor) -> tuple[int, int]:
    dev = _lib.ensure_device(t)
    return dev, _lib.stream_ptr(dev)


def check_same_device(*ts):
    devs = {t.device for t in ts if t is not None}
    assert len(devs) == 1, f"all tensors must be on one device, got {sorted(map(str, devs))}"
