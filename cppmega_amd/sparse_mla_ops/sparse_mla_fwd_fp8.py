"""FP8 (OCP e4m3, tensorwise scale) SparseMLA forward and the quantiser.

Mirrors cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:
``per_token_cast_to_fp8`` (:396-412, TE current/tensorwise scaling with the
per-tensor scale broadcast to one value per row) and
``sparse_mla_fwd_fp8_interface`` (:415-559).  QK^T runs on e4m3 codes and is
multiplied by q_scale[token] * kv_scale[row]; V is dequantised to bf16 per row.
"""
from __future__ import annotations

import os

import torch

from .. import _lib
from ._common import check_same_device, normalize_sm_scale, stream_of
from .sparse_mla_fwd import _launch_fwd

_TE_TENSORWISE_SPARSE_MLA_ALIASES = {"te", "te_current", "te_tensorwise", "tensorwise"}


def _enforce_te_tensorwise_quant_backend() -> None:
    """Same gate as the reference (tilelang_sparse_mla_fwd_fp8.py:35-43)."""
    backend = os.getenv("CPPMEGA_SPARSE_MLA_FP8_QUANT", "te_tensorwise").strip().lower()
    if backend not in _TE_TENSORWISE_SPARSE_MLA_ALIASES:
        raise RuntimeError(
            "CPPMEGA_SPARSE_MLA_FP8_QUANT no longer supports "
            f"{backend!r}. SparseMLA FP8 is hard-wired to current/tensorwise "
            "scaling.")


def tensorwise_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x (bf16 or f32, any shape) -> (e4m3 tensor of the same shape, scale_inv 0-dim f32)."""
    assert x.dtype in (torch.bfloat16, torch.float32), f"quantiser input must be bf16 or f32, got {x.dtype}"
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    scale_inv = torch.empty((), dtype=torch.float32, device=x.device)
    L = _lib.load()
    ws_bytes = int(L.dsa_fp8_quantize_workspace_size())
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _, stream = stream_of(x)
    code = _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F32
    rc = L.dsa_fp8_tensorwise_quantize(x.data_ptr(), x.numel(), code, out.data_ptr(), scale_inv.data_ptr(),
                                       ws.data_ptr(), ws_bytes, stream)
    _lib.check(rc, "dsa_fp8_tensorwise_quantize")
    return out, scale_inv


def fp8_dequantize(x8: torch.Tensor, scale_inv: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """e4m3 tensor (any shape) + one-element scale_inv -> value * scale_inv as bf16 (RNE) or f32
    (the role of Float8Tensor.dequantize() for the tensors SparseMLA_FP8 unpacks)."""
    assert x8.dtype == torch.float8_e4m3fn, f"expected float8_e4m3fn, got {x8.dtype}"
    assert dtype in (torch.bfloat16, torch.float32), f"dequantised dtype must be bf16 or f32, got {dtype}"
    x8 = x8.contiguous()
    scale_inv = scale_inv.reshape(-1)[:1].to(device=x8.device, dtype=torch.float32).contiguous()
    out = torch.empty(x8.shape, dtype=dtype, device=x8.device)
    _, stream = stream_of(x8)
    rc = _lib.load().dsa_fp8_dequantize(x8.data_ptr(), x8.numel(), scale_inv.data_ptr(), out.data_ptr(),
                                        _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32, stream)
    _lib.check(rc, "dsa_fp8_dequantize")
    return out


def per_token_cast_to_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Tensorwise e4m3 cast; the tensor scale is broadcast to shape x.shape[:-1]
    (the historical per-token name and ABI of the reference are kept)."""
    _enforce_te_tensorwise_quant_backend()
    data, scale_inv = tensorwise_quantize(x)
    return data, scale_inv.expand(x.shape[:-1]).contiguous()


def sparse_mla_fwd_fp8_interface(
    q,
    kv,
    indices,
    q_scale=None,
    kv_scale=None,
    sm_scale=None,
    return_p_sum: bool = False,
    d_v=512,
    block_I=64,
    num_stages=2,
    threads=256,
):
    """FP8 sparse-MLA forward -> (out bf16 [B,S,H,d_v], lse2 f32 [B,S,H]).

    q / kv may be bf16 (quantised here) or float8_e4m3fn with q_scale [B,S] /
    kv_scale [B,S_kv] dequant factors (real = fp8 * scale).
    """
    squeeze_batch = q.ndim == 3
    if squeeze_batch:
        q, kv, indices = q.unsqueeze(0), kv.unsqueeze(0), indices.unsqueeze(0)
        if q_scale is not None:
            q_scale = q_scale.unsqueeze(0)
        if kv_scale is not None:
            kv_scale = kv_scale.unsqueeze(0)

    assert return_p_sum is False, "This kernel file is for fwd only"
    assert q.is_contiguous() and kv.is_contiguous() and indices.is_contiguous()
    batch, seq_len, heads, dim_plus_tail_dim = q.shape
    _, seq_len_kv, kv_group, kv_dim = kv.shape
    assert kv_dim == dim_plus_tail_dim, "q and kv must have the same embedding dimension on the last axis"
    dim = d_v
    assert 0 < dim <= dim_plus_tail_dim, f"d_v must be in (0, {dim_plus_tail_dim}], but got {dim}"
    assert kv.shape[0] == batch
    topk = indices.shape[-1]
    assert indices.shape == (batch, seq_len, kv_group, topk)
    assert indices.dtype == torch.int32, f"indices must be int32, got {indices.dtype}"
    assert heads % kv_group == 0

    if q.dtype != torch.float8_e4m3fn:
        q_flat = q.reshape(batch * seq_len, heads * dim_plus_tail_dim)
        q8, qs = per_token_cast_to_fp8(q_flat)
        q = q8.reshape(batch, seq_len, heads, dim_plus_tail_dim)
        q_scale = qs.reshape(batch, seq_len)
    else:
        assert q_scale is not None, "q_scale required when q is pre-quantized FP8"
    if kv.dtype != torch.float8_e4m3fn:
        kv_flat = kv.reshape(batch * seq_len_kv, kv_group * dim_plus_tail_dim)
        k8, ks = per_token_cast_to_fp8(kv_flat)
        kv = k8.reshape(batch, seq_len_kv, kv_group, dim_plus_tail_dim)
        kv_scale = ks.reshape(batch, seq_len_kv)
    else:
        assert kv_scale is not None, "kv_scale required when kv is pre-quantized FP8"
    q_scale = q_scale.to(torch.float32).reshape(batch, seq_len).contiguous()
    kv_scale = kv_scale.to(torch.float32).reshape(batch, seq_len_kv).contiguous()
    check_same_device(q, kv, indices, q_scale, kv_scale)

    scale = normalize_sm_scale(sm_scale, dim_plus_tail_dim)
    out, lse = _launch_fwd(q.contiguous(), kv.contiguous(), indices, scale, dim, _lib.DTYPE_E4M3,
                           q_scale, kv_scale)
    if squeeze_batch:
        out, lse = out.squeeze(0), lse.squeeze(0)
    return out, lse
