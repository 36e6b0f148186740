"""MXFP8 block-scaled SparseMLA on gfx950.

Drop-in for cppmega's experimental block-scaled path:
  * ``sparse_mla_blockscaled_mxfp8_fwd_interface`` (tilelang_sparse_mla_blockscaled_fused.py:694-793)
    and the public ``sparse_mla_blockscaled_mxfp8_forward`` (sparse_mla.py:180-219);
  * ``sparse_mla_blockscaled_mxfp8_backward`` (sparse_mla.py:222-262), which
    returns gradients with respect to the logical dequantised Q and KV.

Inputs are pre-quantised MXFP8 payloads: q_data [B,S,H,D] / kv_data [B,S_kv,G,D]
float8_e4m3fn with f32 scales q_scale [B,S,H,D/32] / kv_scale [B,S_kv,G,D/32],
one per 32 consecutive channels; indices [B,S,G,topk] int32 (-1 sentinel).
The forward is one gfx950 kernel (``dsa_sparse_mla_fwd`` with
``DSA_DTYPE_MXFP8``): every 32-channel block's q.k over the e4m3 codes runs on
MFMA and is scaled by the two block scales before the blocks are summed,
online exp2 softmax, V dequantised per block into LDS, PV on MFMA, LSE in log2
units.  The backward dequantises Q and KV to bf16 with their block scales
(``dsa_fp8_dequantize_blockwise``), recomputes the forward in bf16 and runs the
bf16 SparseMLA backward, i.e. the gradient the reference's correctness
backward defines (tilelang_sparse_mla_blockscaled_fused.py:1015-1051) without
materialising scores; the reference's own TileLang backward is disabled
(it produced non-finite gradients), so this path needs no acknowledgement
variable.  Both raise unless ``CPPMEGA_SPARSE_MLA_BLOCKSCALED_FUSED=1``, as the
reference's public wrappers do.
"""
from __future__ import annotations

import os

import torch

from .. import _lib
from ._common import normalize_sm_scale, stream_of

__all__ = [
    "MXFP8_BLOCK_SIZE",
    "mxfp8_dequantize",
    "sparse_mla_blockscaled_mxfp8_backward",
    "sparse_mla_blockscaled_mxfp8_forward",
    "sparse_mla_blockscaled_mxfp8_fwd_interface",
]

MXFP8_BLOCK_SIZE = 32
_BLOCKSCALED_FUSED_ENV = "CPPMEGA_SPARSE_MLA_BLOCKSCALED_FUSED"


def _env_enabled(name: str) -> bool:
    return os.getenv(name, "0").strip().lower() in ("1", "true", "yes", "on")


def _validate_mxfp8_inputs(q_data, kv_data, q_scale, kv_scale, indices, *, d_v):
    """Same checks and error types as the reference (tilelang_sparse_mla_blockscaled_fused.py:84-157)."""
    for name, tensor in (("q_data", q_data), ("kv_data", kv_data), ("q_scale", q_scale), ("kv_scale", kv_scale),
                         ("indices", indices)):
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if q_data.device.type != "cuda":
        raise RuntimeError("block-scaled SparseMLA requires GPU tensors")
    if not (q_data.device == kv_data.device == q_scale.device == kv_scale.device == indices.device):
        raise ValueError("all block-scaled SparseMLA tensors must be on the same device")
    if q_data.dtype != torch.float8_e4m3fn or kv_data.dtype != torch.float8_e4m3fn:
        raise ValueError("MXFP8 block-scaled SparseMLA data tensors must be torch.float8_e4m3fn")
    if q_scale.dtype != torch.float32 or kv_scale.dtype != torch.float32:
        raise ValueError("MXFP8 block-scaled SparseMLA scales must be torch.float32")
    if indices.dtype != torch.int32:
        raise ValueError("indices must be torch.int32 with -1 sentinel")
    if q_data.ndim != 4 or kv_data.ndim != 4 or q_scale.ndim != 4 or kv_scale.ndim != 4:
        raise ValueError("q_data, kv_data, q_scale and kv_scale must be rank 4")
    if indices.ndim != 4:
        raise ValueError("indices must be rank 4 [B,S,G,topk]")
    batch, seq_len, heads, dim_total = q_data.shape
    kv_batch, seq_len_kv, kv_group, kv_dim = kv_data.shape
    if batch != kv_batch:
        raise ValueError(f"batch mismatch: q={batch}, kv={kv_batch}")
    if dim_total != kv_dim:
        raise ValueError(f"q/kv dim mismatch: q={dim_total}, kv={kv_dim}")
    if dim_total % MXFP8_BLOCK_SIZE:
        raise ValueError(f"MXFP8 D_total must be divisible by {MXFP8_BLOCK_SIZE}, got {dim_total}")
    if d_v <= 0 or d_v > dim_total:
        raise ValueError(f"d_v must be in (0, {dim_total}], got {d_v}")
    if d_v % 16:
        raise ValueError(f"d_v must be divisible by 16, got {d_v}")
    tail_dim = dim_total - d_v
    if tail_dim <= 0 or tail_dim % 16:
        raise ValueError("block-scaled SparseMLA requires a positive tail_dim divisible by 16; "
                         f"got tail_dim={tail_dim}")
    if heads % kv_group:
        raise ValueError(f"heads={heads} must be divisible by kv_group={kv_group}")
    topk = indices.shape[-1]
    if indices.shape != (batch, seq_len, kv_group, topk):
        raise ValueError(f"indices shape mismatch: expected {(batch, seq_len, kv_group, topk)}, "
                         f"got {tuple(indices.shape)}")
    nb = dim_total // MXFP8_BLOCK_SIZE
    if q_scale.shape != (batch, seq_len, heads, nb):
        raise ValueError(f"q_scale shape mismatch: expected {(batch, seq_len, heads, nb)}, got {tuple(q_scale.shape)}")
    if kv_scale.shape != (batch, seq_len_kv, kv_group, nb):
        raise ValueError(f"kv_scale shape mismatch: expected {(batch, seq_len_kv, kv_group, nb)}, "
                         f"got {tuple(kv_scale.shape)}")
    return batch, seq_len, seq_len_kv, heads, dim_total, kv_group, topk


def mxfp8_dequantize(data, scale, dtype=torch.bfloat16):
    """e4m3 [..., D] with f32 block scales [..., D/32] -> value * scale (bf16 RNE or f32),
    the role of _dequantize_mxfp8_tensor (tilelang_sparse_mla_blockscaled_fused.py:961-969)."""
    if data.dtype != torch.float8_e4m3fn or scale.dtype != torch.float32:
        raise ValueError("mxfp8_dequantize expects float8_e4m3fn data and float32 scales")
    if scale.shape[:-1] != data.shape[:-1] or scale.shape[-1] * MXFP8_BLOCK_SIZE != data.shape[-1]:
        raise ValueError(f"scale {tuple(scale.shape)} does not hold one value per 32 channels of {tuple(data.shape)}")
    data, scale = data.contiguous(), scale.contiguous()
    out = torch.empty(data.shape, dtype=dtype, device=data.device)
    dev = _lib.ensure_device(data)
    rc = _lib.load().dsa_fp8_dequantize_blockwise(
        data.data_ptr(), data.numel(), MXFP8_BLOCK_SIZE, scale.data_ptr(), out.data_ptr(),
        _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F32, _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_fp8_dequantize_blockwise")
    return out


def sparse_mla_blockscaled_mxfp8_fwd_interface(q_data, kv_data, q_scale, kv_scale, indices, *, sm_scale=None,
                                               d_v: int = 512, block_i: int = 64, num_stages: int = 2,
                                               threads: int = 256):
    """Fused MXFP8 block-scaled SparseMLA forward -> (out bf16 [B,S,H,d_v], lse2 f32 [B,S,H]).

    block_i / num_stages / threads are the reference's TileLang tuning knobs,
    accepted and unused.  3-D inputs (no batch) give 3-D outputs."""
    del block_i, num_stages, threads
    squeeze_batch = q_data.ndim == 3
    if squeeze_batch:
        q_data, kv_data, q_scale, kv_scale, indices = (t.unsqueeze(0) for t in (q_data, kv_data, q_scale, kv_scale,
                                                                                 indices))
    batch, seq_len, seq_len_kv, heads, dim_total, kv_group, topk = _validate_mxfp8_inputs(
        q_data, kv_data, q_scale, kv_scale, indices, d_v=d_v)
    scale = normalize_sm_scale(sm_scale, dim_total)
    out = torch.empty((batch, seq_len, heads, d_v), dtype=torch.bfloat16, device=q_data.device)
    lse = torch.empty((batch, seq_len, heads), dtype=torch.float32, device=q_data.device)
    dev, stream = stream_of(q_data)
    L = _lib.load()
    # the kv rows are dequantised to bf16 once per call (with their block scales) into a
    # workspace; when every block scale is a power of two (so the dequantisation is
    # exact) the bf16 kernel runs on them with q converted at load, otherwise the
    # block-scaled e4m3 kernel runs (chosen on the device, no host sync)
    ws_bytes = int(L.dsa_sparse_mla_fwd_workspace_size(batch, seq_len_kv, kv_group, dim_total, d_v,
                                                       _lib.DTYPE_MXFP8))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q_data.device) if ws_bytes else None
    rc = L.dsa_sparse_mla_fwd_ws(
        q_data.data_ptr(), kv_data.data_ptr(), indices.data_ptr(), out.data_ptr(), lse.data_ptr(),
        batch, seq_len, seq_len_kv, heads, kv_group, dim_total, d_v, topk, scale, _lib.DTYPE_MXFP8,
        q_scale.data_ptr(), kv_scale.data_ptr(), _lib.ptr(ws), ws_bytes, stream)
    _lib.check(rc, "dsa_sparse_mla_fwd_ws(mxfp8)")
    if squeeze_batch:
        out, lse = out.squeeze(0), lse.squeeze(0)
    return out, lse


def _require_enabled():
    if not _env_enabled(_BLOCKSCALED_FUSED_ENV):
        raise RuntimeError(f"experimental fused block-scaled SparseMLA requires {_BLOCKSCALED_FUSED_ENV}=1")


def sparse_mla_blockscaled_mxfp8_forward(q_data, kv_data, q_scale, kv_scale, indices, *, softmax_scale, d_v: int,
                                         block_i: int = 64, num_stages: int = 2, threads: int = 256):
    """Public block-scaled forward (raises unless CPPMEGA_SPARSE_MLA_BLOCKSCALED_FUSED=1)."""
    _require_enabled()
    return sparse_mla_blockscaled_mxfp8_fwd_interface(q_data, kv_data, q_scale, kv_scale, indices,
                                                      sm_scale=softmax_scale, d_v=d_v, block_i=block_i,
                                                      num_stages=num_stages, threads=threads)


def sparse_mla_blockscaled_mxfp8_backward(q_data, kv_data, q_scale, kv_scale, out, grad_out, indices, lse, *,
                                          softmax_scale, d_v: int, block_size: int = 32, num_stages: int = 0,
                                          threads: int = 128):
    """(dq, dkv) bf16 with respect to the dequantised Q [B,S,H,D] and KV [B,S_kv,G,D].

    ``out`` / ``lse`` of the block-scaled forward are not needed (the
    reference's correctness backward discards them too): the bf16 forward on
    the dequantised tensors is recomputed, then the bf16 backward runs."""
    del out, lse, block_size, num_stages, threads
    _require_enabled()
    from .sparse_mla_bwd import sparse_mla_bwd
    from .sparse_mla_fwd import sparse_mla_fwd_interface

    _validate_mxfp8_inputs(q_data, kv_data, q_scale, kv_scale, indices, d_v=d_v)
    q = mxfp8_dequantize(q_data, q_scale)
    kv = mxfp8_dequantize(kv_data, kv_scale)
    o_b, lse_b = sparse_mla_fwd_interface(q, kv, indices, sm_scale=softmax_scale, d_v=d_v)
    return sparse_mla_bwd(q, kv, o_b, grad_out.to(torch.bfloat16).contiguous(), indices, lse_b,
                          sm_scale=softmax_scale, d_v=d_v)
