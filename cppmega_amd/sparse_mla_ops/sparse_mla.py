"""SparseMLA autograd functions and Megatron-layout adapters (gfx950 HIP).

Drop-in for cppmega/megatron/sparse_mla_ops/sparse_mla.py:
  * ``SparseMLA`` (:356-411) — bf16 forward/backward;
  * ``SparseMLA_FP8`` (:414-556) — e4m3 tensorwise forward/backward, accepting
    bf16 input (quantised here), a Float8Tensor-like object exposing
    ``_data`` / ``_scale_inv`` (zero-copy), or raising ``ValueError`` for raw
    float8 input without a scale;
  * ``sparse_mla_as_unfused_dsa`` / ``sparse_mla_fp8_as_unfused_dsa`` (:559-686)
    — Megatron ``unfused_dsa_fn`` signature adapters;
  * ``fused_sparse_mla_absorbed_fp8`` (:689-734).

Tensor layouts (packed latent KV, MQA):
  q       [batch, seq, heads, dim+tail]       (3-D without batch also accepted)
  kv      [batch, seq_kv, kv_group, dim+tail] (V = kv[..., :d_v])
  indices [batch, seq, kv_group, topk] int32, -1 = masked
  returns (out [batch, seq, heads, d_v] bf16, lse [batch, seq, heads] f32, log2 units)
"""
from __future__ import annotations

import logging

import torch

from ._common import unwrap_quantized
from .sparse_mla_bwd import build_inverse_index, side_stream, sparse_mla_bwd
from .sparse_mla_bwd_fp8 import sparse_mla_bwd_fp8
from .sparse_mla_fwd import sparse_mla_fwd_interface
from .sparse_mla_fwd_fp8 import _enforce_te_tensorwise_quant_backend, per_token_cast_to_fp8, \
    sparse_mla_fwd_fp8_interface

log = logging.getLogger(__name__)


def _extract_fp8_data(t):
    """(fp8 data, scale_inv) from a Float8Tensor-like object, else (None, None).

    Duck-typed on the ``_data`` / ``_scale_inv`` attributes TE's Float8Tensor
    exposes (cppmega/megatron/sparse_mla_ops/sparse_mla.py:310-353), so a ROCm
    Transformer Engine tensor is taken without a copy; TE itself is optional.
    """
    data = getattr(t, "_data", None)
    scale_inv = getattr(t, "_scale_inv", None)
    if data is None or scale_inv is None or not isinstance(data, torch.Tensor):
        return None, None
    if data.dtype == torch.float8_e4m3fn:
        fp8 = data
    elif data.dtype == torch.uint8 and getattr(getattr(t, "_fp8_dtype", None), "name", None) == "kFloat8E4M3":
        fp8 = data.view(torch.float8_e4m3fn)
    else:
        return None, None
    if data.data_ptr() == 0:
        return None, None
    return fp8, scale_inv


class SparseMLA(torch.autograd.Function):
    """Sparse MLA attention over packed latent KV (bf16), gfx950 kernels."""

    @staticmethod
    def forward(ctx, q, kv, indices, scaling, d_v=None):
        q = unwrap_quantized(q)
        kv = unwrap_quantized(kv)
        indices = indices.contiguous()
        q, kv = q.contiguous(), kv.contiguous()
        ctx.scaling = scaling
        if d_v is None:
            d_v = q.shape[-1]
        # the backward's inverse index depends on the indices alone: build it on a
        # second stream while the forward kernel runs (the forward is queued
        # first; the build waits only for the work before it)
        need_index = ctx.needs_input_grad[0] or ctx.needs_input_grad[1]
        ready = torch.cuda.Event() if need_index else None
        if ready is not None:
            ready.record()
        out, lse = sparse_mla_fwd_interface(q, kv, indices, sm_scale=scaling, d_v=d_v)
        ctx.inverse_index = (build_inverse_index(q, kv, indices, d_v, stream=side_stream(q.device), after=ready)
                             if need_index else None)
        ctx.d_v = d_v
        ctx.save_for_backward(q, kv, indices, out, lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_output, grad_lse):
        q, kv, indices, out, lse = ctx.saved_tensors
        dq, dkv = sparse_mla_bwd(q, kv, out, grad_output.contiguous(), indices, lse, sm_scale=ctx.scaling,
                                 inverse_index=ctx.inverse_index)
        ctx.inverse_index = None
        return dq, dkv, None, None, None


def _broadcast_scale(scale, t):
    lead = t.shape[:2] if t.ndim == 4 else t.shape[:1]
    return scale.reshape(-1)[:1].to(torch.float32).expand(*lead).contiguous()


class SparseMLA_FP8(torch.autograd.Function):
    """Sparse MLA with e4m3 (tensorwise) QK^T forward and backward, bf16 outputs."""

    @staticmethod
    def forward(ctx, q, kv, indices, scaling, d_v=None):
        _enforce_te_tensorwise_quant_backend()
        q8, q_te_scale = _extract_fp8_data(q)
        k8, kv_te_scale = _extract_fp8_data(kv)
        q_scale = kv_scale = None
        if q8 is not None:
            q8 = q8.contiguous()
            q_scale = _broadcast_scale(q_te_scale, q8)
        else:
            q = unwrap_quantized(q).contiguous()
        if k8 is not None:
            k8 = k8.contiguous()
            kv_scale = _broadcast_scale(kv_te_scale, k8)
        else:
            kv = unwrap_quantized(kv).contiguous()
        indices = indices.contiguous()
        ctx.scaling = scaling
        if d_v is None:
            d_v = (q8 if q8 is not None else q).shape[-1]

        if q8 is None:
            if q.dtype == torch.float8_e4m3fn:
                raise ValueError("SparseMLA_FP8.forward: q is raw float8_e4m3fn without scale. "
                                 "Pass BF16 or a Float8Tensor.")
            heads, dim_total = q.shape[-2], q.shape[-1]
            q8_flat, qs_flat = per_token_cast_to_fp8(q.reshape(-1, heads * dim_total))
            q8 = q8_flat.reshape(q.shape)
            q_scale = qs_flat.reshape(q.shape[:-2])
        if k8 is None:
            if kv.dtype == torch.float8_e4m3fn:
                raise ValueError("SparseMLA_FP8.forward: kv is raw float8_e4m3fn without scale. "
                                 "Pass BF16 or a Float8Tensor.")
            group, dim_total = kv.shape[-2], kv.shape[-1]
            k8_flat, ks_flat = per_token_cast_to_fp8(kv.reshape(-1, group * dim_total))
            k8 = k8_flat.reshape(kv.shape)
            kv_scale = ks_flat.reshape(kv.shape[:-2])

        need_index = ctx.needs_input_grad[0] or ctx.needs_input_grad[1]
        ready = torch.cuda.Event() if need_index else None
        if ready is not None:
            ready.record()
        out, lse = sparse_mla_fwd_fp8_interface(q8, k8, indices, q_scale=q_scale, kv_scale=kv_scale,
                                                sm_scale=scaling, d_v=d_v)
        ctx.inverse_index = (build_inverse_index(q8, k8, indices, d_v, stream=side_stream(q8.device), after=ready)
                             if need_index else None)
        ctx.d_v = d_v
        ctx.save_for_backward(q8, k8, q_scale, kv_scale, indices, out, lse)
        return out, lse

    @staticmethod
    def backward(ctx, grad_output, grad_lse):
        q8, k8, q_scale, kv_scale, indices, out, lse = ctx.saved_tensors
        dq, dkv = sparse_mla_bwd_fp8(q8, k8, q_scale, kv_scale, out, grad_output.contiguous(), indices, lse,
                                     sm_scale=ctx.scaling, inverse_index=ctx.inverse_index)
        ctx.inverse_index = None
        return dq, dkv, None, None, None


def _megatron_to_sparse(query, key, topk_indices):
    """[sq,b,np,hn] / [sk,b,np,hn] / [b,sq,topk] -> BSHD q, packed kv, int32 indices (-1 = invalid)."""
    sk = key.shape[0]
    q = query.permute(1, 0, 2, 3).contiguous()
    kv = key.permute(1, 0, 2, 3)[:, :, 0:1, :].contiguous()
    idx = topk_indices.to(torch.int32).unsqueeze(2)
    idx = torch.where((idx >= 0) & (idx < sk), idx, torch.full_like(idx, -1)).contiguous()
    return q, kv, idx


def sparse_mla_fp8_as_unfused_dsa(query, key, value, topk_indices, softmax_scale, **kwargs):
    """Megatron ``unfused_dsa_fn`` replacement through SparseMLA_FP8 -> [sq, b, np * hnv]."""
    sq, b, np_, _ = query.shape
    hnv = value.shape[3]
    q, kv, idx = _megatron_to_sparse(query, key, topk_indices)
    out, _ = SparseMLA_FP8.apply(q, kv, idx, softmax_scale, hnv)
    return out.permute(1, 0, 2, 3).contiguous().reshape(sq, b, np_ * hnv)


_sparse_mla_unfused_diag_logged = False


def sparse_mla_as_unfused_dsa(query, key, value, topk_indices, softmax_scale, **kwargs):
    """Megatron ``unfused_dsa_fn`` replacement through SparseMLA -> [sq, b, np * hnv].

    query [sq, b, np, hn], key [sk, b, np, hn] (the latent; heads share it),
    value [sk, b, np, hnv] (a prefix of key), topk_indices [b, sq, topk] int64.
    mask / varlen kwargs are ignored: masking travels in the -1 sentinel.
    """
    global _sparse_mla_unfused_diag_logged
    if not _sparse_mla_unfused_diag_logged:
        _sparse_mla_unfused_diag_logged = True
        log.info("[sparse_mla] ACTIVE (gfx950 HIP): query dtype=%s shape=%s key shape=%s",
                 query.dtype, tuple(query.shape), tuple(key.shape))
    sq, b, np_, _ = query.shape
    hnv = value.shape[3]
    q, kv, idx = _megatron_to_sparse(query, key, topk_indices)
    out, _ = SparseMLA.apply(q, kv, idx, softmax_scale, hnv)
    return out.permute(1, 0, 2, 3).contiguous().reshape(sq, b, np_ * hnv)


def fused_sparse_mla_absorbed_fp8(query, key, topk_indices, softmax_scale, v_channels):
    """Absorbed-MLA FP8 path: query [sq,b,np,d], key [skv,b,1,d], topk [b,sq,topk]
    -> [sq, b, np, v_channels], or None when the shapes are not supported."""
    if query.ndim != 4 or key.ndim != 4 or topk_indices.ndim != 3:
        return None
    if key.size(2) != 1:
        return None
    if query.size(1) != key.size(1) or topk_indices.size(0) != query.size(1):
        return None
    if topk_indices.size(1) != query.size(0):
        return None
    if query.size(-1) != key.size(-1):
        return None
    if topk_indices.size(-1) % 64 != 0:
        return None
    outs = []
    for bi in range(query.size(1)):
        q_t = query[:, bi].contiguous()
        kv_t = key[:, bi].contiguous()
        idx_t = topk_indices[bi].unsqueeze(1).to(torch.int32).contiguous()
        out, _ = SparseMLA_FP8.apply(q_t, kv_t, idx_t, softmax_scale, v_channels)
        if out.ndim != 3 or out.size(-1) != v_channels:
            return None
        outs.append(out)
    if not outs:
        return None
    return torch.stack(outs, dim=1).contiguous()


_PATCH_FLAG = "__cppmega_sparse_dsa_patched__"


def apply_sparse_mla_patch(fp8: bool | None = None, dsa_module=None) -> bool:
    """Route Megatron DSA sparse attention through these kernels.

    The reference does this inline in its launch shims
    (scripts/remote_smoke_h200_dsa_9_4_m.sh:346-373,
    scripts/cppmega_fp8_shim.py:3079-3085): ``dsa.unfused_dsa_fn`` becomes the
    bf16 or FP8 adapter (chosen by CPPMEGA_DSA_FP8_ATTENTION=1 unless ``fp8``
    is given) and ``dsa.SparseMLA`` becomes SparseMLA (or SparseMLA_FP8), which
    Megatron's ``_fused_sparse_mla_absorbed`` calls once per batch element.
    Returns False when the module has no ``unfused_dsa_fn`` to replace.
    """
    import os

    if dsa_module is None:
        from megatron.core.transformer.experimental_attention_variant import dsa as dsa_module
    if fp8 is None:
        fp8 = os.environ.get("CPPMEGA_DSA_FP8_ATTENTION", "0") == "1"
    existing = getattr(dsa_module, "unfused_dsa_fn", None)
    if existing is None:
        return False
    if not getattr(existing, _PATCH_FLAG, False):
        fn = sparse_mla_fp8_as_unfused_dsa if fp8 else sparse_mla_as_unfused_dsa
        setattr(fn, _PATCH_FLAG, True)
        dsa_module.unfused_dsa_fn = fn
    dsa_module.SparseMLA = SparseMLA_FP8 if fp8 else SparseMLA
    log.info("SparseMLA %s installed into %s", "FP8" if fp8 else "BF16", getattr(dsa_module, "__name__", "dsa"))
    return True
