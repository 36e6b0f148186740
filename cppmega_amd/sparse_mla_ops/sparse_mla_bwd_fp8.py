"""FP8 (OCP e4m3, tensorwise scale) SparseMLA backward.

Mirrors ``sparse_mla_bwd_fp8`` of
cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd_fp8.py:492-630:
QK^T is recomputed on e4m3 codes times q_scale * kv_scale, the dP / dQ / dKV
GEMMs use bf16-dequantised Q and KV, and dq / dkv are bf16 gradients with
respect to the dequantised values.  dKV is reduced deterministically.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check_same_device, normalize_sm_scale
from .sparse_mla_bwd import _launch_bwd, _prep_delta


def sparse_mla_bwd_fp8(q, kv, q_scale, kv_scale, o, do, indices, lse, sm_scale=None, is_casual=True,
                       return_kernel=False, delta=None, *, inverse_index=None, pass_bytes=None):
    """Return (dq, dkv) bf16 for e4m3 q [B,S,H,D] / kv [B,S_kv,G,D] with scales [B,S] / [B,S_kv].
    ``inverse_index`` and ``pass_bytes``: as for ``sparse_mla_bwd``."""
    squeeze_batch = q.ndim == 3
    if squeeze_batch:
        q, kv, o, do = q.unsqueeze(0), kv.unsqueeze(0), o.unsqueeze(0), do.unsqueeze(0)
        q_scale, kv_scale = q_scale.unsqueeze(0), kv_scale.unsqueeze(0)
        indices, lse = indices.unsqueeze(0), lse.unsqueeze(0)

    assert q.is_contiguous()
    assert kv.is_contiguous()
    assert q_scale.is_contiguous()
    assert kv_scale.is_contiguous()
    assert indices.is_contiguous()
    assert lse.is_contiguous()
    B, S, H, dim_plus_tail_dim = q.shape
    _, S_kv, kv_group, _ = kv.shape
    assert kv.shape[-1] == dim_plus_tail_dim
    assert kv.shape[0] == B
    D = o.shape[-1]
    assert dim_plus_tail_dim >= D, \
        f"Invalid dimensions: dim_plus_tail_dim={dim_plus_tail_dim} is smaller than base D={D}"
    topk = indices.shape[-1]
    assert indices.shape == (B, S, kv_group, topk)
    assert lse.shape == (B, S, H)
    assert q_scale.shape == (B, S)
    assert kv_scale.shape == (B, S_kv)
    assert q.dtype == torch.float8_e4m3fn and kv.dtype == torch.float8_e4m3fn
    check_same_device(q, kv, q_scale, kv_scale, o, do, indices, lse)
    o = o.to(torch.bfloat16).contiguous()
    do = do.to(torch.bfloat16).contiguous()
    delta = _prep_delta(delta, B, S, H)
    scale = normalize_sm_scale(sm_scale, dim_plus_tail_dim)
    dq, dkv = _launch_bwd(q, kv, o, do, indices, lse, delta, scale, _lib.DTYPE_E4M3,
                          q_scale.to(torch.float32).contiguous(), kv_scale.to(torch.float32).contiguous(),
                          inverse_index=inverse_index, pass_bytes=pass_bytes)
    if squeeze_batch:
        dq, dkv = dq.squeeze(0), dkv.squeeze(0)
    return dq, dkv
