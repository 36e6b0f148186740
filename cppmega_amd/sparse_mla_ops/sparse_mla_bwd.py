"""SparseMLA backward entry point (bf16), backed by the gfx950 HIP kernels.

Mirrors ``sparse_mla_bwd`` of
cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_bwd.py:422-531 (which
runs preprocess -> bwd -> postprocess).  Differences by design: dKV is reduced
deterministically (no float atomics), so two calls on the same inputs are
bitwise identical, and no shape bucketing is needed.  ``is_casual`` and
``return_kernel`` are accepted for signature compatibility: causality is
carried by the indices, and there is no JIT kernel object to return.
"""
from __future__ import annotations

import os

import torch

from .. import _lib
from ._common import check_same_device, normalize_sm_scale, stream_of, unwrap_quantized


def fp32_partials_default() -> bool:
    """CPPMEGA_AMD_BWD_FP32_PARTIALS=1 keeps the per-(token, slot) dKV rows in fp32
    (exact fp32 accumulation, 2x the workspace traffic); the default stores
    each row as fp16 scaled by a per-row power of two (11 significant bits,
    placed from a bound on the row's magnitudes: max|Q| sum|dS| + max|dO| sum P)
    before the deterministic fp32 reduction."""
    return os.getenv("CPPMEGA_AMD_BWD_FP32_PARTIALS", "0").strip().lower() in {"1", "true", "yes", "on"}


def _launch_bwd(q, kv, o, do, indices, lse, delta, sm_scale, dtype_code, q_scale=None, kv_scale=None,
                fp32_partials=None):
    B, S, H, D = q.shape
    _, S_kv, G, _ = kv.shape
    d_v = o.shape[-1]
    topk = indices.shape[-1]
    if fp32_partials is None:
        fp32_partials = fp32_partials_default()
    flags = _lib.BWD_FP32_PARTIALS if fp32_partials else 0
    L = _lib.load()
    ws_bytes = int(L.dsa_sparse_mla_bwd_workspace_size(B, S, S_kv, H, G, D, d_v, topk, flags))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    dq = torch.empty((B, S, H, D), dtype=torch.bfloat16, device=q.device)
    dkv = torch.empty((B, S_kv, G, D), dtype=torch.bfloat16, device=q.device)
    _, stream = stream_of(q)
    rc = L.dsa_sparse_mla_bwd(
        q.data_ptr(), kv.data_ptr(), o.data_ptr(), do.data_ptr(), indices.data_ptr(),
        lse.data_ptr(), _lib.ptr(delta), dq.data_ptr(), dkv.data_ptr(), ws.data_ptr(), ws_bytes,
        B, S, S_kv, H, G, D, d_v, topk, float(sm_scale), dtype_code,
        _lib.ptr(q_scale), _lib.ptr(kv_scale), flags, stream)
    _lib.check(rc, "dsa_sparse_mla_bwd")
    return dq, dkv


def _prep_delta(delta, B, S, H):
    if delta is None:
        return None
    if delta.ndim == 2:
        delta = delta.unsqueeze(0)
    assert delta.shape == (B, S, H), f"delta must be [B, S, H], got {tuple(delta.shape)}"
    return delta.to(torch.float32).contiguous()


def sparse_mla_bwd(q, kv, o, do, indices, lse, sm_scale=None, d_v=None, is_casual=True,
                   return_kernel=False, delta=None, *, fp32_partials=None):
    """Run the sparse-MLA backward and return (dq, dkv), both bf16.

    Accepts 3-D [seq, heads, dim] or 4-D [batch, seq, heads, dim] tensors;
    ``lse`` is the forward's log2-unit LSE.  grad of lse is not an input (the
    reference ignores it too).  ``fp32_partials`` (keyword only; default from
    CPPMEGA_AMD_BWD_FP32_PARTIALS) keeps the dKV contribution rows in fp32.
    """
    q = unwrap_quantized(q)
    kv = unwrap_quantized(kv)
    o = unwrap_quantized(o)
    do = unwrap_quantized(do)
    squeeze_batch = q.ndim == 3
    if squeeze_batch:
        q, kv, o, do = q.unsqueeze(0), kv.unsqueeze(0), o.unsqueeze(0), do.unsqueeze(0)
        indices, lse = indices.unsqueeze(0), lse.unsqueeze(0)

    assert q.is_contiguous()
    assert kv.is_contiguous()
    assert indices.is_contiguous()
    assert lse.is_contiguous()
    B, S, H, dim_plus_tail_dim = q.shape
    _, S_kv, kv_group, _ = kv.shape
    assert kv.shape[-1] == dim_plus_tail_dim
    assert kv.shape[0] == B
    D = o.shape[-1]
    if d_v is not None:
        assert int(d_v) == D, f"d_v={d_v} does not match o.shape[-1]={D}"
    assert dim_plus_tail_dim >= D, \
        f"Invalid dimensions: dim_plus_tail_dim={dim_plus_tail_dim} is smaller than base D={D}"
    topk = indices.shape[-1]
    assert indices.shape == (B, S, kv_group, topk)
    assert lse.shape == (B, S, H)
    assert o.shape == (B, S, H, D) and do.shape == (B, S, H, D)
    assert q.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16
    assert indices.dtype == torch.int32 and lse.dtype == torch.float32
    check_same_device(q, kv, o, do, indices, lse)
    o = o.to(torch.bfloat16).contiguous()
    do = do.to(torch.bfloat16).contiguous()
    delta = _prep_delta(delta, B, S, H)

    scale = normalize_sm_scale(sm_scale, dim_plus_tail_dim)
    dq, dkv = _launch_bwd(q, kv, o, do, indices, lse, delta, scale, _lib.DTYPE_BF16,
                          fp32_partials=fp32_partials)
    if squeeze_batch:
        dq, dkv = dq.squeeze(0), dkv.squeeze(0)
    return dq, dkv
