"""SparseMLA forward entry point (bf16), backed by the gfx950 HIP kernel.

Mirrors ``sparse_mla_fwd_interface`` of
cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd.py:293-391: same
arguments, same 3-D / 4-D handling, same assertions.  The kernel takes any
sequence length and top-k directly, so the reference's shape bucketing
(padding to multiples of 256 / block_I) is not needed; results are identical
because padded slots carry the -1 sentinel there.  ``block_I``,
``num_stages`` and ``threads`` are TileLang tuning knobs, accepted for
signature compatibility and ignored.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import check_same_device, normalize_sm_scale, stream_of, unwrap_quantized


def _launch_fwd(q, kv, indices, sm_scale, d_v, dtype_code, q_scale=None, kv_scale=None):
    """q [B,S,H,D], kv [B,Skv,G,D], indices [B,S,G,topk] (all contiguous) -> (out, lse2)."""
    B, S, H, D = q.shape
    _, S_kv, G, _ = kv.shape
    topk = indices.shape[-1]
    out = torch.empty((B, S, H, d_v), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=q.device)
    _, stream = stream_of(q)
    L = _lib.load()
    # e4m3: the V rows are dequantised to bf16 once per call into a workspace
    ws_bytes = int(L.dsa_sparse_mla_fwd_workspace_size(B, S_kv, G, D, d_v, dtype_code))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device) if ws_bytes else None
    rc = L.dsa_sparse_mla_fwd_ws(
        q.data_ptr(), kv.data_ptr(), indices.data_ptr(), out.data_ptr(), lse.data_ptr(),
        B, S, S_kv, H, G, D, d_v, topk, float(sm_scale), dtype_code,
        _lib.ptr(q_scale), _lib.ptr(kv_scale), _lib.ptr(ws), ws_bytes, stream)
    _lib.check(rc, "dsa_sparse_mla_fwd_ws")
    return out, lse


def sparse_mla_fwd_interface(
    q,
    kv,
    indices,
    sm_scale=None,
    return_p_sum: bool = False,
    d_v=512,
    block_I=64,
    num_stages=2,
    threads=256,
):
    """Run the sparse-MLA forward kernel and return (out, lse2).

    q [batch, seq, heads, dim+tail] (or 3-D without batch), kv
    [batch, seq_kv, kv_group, dim+tail], indices [batch, seq, kv_group, topk]
    int32 with -1 (or any out-of-range value) masking a slot.  out is bf16
    [batch, seq, heads, d_v]; lse2 is fp32 [batch, seq, heads] in log2 units.
    """
    q = unwrap_quantized(q)
    kv = unwrap_quantized(kv)
    squeeze_batch = q.ndim == 3
    if squeeze_batch:
        q = q.unsqueeze(0)
        kv = kv.unsqueeze(0)
        indices = indices.unsqueeze(0)

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
    assert heads % kv_group == 0, f"heads={heads} must be a multiple of kv_group={kv_group}"
    assert q.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16, \
        f"bf16 q/kv required (got {q.dtype}, {kv.dtype}); use sparse_mla_fwd_fp8_interface for fp8"
    assert indices.dtype == torch.int32, f"indices must be int32, got {indices.dtype}"
    check_same_device(q, kv, indices)

    scale = normalize_sm_scale(sm_scale, dim_plus_tail_dim)
    out, lse = _launch_fwd(q, kv, indices, scale, dim, _lib.DTYPE_BF16)
    if squeeze_batch:
        out = out.squeeze(0)
        lse = lse.squeeze(0)
    return out, lse
