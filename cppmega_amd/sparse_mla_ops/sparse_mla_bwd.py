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


class InverseIndex:
    """The backward's inverse index (kv row -> entries in order), built from the
    indices alone by ``build_inverse_index`` ahead of the backward -- e.g. on a
    second stream while the forward runs -- and consumed by ``sparse_mla_bwd``
    / ``sparse_mla_bwd_fp8`` (``inverse_index=``), which then run only the main
    kernel and the dKV reduction.  Holds the index buffer, the event that ends
    its build (None when built on the caller's stream) and the call shape it
    was built for; the indices must not change in between."""

    __slots__ = ("buf", "event", "key")

    def __init__(self, buf, event, key):
        self.buf, self.event, self.key = buf, event, key


_SIDE_STREAMS: dict = {}


def side_stream(device) -> torch.cuda.Stream:
    """A second stream of ``device`` (default priority) for work that overlaps the
    current stream, e.g. ``build_inverse_index`` during the forward."""
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    s = _SIDE_STREAMS.get(idx)
    if s is None:
        s = _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return s


def _bwd_flags(fp32_partials):
    if fp32_partials is None:
        fp32_partials = fp32_partials_default()
    return _lib.BWD_FP32_PARTIALS if fp32_partials else 0


def _pass_bytes(pass_bytes):
    """The C-ABI's per-pass cap on the partial dKV rows: 0 selects its default (4 GiB); caps are
    lowered to at most 4 GiB - 1 MiB."""
    if pass_bytes is None:
        return 0
    pass_bytes = int(pass_bytes)
    if pass_bytes < 0:
        raise ValueError(f"pass_bytes must be >= 0, got {pass_bytes}")
    return pass_bytes


def build_inverse_index(q, kv, indices, d_v, *, fp32_partials=None, stream=None, after=None, pass_bytes=None):
    """Build the backward's inverse index for q [B,S,H,D] (or 3-D), kv
    [B,S_kv,G,D] and indices [B,S,G,topk] int32; returns an ``InverseIndex``,
    or None when the backward runs in several passes (it then builds its index
    per pass; ``pass_bytes`` is the per-pass cap, as for ``sparse_mla_bwd``).  With ``stream`` (e.g. ``side_stream(q.device)``) the build runs
    there after the work already queued on the current stream (or, with
    ``after``, a ``torch.cuda.Event`` recorded on it, after the work up to
    that event: work queued since, such as the forward kernel, does not delay
    the build), and the backward waits for it through an event."""
    if q.ndim == 3:
        q, kv, indices = q.unsqueeze(0), kv.unsqueeze(0), indices.unsqueeze(0)
    assert indices.is_contiguous() and indices.dtype == torch.int32
    B, S, H, D = q.shape
    _, S_kv, G, _ = kv.shape
    topk = indices.shape[-1]
    flags = _bwd_flags(fp32_partials)
    cap = _pass_bytes(pass_bytes)
    L = _lib.load()
    n = int(L.dsa_sparse_mla_bwd_index_size(B, S, S_kv, H, G, D, int(d_v), topk, flags, cap))
    if n == 0:
        return None
    cur = torch.cuda.current_stream(q.device)
    side = stream if stream is not None else cur
    buf = torch.empty(n, dtype=torch.uint8, device=q.device)
    if side != cur:
        if after is not None:
            side.wait_event(after)
        else:
            side.wait_stream(cur)
    rc = L.dsa_sparse_mla_bwd_build_index(indices.data_ptr(), B, S, S_kv, H, G, D, int(d_v), topk, flags, cap,
                                          buf.data_ptr(), n, side.cuda_stream)
    _lib.check(rc, "dsa_sparse_mla_bwd_build_index")
    event = None
    if side != cur:
        if not torch.cuda.is_current_stream_capturing():  # a capture keeps its pool alive itself
            buf.record_stream(side)
            indices.record_stream(side)
        event = torch.cuda.Event()
        event.record(side)
    return InverseIndex(buf, event, (B, S, S_kv, H, G, D, int(d_v), topk, flags, cap, indices.data_ptr()))


def _launch_bwd(q, kv, o, do, indices, lse, delta, sm_scale, dtype_code, q_scale=None, kv_scale=None,
                fp32_partials=None, inverse_index=None, pass_bytes=None):
    B, S, H, D = q.shape
    _, S_kv, G, _ = kv.shape
    d_v = o.shape[-1]
    topk = indices.shape[-1]
    flags = _bwd_flags(fp32_partials)
    cap = _pass_bytes(pass_bytes)
    L = _lib.load()
    dq = torch.empty((B, S, H, D), dtype=torch.bfloat16, device=q.device)
    dkv = torch.empty((B, S_kv, G, D), dtype=torch.bfloat16, device=q.device)
    _, stream = stream_of(q)
    if inverse_index is not None:
        key = (B, S, S_kv, H, G, D, d_v, topk, flags, cap, indices.data_ptr())
        if inverse_index.key != key:
            raise ValueError(f"inverse_index was built for another call: built for {inverse_index.key}, "
                             f"called with {key} (B, S, S_kv, H, G, D, d_v, topk, flags, pass_bytes, indices)")
        if inverse_index.event is not None:
            torch.cuda.current_stream(q.device).wait_event(inverse_index.event)
        ws_bytes = int(L.dsa_sparse_mla_bwd_indexed_workspace_size(B, S, S_kv, H, G, D, d_v, topk, flags, cap))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        ix = inverse_index.buf
        rc = L.dsa_sparse_mla_bwd_indexed(
            q.data_ptr(), kv.data_ptr(), o.data_ptr(), do.data_ptr(), indices.data_ptr(),
            lse.data_ptr(), _lib.ptr(delta), dq.data_ptr(), dkv.data_ptr(), ix.data_ptr(), ix.numel(),
            ws.data_ptr(), ws_bytes, B, S, S_kv, H, G, D, d_v, topk, float(sm_scale), dtype_code,
            _lib.ptr(q_scale), _lib.ptr(kv_scale), flags, cap, stream)
        _lib.check(rc, "dsa_sparse_mla_bwd_indexed")
        return dq, dkv
    ws_bytes = int(L.dsa_sparse_mla_bwd_workspace_size(B, S, S_kv, H, G, D, d_v, topk, flags, cap))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    rc = L.dsa_sparse_mla_bwd(
        q.data_ptr(), kv.data_ptr(), o.data_ptr(), do.data_ptr(), indices.data_ptr(),
        lse.data_ptr(), _lib.ptr(delta), dq.data_ptr(), dkv.data_ptr(), ws.data_ptr(), ws_bytes,
        B, S, S_kv, H, G, D, d_v, topk, float(sm_scale), dtype_code,
        _lib.ptr(q_scale), _lib.ptr(kv_scale), flags, cap, stream)
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
                   return_kernel=False, delta=None, *, fp32_partials=None, inverse_index=None, pass_bytes=None):
    """Run the sparse-MLA backward and return (dq, dkv), both bf16.

    Accepts 3-D [seq, heads, dim] or 4-D [batch, seq, heads, dim] tensors;
    ``lse`` is the forward's log2-unit LSE.  grad of lse is not an input (the
    reference ignores it too).  ``fp32_partials`` (keyword only; default from
    CPPMEGA_AMD_BWD_FP32_PARTIALS) keeps the dKV contribution rows in fp32.
    ``inverse_index`` (keyword only): an ``InverseIndex`` from
    ``build_inverse_index`` for these indices, built ahead of the call.
    ``pass_bytes`` (keyword only): the per-pass cap on the partial dKV rows
    (bytes; None or 0 = 4 GiB); the backward runs in passes over token ranges
    whose rows fit it, so its workspace stays bounded.
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
                          fp32_partials=fp32_partials, inverse_index=inverse_index, pass_bytes=pass_bytes)
    if squeeze_batch:
        dq, dkv = dq.squeeze(0), dkv.squeeze(0)
    return dq, dkv
