"""Deterministic top-k over indexer scores, and the fused indexer + top-k entry.

``topk_indices`` replaces the top-k inside Megatron's ``fused_qk_topk_naive``
(``index_scores.topk(min(topk, seqlen), dim=-1)[1]``, restated in
scripts/modal_dsa_indexer_bench.py:188-194) with a deterministic contract:
candidates of a row are columns [start, end), the min(topk, end - start)
largest scores are chosen, equal scores prefer the lower column, NaN ranks as
+inf, -0.0 equals +0.0, and the chosen columns come back ascending, int32,
padded with -1.  ``fused_qk_topk_naive`` keeps Megatron's signature and return
convention (scores, indices) on top of it.
"""
from __future__ import annotations

import torch

from . import _lib
from .dsa_indexer_fused_patch import CAUSAL_LOWER, CAUSAL_NEG_INF, CAUSAL_NONE, index_scores


def topk_indices(scores, topk, causal=True, starts=None, ends=None, causal_offset=0, seq_q=None):
    """scores [..., sq, sk] f32 -> [..., sq, topk] int32 (ascending, -1 padded).

    causal=True uses the window [0, min(sk, t + 1 + causal_offset)) for row t of
    each [sq, sk] matrix; starts / ends (int32, one per row) override it.
    """
    assert scores.dtype == torch.float32, f"scores must be fp32, got {scores.dtype}"
    assert topk > 0
    if scores.stride(-1) != 1:
        scores = scores.contiguous()
    sk = scores.shape[-1]
    sq = scores.shape[-2] if scores.dim() >= 2 else 1
    lead = scores.shape[:-1]
    rows = 1
    for s in lead:
        rows *= int(s)
    flat = scores.reshape(rows, sk) if scores.is_contiguous() else scores.contiguous().reshape(rows, sk)
    out = torch.empty((*lead, topk), dtype=torch.int32, device=scores.device)
    if starts is not None or ends is not None:
        assert starts is not None and ends is not None, "give both starts and ends"
        starts = starts.to(torch.int32).reshape(rows).contiguous()
        ends = ends.to(torch.int32).reshape(rows).contiguous()
    dev = _lib.ensure_device(scores)
    rc = _lib.load().dsa_topk(
        flat.data_ptr(), rows, sk, flat.stride(0), int(seq_q or sq), 1 if causal else 0, int(causal_offset),
        _lib.ptr(starts), _lib.ptr(ends), int(topk), out.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_topk")
    return out


def indexer_topk(q, k, weights, index_topk, use_relu=True, causal=True, q_scale=None, k_scale=None,
                 return_scores=False):
    """Fused hot path: causal indexer scores (lower triangle only) + deterministic top-k.

    q [sq,b,h,d], k [sk,b,d], weights [sq,b,h] -> indices [b, sq, index_topk] int32.
    """
    mode = CAUSAL_LOWER if causal else CAUSAL_NONE
    scores = index_scores(q, weights, k, use_relu=use_relu, causal=mode, q_scale=q_scale, k_scale=k_scale)
    idx = topk_indices(scores, index_topk, causal=causal)
    return (scores, idx) if return_scores else idx


def fused_qk_topk_naive(q, k, weights, index_topk, mask=None, varlen_starts=None, varlen_ends=None,
                        key_positions=None, use_relu=True):
    """Megatron-compatible (scores [b,sq,sk] f32, topk_indices [b,sq,topk] int64).

    mask=None scores every key (no causal window), as Megatron does; a float
    additive mask [sq, sk] (0 / -inf) restricts each row to its finite entries,
    which must form one contiguous window per row (causal or sliding); varlen
    starts / ends give the windows directly.  Rows with fewer candidates than
    topk are padded with -1.
    """
    if key_positions is not None:
        raise NotImplementedError("key_positions remapping is not supported by the gfx950 top-k")
    scores = index_scores(q, weights, k, use_relu=use_relu, causal=CAUSAL_NONE)
    b, sq, sk = scores.shape
    if varlen_starts is not None or varlen_ends is not None:
        starts = varlen_starts.to(torch.int32).expand(b, sq).contiguous()
        ends = varlen_ends.to(torch.int32).expand(b, sq).contiguous()
        idx = topk_indices(scores, index_topk, causal=False, starts=starts, ends=ends)
    elif mask is not None:
        finite = torch.isfinite(mask.float()).reshape(-1, sq, sk)
        cols = torch.arange(sk, device=scores.device)
        has = finite.any(-1)
        first = torch.where(has, torch.where(finite, cols, sk).amin(-1), torch.zeros_like(cols[:1]))
        last = torch.where(has, torch.where(finite, cols, -1).amax(-1) + 1, torch.zeros_like(cols[:1]))
        span_ok = (finite.sum(-1) == (last - first)).all()
        if not bool(span_ok):
            raise ValueError("mask rows must be contiguous windows of finite entries")
        idx = topk_indices(scores, index_topk, causal=False,
                           starts=first.expand(b, sq).contiguous(), ends=last.expand(b, sq).contiguous())
    else:
        idx = topk_indices(scores, index_topk, causal=False)
    return scores, idx.to(torch.int64)


__all__ = ["CAUSAL_LOWER", "CAUSAL_NEG_INF", "CAUSAL_NONE", "fused_qk_topk_naive", "indexer_topk",
           "topk_indices"]
