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
from .dsa_indexer_fused_patch import (CAUSAL_LOWER, CAUSAL_NEG_INF, CAUSAL_NONE, CAUSAL_WINDOW, IndexScores,
                                      index_scores)


def _scores(q, weights, k, use_relu, causal, starts=None, ends=None, mask=None, row_plain=None):
    """index_scores, through the differentiable IndexScores when grad mode is on
    and q, weights or k requires grad (the scores Megatron's loss consumes)."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, weights, k)):
        return IndexScores.apply(q, weights, k, use_relu, causal, starts, ends, mask, row_plain)
    return index_scores(q, weights, k, use_relu=use_relu, causal=causal, starts=starts, ends=ends, mask=mask,
                        row_plain=row_plain)


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
    lib = _lib.load()
    # rows over 32768 columns run in segment passes through a workspace
    ws_bytes = int(lib.dsa_topk_workspace_size(rows, sk, int(topk)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=scores.device) if ws_bytes else None
    rc = lib.dsa_topk_ws(
        flat.data_ptr(), rows, sk, flat.stride(0), int(seq_q or sq), 1 if causal else 0, int(causal_offset),
        _lib.ptr(starts), _lib.ptr(ends), int(topk), out.data_ptr(), _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev))
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


def _row_windows(x, b, sq, what):
    """A per-row int tensor ([sq], [b, sq] or [b * sq]) as int32 [b, sq]."""
    x = x.to(torch.int32)
    if x.numel() == sq:
        return x.reshape(1, sq).expand(b, sq)
    if x.numel() == b * sq:
        return x.reshape(b, sq)
    raise ValueError(f"{what} has {x.numel()} entries; expected {sq} or {b * sq} (one per query row)")


def mask_windows(mask, b, sq, sk):
    """Candidate windows of an additive mask broadcastable to [b, sq, sk]:
    (starts, ends, plain), int32 [b, sq] each -- the first finite column of
    every row, one past its last ((0, 0) for a row without one), and 1 where
    every entry in between is +0.0 (no finite bias, no -inf hole).  One kernel
    (dsa_mask_windows) reads the mask once; no host synchronisation."""
    m = mask.to(dtype=torch.float32).reshape(-1, sq, sk)
    if m.shape[0] not in (1, b):
        raise ValueError(f"mask {tuple(mask.shape)} does not broadcast to {(b, sq, sk)}")
    m = m.contiguous()
    starts = torch.empty((b, sq), dtype=torch.int32, device=m.device)
    ends = torch.empty_like(starts)
    plain = torch.empty_like(starts)
    dev = _lib.ensure_device(m)
    rc = _lib.load().dsa_mask_windows(m.data_ptr(), m.shape[0], b, sq, sk, starts.data_ptr(), ends.data_ptr(),
                                      plain.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_mask_windows")
    return starts, ends, plain


def finalize_picks(scores, idx, plain=None):
    """idx [b, sq, k] int32 (ascending, -1 padded) -> int64, with the picks whose
    score in ``scores`` [b, sq, sk] is -inf (holes inside a window that held
    fewer finite columns than k) turned into -1 and the rest kept ascending,
    on every row not flagged in ``plain`` (int32 [b, sq]; None: every row is
    checked).  One kernel (dsa_topk_finalize)."""
    assert scores.dtype == torch.float32 and scores.is_contiguous() and idx.dtype == torch.int32
    sk = scores.shape[-1]
    rows = idx.numel() // idx.shape[-1]
    idx = idx.contiguous()
    out = torch.empty(idx.shape, dtype=torch.int64, device=idx.device)
    if plain is not None:
        plain = plain.to(torch.int32).expand(*idx.shape[:-1]).contiguous()
    dev = _lib.ensure_device(idx)
    rc = _lib.load().dsa_topk_finalize(scores.data_ptr(), sk, idx.data_ptr(), rows, idx.shape[-1], _lib.ptr(plain),
                                       out.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_topk_finalize")
    return out


def indexer_topk_streaming(q, k, weights, index_topk, use_relu=True, causal=True, q_scale=None, k_scale=None,
                           return_scores=False, max_scratch_bytes=64 << 20, chunk_rows=None):
    """Indexer scores + deterministic top-k without the [b, sq, sk] score matrix:
    q [sq,b,h,d] (bf16 or e4m3), k [sk,b,d], weights [sq,b,h] -> indices
    [b, sq, index_topk] int32 (ascending, -1 padded), and with
    ``return_scores`` also the selected scores [b, sq, index_topk] f32 (-inf
    on padding).  Query rows go through a scratch of at most
    ``max_scratch_bytes`` (or ``chunk_rows`` rows) in chunks; the indices are
    bit-identical to ``topk_indices`` over the full scores.  With
    ``max_scratch_bytes=0`` (and no ``chunk_rows``) no scratch is used at all:
    the top-k runs folded into the score tiles (``indexer_topk_fused``), for
    index_topk up to ``indexer_topk_fused_max_topk(h, d)``.  The reference's
    stated target for its indexer (docs/status/cppmega_architecture_status.md:340-362)."""
    assert q.dim() == 4 and k.dim() == 3 and weights.dim() == 3
    sq, b, h, d = q.shape
    sk = k.shape[0]
    fp8 = q.dtype == torch.float8_e4m3fn
    if fp8:
        assert k.dtype == torch.float8_e4m3fn and q_scale is not None and k_scale is not None, \
            "e4m3 indexer inputs need q_scale and k_scale"
        q_scale = q_scale.reshape(-1)[:1].to(torch.float32).contiguous()
        k_scale = k_scale.reshape(-1)[:1].to(torch.float32).contiguous()
    elif q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise TypeError(f"indexer q/k must be bf16 or float8_e4m3fn, got {q.dtype}/{k.dtype}")
    if weights.dtype not in (torch.float32, torch.bfloat16):
        weights = weights.float()
    q, k, weights = q.contiguous(), k.contiguous(), weights.contiguous()
    if chunk_rows is None and int(max_scratch_bytes) == 0:
        if int(index_topk) > indexer_topk_fused_max_topk(h, d):
            raise ValueError(f"no scratch: index_topk {index_topk} exceeds the fused path's "
                             f"{indexer_topk_fused_max_topk(h, d)} for h={h}, d={d}")
        return indexer_topk_fused(q, k, weights, index_topk, use_relu=use_relu, causal=causal, q_scale=q_scale,
                                  k_scale=k_scale, return_scores=return_scores)
    if chunk_rows is None:
        chunk_rows = max(1, int(max_scratch_bytes) // max(1, b * sk * 4))
    lib = _lib.load()
    ws_bytes = int(lib.dsa_indexer_topk_streaming_workspace_size(b, sq, sk, int(chunk_rows)))
    # rows over 32768 keys: room for the top-k's segment passes of a chunk too
    ws_bytes += 256 + int(lib.dsa_topk_workspace_size(b * min(int(chunk_rows), sq), sk, int(index_topk)))
    dev = _lib.ensure_device(q)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    idx = torch.empty((b, sq, int(index_topk)), dtype=torch.int32, device=q.device)
    vals = torch.empty((b, sq, int(index_topk)), dtype=torch.float32, device=q.device) if return_scores else None
    rc = lib.dsa_indexer_topk_streaming(
        q.data_ptr(), weights.data_ptr(), k.data_ptr(), idx.data_ptr(), _lib.ptr(vals), b, sq, sk, h, d,
        _lib.DTYPE_E4M3 if fp8 else _lib.DTYPE_BF16,
        _lib.DTYPE_F32 if weights.dtype == torch.float32 else _lib.DTYPE_BF16,
        _lib.ptr(q_scale), _lib.ptr(k_scale), int(index_topk), 1 if causal else 0, 1 if use_relu else 0,
        ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_indexer_topk_streaming")
    return (idx, vals) if return_scores else idx


def indexer_topk_fused_max_topk(heads, head_dim):
    """Largest index_topk ``indexer_topk_fused`` takes for this indexer shape (0: none)."""
    return int(_lib.load().dsa_indexer_topk_fused_max_topk(int(heads), int(head_dim)))


def indexer_topk_fused(q, k, weights, index_topk, use_relu=True, causal=True, q_scale=None, k_scale=None,
                       return_scores=False):
    """``indexer_topk_streaming``'s result with the top-k folded into the
    indexer: no score matrix, no scratch.  Each query row keeps a bounded
    candidate list on chip while its keys are scored; the indices (and
    scores) are bit-identical to ``topk_indices`` over the full scores.
    index_topk must not exceed ``indexer_topk_fused_max_topk(h, d)``."""
    assert q.dim() == 4 and k.dim() == 3 and weights.dim() == 3
    sq, b, h, d = q.shape
    sk = k.shape[0]
    fp8 = q.dtype == torch.float8_e4m3fn
    if fp8:
        assert k.dtype == torch.float8_e4m3fn and q_scale is not None and k_scale is not None, \
            "e4m3 indexer inputs need q_scale and k_scale"
        q_scale = q_scale.reshape(-1)[:1].to(torch.float32).contiguous()
        k_scale = k_scale.reshape(-1)[:1].to(torch.float32).contiguous()
    elif q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise TypeError(f"indexer q/k must be bf16 or float8_e4m3fn, got {q.dtype}/{k.dtype}")
    if weights.dtype not in (torch.float32, torch.bfloat16):
        weights = weights.float()
    q, k, weights = q.contiguous(), k.contiguous(), weights.contiguous()
    lib = _lib.load()
    dev = _lib.ensure_device(q)
    idx = torch.empty((b, sq, int(index_topk)), dtype=torch.int32, device=q.device)
    vals = torch.empty((b, sq, int(index_topk)), dtype=torch.float32, device=q.device) if return_scores else None
    rc = lib.dsa_indexer_topk_fused(
        q.data_ptr(), weights.data_ptr(), k.data_ptr(), idx.data_ptr(), _lib.ptr(vals), b, sq, sk, h, d,
        _lib.DTYPE_E4M3 if fp8 else _lib.DTYPE_BF16,
        _lib.DTYPE_F32 if weights.dtype == torch.float32 else _lib.DTYPE_BF16,
        _lib.ptr(q_scale), _lib.ptr(k_scale), int(index_topk), 1 if causal else 0, 1 if use_relu else 0,
        _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_indexer_topk_fused")
    return (idx, vals) if return_scores else idx


def fused_qk_topk_naive(q, k, weights, index_topk, mask=None, varlen_starts=None, varlen_ends=None,
                        key_positions=None, use_relu=True):
    """Megatron ``fused_qk_topk_naive`` on gfx950 -> (scores [b,sq,sk] f32, indices [b,sq,k] int64).

    k = min(index_topk, sq), the reference's ``min(index_topk, seqlen)`` with
    seqlen = q.size(0) (scripts/modal_dsa_indexer_bench.py:188-194); the call
    shapes are Megatron's (cppmega/megatron/lemyx_dsa_warmup.py:169-176,
    index_cache_patch.py:148-153).

    * mask=None, no varlen: every key is a candidate; scores are the unmasked
      indexer scores.
    * mask: an additive float mask broadcastable to [b, sq, sk] (0 / -inf, or
      any finite bias): the scores returned are ``index_scores + mask``; the
      candidates of a row are its finite-mask columns.
    * varlen_starts / varlen_ends (one per query row): the candidates of row t
      are the keys whose position lies in [start_t, end_t); a key's position
      is its column, or key_positions[s] (shape [sk] or [b, sk]) when given.
      Scores outside are -inf.

    Selection is deterministic (ties to the lower column), the chosen columns
    ascend, and a row with fewer candidates than k is padded with -1.  Key
    tiles outside every row window of a query block are not computed, so a
    causal mask costs the lower-triangle work.  Everything runs on the device:
    no host synchronisation, so the call can be captured in a graph.
    Parity unpinned against Megatron's own masking (not vendored): the
    candidate sets above are this build's contract.
    """
    sq, b = int(q.shape[0]), int(q.shape[1])
    sk = int(k.shape[0])
    topk_k = min(int(index_topk), sq)
    varlen = varlen_starts is not None or varlen_ends is not None
    if mask is None and not varlen:
        scores = _scores(q, weights, k, use_relu, CAUSAL_NONE)
        return scores, topk_indices(scores.detach(), topk_k, causal=False).to(torch.int64)
    dev = q.device
    add = None if mask is None else mask.to(device=dev, dtype=torch.float32)
    if varlen:
        assert varlen_starts is not None and varlen_ends is not None, "give both varlen_starts and varlen_ends"
        vs = _row_windows(varlen_starts.to(dev), b, sq, "varlen_starts")
        ve = _row_windows(varlen_ends.to(dev), b, sq, "varlen_ends")
    if add is not None:
        add = add.reshape(-1, sq, sk)                                                # [1 or b, sq, sk]
    plain = None
    if varlen and key_positions is not None:
        # a key's position need not be its column: the windows become an additive mask
        kp = key_positions.to(device=dev, dtype=torch.int64).reshape(-1, 1, sk)    # [1 or b, 1, sk]
        ok = (kp >= vs.unsqueeze(-1)) & (kp < ve.unsqueeze(-1))                    # [b, sq, sk]
        kmask = torch.zeros(ok.shape, dtype=torch.float32, device=dev).masked_fill_(~ok, float("-inf"))
        add = kmask if add is None else add + kmask
        starts, ends, plain = mask_windows(add, b, sq, sk)
    elif add is not None:
        starts, ends, plain = mask_windows(add, b, sq, sk)
        if varlen:  # a narrower window of a plain row is still plain
            starts, ends = torch.maximum(starts, vs).contiguous(), torch.minimum(ends, ve).contiguous()
    else:
        starts, ends = vs.contiguous(), ve.contiguous()
    scores = _scores(q, weights, k, use_relu, CAUSAL_WINDOW, starts, ends, add, plain)
    idx = topk_indices(scores.detach(), topk_k, causal=False, starts=starts, ends=ends)
    if add is None:  # raw scores inside the windows: no -inf pick
        return scores, idx.to(torch.int64)
    return scores, finalize_picks(scores.detach(), idx, plain)


_TOPK_MARKER = "__cppmega_amd_dsa_topk_patched__"


def apply_dsa_topk_patch(*, force: bool = False, dsa_module=None) -> bool:
    """Install this module's ``fused_qk_topk_naive`` as Megatron's
    ``dsa.fused_qk_topk_naive`` (what DSAttention, the fused indexer loss and
    IndexCache call: cppmega/megatron/lemyx_dsa_warmup.py:169-176,
    index_cache_patch.py:148-153).  Idempotent; raises when the attribute is
    absent (Megatron version mismatch)."""
    if dsa_module is None:
        from megatron.core.transformer.experimental_attention_variant import dsa as dsa_module
    existing = getattr(dsa_module, "fused_qk_topk_naive", None)
    if existing is None:
        raise RuntimeError("dsa.fused_qk_topk_naive not found - Megatron version mismatch?")
    if getattr(existing, _TOPK_MARKER, False) and not force:
        return True

    def _fused_qk_topk_gfx950(q, k, weights, index_topk, mask=None, varlen_starts=None, varlen_ends=None,
                              key_positions=None, use_relu=True, **kwargs):
        return fused_qk_topk_naive(q, k, weights, index_topk, mask=mask, varlen_starts=varlen_starts,
                                   varlen_ends=varlen_ends, key_positions=key_positions, use_relu=use_relu)

    setattr(_fused_qk_topk_gfx950, _TOPK_MARKER, True)
    dsa_module.fused_qk_topk_naive = _fused_qk_topk_gfx950
    return True


__all__ = ["CAUSAL_LOWER", "CAUSAL_NEG_INF", "CAUSAL_NONE", "CAUSAL_WINDOW", "apply_dsa_topk_patch",
           "finalize_picks", "fused_qk_topk_naive", "indexer_topk", "indexer_topk_streaming", "mask_windows",
           "topk_indices"]
