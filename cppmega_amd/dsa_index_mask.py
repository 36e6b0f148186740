"""Top-k index mask of the DSA sparse indexer loss on gfx950.

Drop-in for Megatron's ``_scatter_topk_into_index_mask`` in the CUDA-graph-safe
form cppmega patches in (cppmega/megatron/upstream_patches/apply_dsa_cg_patches.py:267-291;
its eager oracle is upstream_prs/examples/01_dsa_cuda_graph_safety/reproducer.py:124-138):

  * ``scatter_topk_into_index_mask(index_mask, idx_chunk, s0, s1)`` sets
    ``index_mask[b, s0 + r, idx_chunk[b, r, j]] = 0`` for every non-negative
    index, in place, and returns the mask (the caller has filled it with -inf);
  * ``topk_index_mask(topk_indices, s_kv)`` builds the whole [b, s_q, s_kv]
    mask (-inf, 0 on the top-k columns) in one pass, replacing the caller's
    ``torch.full(..., -inf)`` plus the scatter.

Both are one kernel launch with no host synchronisation (no ``.any()`` /
``.item()``), so they can be captured in a HIP graph.  Indices at or past
s_kv are skipped, where the reference's ``scatter_`` would raise.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["scatter_topk_into_index_mask", "topk_index_mask"]


def _launch(idx, mask, row0, rows, value, fill, fill_rows):
    if idx.dtype not in (torch.int64, torch.int32):
        raise TypeError(f"top-k indices must be int64 or int32, got {idx.dtype}")
    assert mask.dtype == torch.float32 and mask.dim() == 3 and mask.is_contiguous(), \
        "index_mask must be a contiguous [b, s_q, s_kv] float32 tensor"
    b, sq, sk = mask.shape
    assert idx.dim() == 3 and idx.shape[0] == b and idx.shape[1] == rows, \
        f"indices {tuple(idx.shape)} do not cover rows [{row0}, {row0 + rows}) of a batch-{b} mask"
    idx = idx.contiguous()
    dev = _lib.ensure_device(mask)
    rc = _lib.load().dsa_topk_index_mask(
        idx.data_ptr(), _lib.DTYPE_I64 if idx.dtype == torch.int64 else _lib.DTYPE_I32, idx.shape[-1],
        mask.data_ptr(), b, sq, sk, row0, rows, float(value), float(fill), 1 if fill_rows else 0,
        _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_topk_index_mask")
    return mask


def scatter_topk_into_index_mask(index_mask, idx_chunk, s0=0, s1=None):
    """In place: 0 at the (non-negative) top-k columns of rows [s0, s1); returns index_mask."""
    s1 = index_mask.shape[1] if s1 is None else s1
    return _launch(idx_chunk, index_mask, s0, s1 - s0, 0.0, float("-inf"), False)


def topk_index_mask(topk_indices, s_kv, value=0.0, fill=float("-inf"), out=None):
    """[b, s_q, topk] indices -> [b, s_q, s_kv] f32 mask: `value` on listed columns, `fill` elsewhere."""
    b, sq, _ = topk_indices.shape
    if out is None:
        out = torch.empty((b, sq, s_kv), dtype=torch.float32, device=topk_indices.device)
    return _launch(topk_indices, out, 0, sq, value, fill, True)
