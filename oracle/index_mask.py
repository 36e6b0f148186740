"""CPU restatement of the top-k index mask of the sparse indexer loss.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

scatter_topk_into_index_mask restates the eager oracle of Megatron's
``_scatter_topk_into_index_mask``
(upstream_prs/examples/01_dsa_cuda_graph_safety/reproducer.py:124-138): for
every non-negative index of idx_chunk [b, s1 - s0, topk], mask[b, s0 + r, idx]
= 0; everything else unchanged.  Indices >= s_kv are skipped here (the
reference's advanced indexing would raise).

Pinned by (tests/test_oracle_index_mask.py): torch's own scatter_ on
sentinel-free chunks, the branchless clamp + scatter + column-0 fixup form
cppmega patches in (apply_dsa_cg_patches.py:278-288) on chunks with sentinels,
and a pure-Python fixture (tests/golden/index_mask.npz).
"""
from __future__ import annotations

import torch


def scatter_topk_into_index_mask(index_mask, idx_chunk, s0, s1, value=0.0):
    out = index_mask.clone()
    sk = out.shape[-1]
    valid = (idx_chunk >= 0) & (idx_chunk < sk)
    b_idx, q_rel, t_idx = torch.where(valid)
    out[b_idx, q_rel + s0, idx_chunk[b_idx, q_rel, t_idx].long()] = value
    return out


def topk_index_mask(topk_indices, sk, value=0.0, fill=float("-inf")):
    b, sq, _ = topk_indices.shape
    base = torch.full((b, sq, sk), fill, dtype=torch.float32)
    return scatter_topk_into_index_mask(base, topk_indices, 0, sq, value)
