"""Pinning of the index-mask oracle (oracle/index_mask.py) against torch's
scatter_, the branchless form cppmega patches in, and a pure-Python fixture."""
from __future__ import annotations

import numpy as np
import torch

from oracle import index_mask as oim
from tests._util import load_golden


def _patched_branchless(index_mask, idx_chunk, s0, s1):
    """The clamp + scatter + column-0 fixup of apply_dsa_cg_patches.py:278-288 (restated)."""
    out = index_mask.clone()
    sentinel = idx_chunk < 0
    out[:, s0:s1].scatter_(-1, idx_chunk.clamp(min=0), 0.0)
    has_sent = sentinel.any(dim=-1)
    has_real0 = ((idx_chunk == 0) & ~sentinel).any(dim=-1)
    out[:, s0:s1, 0].masked_fill_(has_sent & ~has_real0, float("-inf"))
    return out


def test_fixture():
    z = load_golden("index_mask.npz")
    idx = torch.from_numpy(z["idx"])
    s0, s1, sk = int(z["s0"]), int(z["s1"]), int(z["s_kv"])
    base = torch.full((idx.shape[0], 64, sk), float("-inf"))
    got = oim.scatter_topk_into_index_mask(base, idx, s0, s1)
    assert torch.equal(got, torch.from_numpy(z["mask"]))


def test_matches_torch_scatter_without_sentinels():
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 100, (2, 30, 12), generator=g)
    base = torch.full((2, 50, 100), float("-inf"))
    ref = base.clone()
    ref[:, 10:40].scatter_(-1, idx, 0.0)
    assert torch.equal(oim.scatter_topk_into_index_mask(base, idx, 10, 40), ref)


def test_matches_branchless_patch_with_sentinels():
    g = torch.Generator().manual_seed(4)
    idx = torch.randint(0, 256, (2, 64, 8), generator=g)
    idx = torch.where(torch.rand(idx.shape, generator=g) < 0.15, torch.full_like(idx, -1), idx)
    idx[0, 0] = -1
    idx[1, 3, :2] = 0
    base = torch.full((2, 64, 256), float("-inf"))
    assert torch.equal(oim.scatter_topk_into_index_mask(base, idx, 0, 64), _patched_branchless(base, idx, 0, 64))


def test_full_mask_form():
    idx = torch.tensor([[[2, -1, 2], [0, 4, 9]]])
    m = oim.topk_index_mask(idx, 6)
    exp = np.full((1, 2, 6), -np.inf, dtype=np.float32)
    exp[0, 0, 2] = 0
    exp[0, 1, [0, 4]] = 0
    assert torch.equal(m, torch.from_numpy(exp))
