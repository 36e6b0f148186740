"""Seeded synthetic inputs for the DSA hot path (the benchmark configurations).

All tensors are generated on the CPU with a fixed torch.Generator so that the
CPU baseline and the GPU run see identical bytes; callers move them to the
device.  Shapes and distributions follow the configurations the benchmark
quotes:
  cfg1  SparseMLA fwd, b=1 s=512 h=16 d_qk=128 d_v=64 topk=64, q/kv ~ N(0,1)*0.5
  cfg2  SparseMLA fwd+bwd, b=2 s=4096 h=32 d_qk=128 d_v=64 topk=256,
        q/kv ~ N(0, 0.5) (0.5 read as the standard deviation), dO ~ N(0,1)
  cfg3  indexer q [s,b,16,64], k [s,b,64] ~ N(0,1) bf16, w ~ N(0,1)/4 f32,
        causal top-k 256
  cfg4  cfg2 shapes, values N(0,1) with 1% outliers x20, e4m3 tensorwise
Indices: for token t, min(t+1, topk) distinct positions drawn uniformly from
[0, t], sorted ascending, padded with -1.
"""
from __future__ import annotations

import torch

DEFAULT_SEED = 1234


def causal_indices(B, S, topk, seed=DEFAULT_SEED, chunk=1024, S_kv=None):
    """int32 [B, S, 1, topk]: uniform distinct causal picks, ascending, -1 padded."""
    S_kv = S if S_kv is None else S_kv
    g = torch.Generator().manual_seed(seed)
    out = torch.full((B, S, 1, topk), -1, dtype=torch.int32)
    cols = torch.arange(S_kv)
    for b in range(B):
        for t0 in range(0, S, chunk):
            t1 = min(S, t0 + chunk)
            keys = torch.rand((t1 - t0, S_kv), generator=g)
            t = torch.arange(t0, t1)[:, None]
            keys = torch.where(cols[None, :] <= t, keys, torch.full_like(keys, -1.0))
            k = min(topk, S_kv)
            val, idx = keys.topk(k, dim=-1)
            idx = torch.where(val >= 0, idx, torch.full_like(idx, S_kv + 1))
            idx, _ = idx.sort(dim=-1)
            idx = torch.where(idx > S_kv, torch.full_like(idx, -1), idx)
            out[b, t0:t1, 0, :k] = idx.to(torch.int32)
    return out


def sparse_mla_inputs(B, S, H, d_qk, d_v, topk, std=0.5, seed=DEFAULT_SEED, S_kv=None, grad=True):
    """dict(q, kv, indices, do, scale) on the CPU (bf16 q/kv/do, int32 indices)."""
    S_kv = S if S_kv is None else S_kv
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn((B, S, H, d_qk), generator=g) * std).to(torch.bfloat16)
    kv = (torch.randn((B, S_kv, 1, d_qk), generator=g) * std).to(torch.bfloat16)
    idx = causal_indices(B, S, topk, seed=seed + 1, S_kv=S_kv)
    d = dict(q=q, kv=kv, indices=idx, scale=d_qk ** -0.5)
    if grad:
        d["do"] = torch.randn((B, S, H, d_v), generator=g).to(torch.bfloat16)
    return d


def outlier_values(shape, seed, frac=0.01, mult=20.0):
    """N(0,1) with a seeded `frac` of entries multiplied by `mult` (cfg4)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    mask = torch.rand(shape, generator=g) < frac
    return torch.where(mask, x * mult, x)


def indexer_inputs(B, S, H, D, seed=DEFAULT_SEED, w_dtype=torch.float32):
    """q [S,B,H,D] bf16, k [S,B,D] bf16, w [S,B,H] ~ N(0,1)/sqrt(H)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((S, B, H, D), generator=g).to(torch.bfloat16)
    k = torch.randn((S, B, D), generator=g).to(torch.bfloat16)
    w = (torch.randn((S, B, H), generator=g) / H ** 0.5).to(w_dtype)
    return dict(q=q, k=k, w=w)
