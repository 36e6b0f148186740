"""The reference's CPU PyTorch path for one DSA layer step, timed as the CPU baseline.

TEST / BENCHMARK INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates, on a bounded sample of query tokens, what the reference runs in
PyTorch for one DSA layer:
  * indexer scores: the per-head fp32 bmm + ReLU + weight + accumulate loop of
    compute_index_scores_fused_bf16 (cppmega/megatron/dsa_indexer_fused_patch.py:71-133)
    over every key (the reference scores the full row; no causal skip);
  * top-k: ``index_scores.topk(min(topk, seqlen), dim=-1)[1]``
    (scripts/modal_dsa_indexer_bench.py:188-194) after a causal -inf mask;
  * SparseMLA forward: batched gather -> masked softmax -> gather
    (scripts/precision_sparse_mla_fullscale.py:77-125 semantics), fp32;
  * SparseMLA backward: torch autograd of that forward.
Per-token cost is independent of the token's position (full-row scores, fixed
top-k), so tokens/s measured on a sample scales to the full workload.
"""
from __future__ import annotations

import os
import time

import torch


def _indexer_topk(q, w, k, topk, t_pos):
    """q [T,b,h,d], w [T,b,h], k [sk,b,d]; t_pos [T] query positions -> idx [b,T,topk] int64."""
    T, b, h, d = q.shape
    sk = k.shape[0]
    scores = torch.zeros((b, T, sk), dtype=torch.float32)
    k_bds = k.float().permute(1, 2, 0).contiguous()
    for hi in range(h):
        q_h = q[:, :, hi, :].float().permute(1, 0, 2).contiguous()
        logits = torch.relu(torch.bmm(q_h, k_bds))
        scores.add_(logits * w[:, :, hi].float().transpose(0, 1).unsqueeze(-1))
    mask = torch.arange(sk)[None, :] > t_pos[:, None]
    scores.masked_fill_(mask[None], float("-inf"))
    return scores.topk(min(topk, sk), dim=-1)[1]


def _sparse_fwd(q, kv, idx, scale, d_v):
    """q [b,T,h,D] fp32 (requires grad), kv [b,sk,D] fp32, idx [b,T,topk] -> out [b,T,h,d_v]."""
    valid = idx >= 0
    safe = idx.clamp_min(0)
    b = q.shape[0]
    rows = torch.stack([kv[i][safe[i]] for i in range(b)])            # [b,T,k,D]
    s = torch.einsum("bthd,btkd->bthk", q, rows) * scale
    s = s.masked_fill(~valid[:, :, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bthk,btkd->bthd", p, rows[..., :d_v])


def layer_step(sample, topk, scale, d_v):
    """One reference-path step over the sampled tokens; returns per-phase seconds."""
    t0 = time.perf_counter()
    with torch.no_grad():
        idx_tok = _indexer_topk(sample["iq"], sample["iw"], sample["ik"], topk, sample["t_pos"])
    t1 = time.perf_counter()
    q = sample["q"].float().requires_grad_()
    kv = sample["kv"].float().requires_grad_()
    out = _sparse_fwd(q, kv, sample["idx"], scale, d_v)
    t2 = time.perf_counter()
    out.backward(sample["do"].float())
    t3 = time.perf_counter()
    del idx_tok
    return {"indexer_topk": t1 - t0, "fwd": t2 - t1, "bwd": t3 - t2}


def make_sample(cfg2, cfg3, tokens):
    """Slice the last `tokens` query positions of batch 0 (full keys / kv kept)."""
    S = cfg2["q"].shape[1]
    sel = torch.arange(S - tokens, S)
    return {
        "iq": cfg3["q"][sel][:, :1].contiguous(), "iw": cfg3["w"][sel][:, :1].contiguous(),
        "ik": cfg3["k"][:, :1].contiguous(), "t_pos": sel,
        "q": cfg2["q"][:1, sel].contiguous(), "kv": cfg2["kv"][:1, :, 0].contiguous(),
        "idx": cfg2["indices"][:1, sel, 0].long(), "do": cfg2["do"][:1, sel].contiguous(),
    }


def time_cpu_baseline(cfg2, cfg3, topk, scale, d_v, tokens=256, reps=3):
    """Median-of-reps tokens/s of the reference CPU path on `tokens` sampled tokens."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    sample = make_sample(cfg2, cfg3, tokens)
    layer_step(sample, topk, scale, d_v)  # warm-up
    runs = [layer_step(sample, topk, scale, d_v) for _ in range(reps)]
    tot = sorted(sum(r.values()) for r in runs)[len(runs) // 2]
    med = {k: sorted(r[k] for r in runs)[len(runs) // 2] for k in runs[0]}
    return {
        "tokens_per_s": tokens / tot, "seconds_per_rep": tot, "cores": torch.get_num_threads(),
        "phases_s": med, "tokens": tokens, "torch": torch.__version__,
    }
