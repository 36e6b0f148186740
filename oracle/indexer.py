"""CPU restatement of the DSA indexer scores.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

compute_index_scores follows compute_index_scores_fused_bf16
(cppmega/megatron/dsa_indexer_fused_patch.py:71-133): a per-head loop that
upcasts q and k to fp32, forms q_h . k with a batched matmul, applies ReLU,
multiplies by the fp32 head weight and accumulates into a [b, sq, sk] fp32
buffer.  compute_index_scores_einsum restates the upstream Megatron form
that the reference test clones (tests/test_dsa_indexer_fused_patch.py:18-30).
index_scores_backward gives the gradients autograd takes through that loop
(to q, weights and k), in float64.
The FP8 form dequantises e4m3 codes with one per-tensor scale for q and one
for k before the same arithmetic.
"""
from __future__ import annotations

import torch


def compute_index_scores(q, weights, k, use_relu=True, q_scale=None, k_scale=None):
    """q [sq,b,h,d], weights [sq,b,h], k [sk,b,d] -> [b, sq, sk] fp32."""
    sq, b, h, d = q.shape
    sk = k.shape[0]
    qs = 1.0 if q_scale is None else float(q_scale)
    ks = 1.0 if k_scale is None else float(k_scale)
    out = torch.zeros((b, sq, sk), dtype=torch.float32)
    k_bds = k.float().permute(1, 2, 0).contiguous()           # [b, d, sk]
    for hi in range(h):
        q_h = q[:, :, hi, :].float().permute(1, 0, 2).contiguous()  # [b, sq, d]
        logits = torch.bmm(q_h, k_bds)
        if q_scale is not None or k_scale is not None:
            logits = logits * (qs * ks)
        if use_relu:
            logits = torch.relu(logits)
        w_h = weights[:, :, hi].float().transpose(0, 1).unsqueeze(-1)
        out.add_(logits * w_h)
    return out


def compute_index_scores_einsum(q, weights, k, use_relu=True):
    """Upstream Megatron `_compute_index_scores` (einsum form)."""
    s = torch.einsum("sbhd,tbd->sbht", q.float(), k.float())
    if use_relu:
        s = torch.relu(s)
    s = s * weights.float().unsqueeze(-1)
    return s.sum(dim=2).transpose(0, 1)


def compute_index_scores_f64(q, weights, k, use_relu=True):
    """Float64 brute force over explicit loops of heads (tiny shapes only)."""
    sq, b, h, d = q.shape
    sk = k.shape[0]
    qd, kd, wd = q.double(), k.double(), weights.double()
    out = torch.zeros((b, sq, sk), dtype=torch.float64)
    for bi in range(b):
        for hi in range(h):
            logits = qd[:, bi, hi, :] @ kd[:, bi, :].T           # [sq, sk]
            if use_relu:
                logits = logits.clamp_min(0)
            out[bi] += logits * wd[:, bi, hi][:, None]
    return out


def index_scores_diff(q, weights, k, use_relu=True):
    """Differentiable float64 restatement of the reference's per-head loop
    (cppmega/megatron/dsa_indexer_fused_patch.py:71-133): per head, q_h . k,
    ReLU, times the head weight, accumulated over heads -> [b, sq, sk].
    Inputs are used as given (float64 leaves that may require grad)."""
    sq, b, h, d = q.shape
    out = None
    for hi in range(h):
        logits = torch.einsum("sbd,tbd->bst", q[:, :, hi, :], k)   # [b, sq, sk]
        if use_relu:
            logits = torch.relu(logits)
        term = logits * weights[:, :, hi].transpose(0, 1).unsqueeze(-1)
        out = term if out is None else out + term
    return out


def index_scores_backward(grad, q, weights, k, use_relu=True, causal=False, starts=None, ends=None):
    """Gradients (dq, dweights, dk) in float64 of the reference's score loop for
    the upstream gradient `grad` [b, sq, sk], by autograd through
    index_scores_diff (what autograd through the reference's torch loop
    computes).  causal=True zeroes grad above the diagonal first (the entries
    a lower-triangle forward never computed); starts / ends ([b, sq] or [sq])
    zero it outside each row's window [start, end) (the entries a window-mode
    forward writes as -inf whatever the raw score).  Pinned by
    torch.autograd.gradcheck (finite differences) and a one-head, one-key
    closed form in tests/test_oracle_indexer_topk_fp8.py."""
    g = grad.detach().double()
    if causal:
        sq, sk = g.shape[-2:]
        g = g.masked_fill(torch.ones(sq, sk, dtype=torch.bool).triu(1), 0.0)
    if starts is not None:
        b, sq, sk = g.shape
        col = torch.arange(sk).view(1, 1, sk)
        st_ = torch.as_tensor(starts).to(torch.int64).expand(b, sq).unsqueeze(-1)
        en_ = torch.as_tensor(ends).to(torch.int64).expand(b, sq).unsqueeze(-1)
        g = g.masked_fill((col < st_) | (col >= en_), 0.0)
    with torch.enable_grad():  # also when called from inside another backward
        qd = q.detach().double().requires_grad_(True)
        wd = weights.detach().double().requires_grad_(True)
        kd = k.detach().double().requires_grad_(True)
        out = index_scores_diff(qd, wd, kd, use_relu)
        dq, dw, dk = torch.autograd.grad(out, (qd, wd, kd), grad_outputs=g)
    return dq, dw, dk


def causal_mask_(scores, fill=float("-inf")):
    """Set score[b, t, s] = fill for s > t (in place) and return it."""
    sq, sk = scores.shape[-2:]
    mask = torch.ones(sq, sk, dtype=torch.bool).triu(1)
    scores.masked_fill_(mask, fill)
    return scores


def flops_causal(b, s, h, d):
    """Algorithmic causal FLOPs: 2 * b * h * d * s (s + 1) / 2."""
    return 2 * b * h * d * s * (s + 1) // 2
