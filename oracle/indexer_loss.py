"""CPU restatement of the DSA indexer KL loss.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The loss that ``compute_dsa_indexer_loss_splitk``
(cppmega/megatron/dsa_splitk_indexer_loss.py:328-468) computes on the GPU and
that the reference test checks it against
(tests/test_dsa_splitk_indexer_loss.py:29-83, a self-contained clone of
Megatron's ``compute_dsa_indexer_loss``):

  attention  a_h[t, s] = softmax_scale * query[t, h] . key[s, h]   (fp32)
             + (sparse) 0 on the top-k columns of row t, -inf elsewhere
             + causal: -inf for s > t
  target     P[t, s]   = mean_h softmax_s(a_h[t, :])
  index      Q[t, s]   = softmax_s(index_scores[t, :] (+ sparse mask))
             -- over every column s in [0, sk): the reference test's index
             softmax has no causal mask (in Megatron the scores it receives
             are already -inf above the diagonal, which makes no difference)
  loss       coeff * mean_{b,t} sum_s P (log(P + 1e-10) - log(Q + 1e-10))

A (b, t) row whose attention scores are all -inf (sparse mode: no top-k column
at or below t) has NaN softmax weights, hence a NaN row loss and a NaN mean, as
in the reference; the same holds for an all -inf index row.

Pinning (tests/test_oracle_indexer_loss.py): a pure-Python float64 fixture
(tests/golden/indexer_loss_*.npz, written from the definition above without
this module), the closed form KL_t = log(sk / (t + 1)) for zero queries and
constant index scores, KL = 0 when the index scores equal the single head's
causal attention logits, torch.nn.functional.kl_div on the same
distributions, linearity in loss_coeff, and planted mistakes (no causal mask,
a causally masked index softmax, a sum over heads, natural vs log2 units)
that the fixture comparison catches.
"""
from __future__ import annotations

import torch

EPS = 1e-10


def sparse_mask(topk_indices, sk, dtype=torch.float64):
    """[b, sq, topk] int -> [b, sq, sk] with 0 at every listed column, -inf elsewhere.

    Columns outside [0, sk) (the -1 padding of a short top-k row) are ignored;
    the reference's ``scatter_`` would reject them.
    """
    b, sq, _ = topk_indices.shape
    m = torch.full((b, sq, sk), float("-inf"), dtype=dtype)
    idx = topk_indices.long()
    ok = (idx >= 0) & (idx < sk)
    bb, tt, jj = torch.nonzero(ok, as_tuple=True)
    m[bb, tt, idx[bb, tt, jj]] = 0.0
    return m


def indexer_kl_rows(index_scores, topk_indices, query, key, softmax_scale, sparse_loss,
                    dtype=torch.float64):
    """Per-position KL [b, sq] (before the mean and loss_coeff).

    index_scores [b, sq, sk] f32, topk_indices [b, sq, topk] int,
    query [sq, b, np, hn], key [sk, b, G, hn] (G = np, or a divisor of np whose
    groups are shared by np / G consecutive heads).
    Follows tests/test_dsa_splitk_indexer_loss.py:47-83.
    """
    sq, b, np_, hn = query.shape
    sk, _, g, _ = key.shape
    assert np_ % g == 0
    q = query.to(dtype).permute(1, 2, 0, 3)                        # [b, np, sq, hn]
    k = key.to(dtype).repeat_interleave(np_ // g, dim=2).permute(1, 2, 3, 0)  # [b, np, hn, sk]
    att = torch.matmul(q, k) * softmax_scale                       # [b, np, sq, sk]
    mask = sparse_mask(topk_indices, sk, dtype) if sparse_loss else None
    if sparse_loss:
        att = att + mask.unsqueeze(1)
    causal = torch.triu(torch.full((sq, sk), float("-inf"), dtype=dtype), diagonal=1)
    att = att + causal
    target = torch.softmax(att, dim=-1).mean(dim=1)                # [b, sq, sk]
    idx_in = index_scores.to(dtype)
    if sparse_loss:
        idx_in = idx_in + mask
    index_probs = torch.softmax(idx_in, dim=-1)
    kl = target * (torch.log(target + EPS) - torch.log(index_probs + EPS))
    return kl.sum(dim=-1)


def compute_dsa_indexer_loss(index_scores, topk_indices, query, key, softmax_scale, loss_coeff,
                             sparse_loss, dtype=torch.float64):
    """Scalar loss = mean over (b, sq) of the per-position KL, times loss_coeff.

    Reference: compute_dsa_indexer_loss_splitk
    (cppmega/megatron/dsa_splitk_indexer_loss.py:328-468; ``out_loss.mean() * loss_coeff``
    at :467) and its test reference (tests/test_dsa_splitk_indexer_loss.py:29-83).
    """
    rows = indexer_kl_rows(index_scores, topk_indices, query, key, softmax_scale, sparse_loss, dtype)
    return rows.mean() * loss_coeff


def indexer_kl_grad(index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss,
                    grad_loss=1.0, dtype=torch.float64):
    """d(loss) / d(index_scores) [b, sq, sk] by autograd of compute_dsa_indexer_loss
    in float64 (query / key are the detached target's inputs, as in Megatron,
    whose indexer gradient is autograd through this same loss).  Pinned by
    torch.autograd.gradcheck against finite differences and by the invariants
    of a softmax gradient (every row sums to zero; zero wherever Q = 0)."""
    z = index_scores.detach().to(dtype).requires_grad_(True)
    loss = compute_dsa_indexer_loss(z, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss, dtype)
    (g,) = torch.autograd.grad(loss, z, grad_outputs=torch.as_tensor(grad_loss, dtype=dtype))
    return g


def kl_flops(b, sq, sk, np_, hn):
    """Algorithmic MFMA work of the causal attention target: two q.k passes
    (softmax statistics, then the recomputed KL), 2 * hn FLOP per (head, t, s <= t)."""
    pairs = sum(min(t + 1, sk) for t in range(sq))
    return 2 * (2 * b * np_ * hn * pairs)


def indexer_kl_rows_at(index_scores, topk_indices, query, key, softmax_scale, sparse_loss, positions,
                       dtype=torch.float64):
    """Per-position KL at the listed (b, t) positions only (same definition as
    indexer_kl_rows; for full-size inputs whose [b, np, sq, sk] form does not fit)."""
    sq, b, np_, hn = query.shape
    sk, _, g, _ = key.shape
    out = []
    for bi, t in positions:
        q = query[t, bi].to(dtype)                                   # [np, hn]
        k = key[:, bi].to(dtype).repeat_interleave(np_ // g, dim=1)  # [sk, np, hn]
        att = torch.einsum("hd,shd->hs", q, k) * softmax_scale       # [np, sk]
        allowed = torch.arange(sk) <= t
        idx_row = index_scores[bi, t].to(dtype)
        if sparse_loss:
            chosen = torch.zeros(sk, dtype=torch.bool)
            cols = topk_indices[bi, t].long()
            cols = cols[(cols >= 0) & (cols < sk)]
            chosen[cols] = True
            allowed = allowed & chosen
            idx_row = idx_row.masked_fill(~chosen, float("-inf"))
        att = att.masked_fill(~allowed, float("-inf"))
        target = torch.softmax(att, dim=-1).mean(dim=0)
        qp = torch.softmax(idx_row, dim=-1)
        out.append(float((target * (torch.log(target + EPS) - torch.log(qp + EPS))).sum()))
    return torch.tensor(out, dtype=dtype)
