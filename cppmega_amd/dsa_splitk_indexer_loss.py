"""DSA indexer KL loss on gfx950 — drop-in for cppmega's split-K indexer loss.

Mirrors cppmega/megatron/dsa_splitk_indexer_loss.py:
  * ``compute_dsa_indexer_loss_splitk(index_scores, topk_indices, query, key,
    softmax_scale, loss_coeff, sparse_loss, pg_collection)`` (:328-468), which
    has the signature of Megatron's ``compute_dsa_indexer_loss``.

The loss is KL(P || Q) averaged over positions and scaled by ``loss_coeff``:
P is the head mean of the causal (and, with ``sparse_loss``, top-k-masked)
attention softmax of ``query`` against ``key``; Q is the softmax of
``index_scores`` (plus the same top-k mask) over all key columns, as in the
reference test's definition (tests/test_dsa_splitk_indexer_loss.py:29-83).
Like the reference's Triton kernels, the [b, np, sq, sk] probabilities are
never materialised.  The reference's scalar carries no autograd history; here,
when ``index_scores`` requires grad, the loss is differentiable with respect to
it as Megatron's ``compute_dsa_indexer_loss`` is (the indexer's only gradient):
``indexer_kl_loss_backward`` recomputes P and writes
dL/dz = g * coeff / (b * sq) * (Q * R - P * Q / (Q + 1e-10)),
R = sum_j P_j Q_j / (Q_j + 1e-10), on the GPU (query and key get no gradient:
P is the detached target, as in Megatron).

``pg_collection`` is accepted for signature compatibility and, as in the
reference, not used: with tensor-parallel heads the caller must combine the
per-rank head averages itself.
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["compute_dsa_indexer_loss_splitk", "indexer_kl_loss", "indexer_kl_loss_backward"]

_HEAD_DIMS = (64, 128, 192, 256)


def _prepare(index_scores, topk_indices, query, key, sparse_loss):
    """Shape / dtype checks shared by the loss and its gradient; returns the
    contiguous operands and the dims the C-ABI takes."""
    assert index_scores.dim() == 3, f"index_scores must be [b, sq, sk], got {tuple(index_scores.shape)}"
    assert query.dim() == 4 and key.dim() == 4, \
        f"query/key must be [s, b, heads, hn], got {tuple(query.shape)} / {tuple(key.shape)}"
    sq, b, np_, hn = query.shape
    sk, bk, g, hk = key.shape
    assert bk == b and hk == hn, f"query {tuple(query.shape)} and key {tuple(key.shape)} disagree"
    assert np_ % g == 0, f"key heads {g} must divide query heads {np_}"
    assert tuple(index_scores.shape) == (b, sq, sk), \
        f"index_scores {tuple(index_scores.shape)} != {(b, sq, sk)}"
    assert hn in _HEAD_DIMS, f"head dim {hn} not supported (one of {_HEAD_DIMS})"
    if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16:
        raise TypeError(f"query/key must be bf16, got {query.dtype}/{key.dtype}")
    if index_scores.dtype != torch.float32:
        index_scores = index_scores.float()
    sparse = bool(sparse_loss)
    if sparse:
        assert topk_indices is not None and topk_indices.dim() == 3 and \
            tuple(topk_indices.shape[:2]) == (b, sq), \
            f"topk_indices must be [b, sq, topk], got {None if topk_indices is None else tuple(topk_indices.shape)}"
        if topk_indices.dtype not in (torch.int64, torch.int32):
            raise TypeError(f"topk_indices must be int64 or int32, got {topk_indices.dtype}")
        topk_indices = topk_indices.contiguous()
        topk = topk_indices.shape[-1]
        tdt = _lib.DTYPE_I64 if topk_indices.dtype == torch.int64 else _lib.DTYPE_I32
    else:
        topk, tdt = 0, _lib.DTYPE_I64
    query, key, index_scores = query.contiguous(), key.contiguous(), index_scores.detach().contiguous()
    dims = (b, sq, sk, np_, g, hn)
    return index_scores, (topk_indices if sparse else None), tdt, topk, query, key, sparse, dims


def _forward(index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss, return_rows):
    index_scores, topk_indices, tdt, topk, query, key, sparse, (b, sq, sk, np_, g, hn) = _prepare(
        index_scores, topk_indices, query, key, sparse_loss)
    dev = _lib.ensure_device(query)
    lib = _lib.load()
    ws_bytes = lib.dsa_indexer_kl_loss_workspace_size(b, sq, sk, np_, hn, 1 if sparse else 0)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=query.device)
    loss = torch.empty((), dtype=torch.float32, device=query.device)
    rows = torch.empty((b, sq), dtype=torch.float32, device=query.device) if return_rows else None
    rc = lib.dsa_indexer_kl_loss(
        index_scores.data_ptr(), _lib.ptr(topk_indices), tdt, topk,
        query.data_ptr(), key.data_ptr(), loss.data_ptr(), _lib.ptr(rows),
        b, sq, sk, np_, g, hn, float(softmax_scale), float(loss_coeff), 1 if sparse else 0,
        ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_indexer_kl_loss")
    return loss, rows


def indexer_kl_loss_backward(grad_loss, index_scores, topk_indices, query, key, softmax_scale, loss_coeff=1.0,
                             sparse_loss=False):
    """dL/d index_scores [b, sq, sk] f32 for the upstream gradient ``grad_loss``
    (a scalar tensor or number) of ``indexer_kl_loss``'s scalar; the target P is
    recomputed on the GPU.  NaN over a row whose loss is NaN."""
    index_scores, topk_indices, tdt, topk, query, key, sparse, (b, sq, sk, np_, g, hn) = _prepare(
        index_scores, topk_indices, query, key, sparse_loss)
    dev = _lib.ensure_device(query)
    lib = _lib.load()
    gl = torch.as_tensor(grad_loss, dtype=torch.float32, device=query.device).reshape(1).contiguous()
    ws_bytes = lib.dsa_indexer_kl_loss_workspace_size(b, sq, sk, np_, hn, 1 if sparse else 0)
    ws = torch.empty(max(int(ws_bytes), 1), dtype=torch.uint8, device=query.device)
    grad = torch.empty((b, sq, sk), dtype=torch.float32, device=query.device)
    rc = lib.dsa_indexer_kl_loss_backward(
        index_scores.data_ptr(), _lib.ptr(topk_indices), tdt, topk, query.data_ptr(), key.data_ptr(),
        gl.data_ptr(), grad.data_ptr(), b, sq, sk, np_, g, hn, float(softmax_scale), float(loss_coeff),
        1 if sparse else 0, ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "dsa_indexer_kl_loss_backward")
    return grad


class _IndexerKLLoss(torch.autograd.Function):
    """Scalar KL loss, differentiable with respect to index_scores only."""

    @staticmethod
    def forward(ctx, index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss):
        loss, _ = _forward(index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss, False)
        ctx.save_for_backward(index_scores, topk_indices if sparse_loss else None, query, key)
        ctx.args = (softmax_scale, loss_coeff, sparse_loss)
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        index_scores, topk_indices, query, key = ctx.saved_tensors
        softmax_scale, loss_coeff, sparse_loss = ctx.args
        grad = indexer_kl_loss_backward(grad_loss, index_scores, topk_indices, query, key, softmax_scale, loss_coeff,
                                        sparse_loss)
        return grad.to(index_scores.dtype), None, None, None, None, None, None


def indexer_kl_loss(index_scores, topk_indices, query, key, softmax_scale, loss_coeff=1.0, sparse_loss=False,
                    return_rows=False):
    """KL indexer loss on the GPU.

    index_scores [b, sq, sk] f32; topk_indices [b, sq, topk] int64 / int32 (read
    when ``sparse_loss``; entries outside [0, sk) are ignored); query
    [sq, b, np, hn] bf16; key [sk, b, g, hn] bf16 with g == np (the reference
    layout) or a divisor of np (grouped key heads).  Returns the scalar loss
    (0-dim f32), and with ``return_rows`` also the per-position KL [b, sq].
    The scalar is differentiable with respect to ``index_scores`` when that
    requires grad (and ``return_rows`` is off).
    """
    if index_scores.requires_grad and torch.is_grad_enabled() and not return_rows:
        return _IndexerKLLoss.apply(index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss)
    loss, rows = _forward(index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss, return_rows)
    return (loss, rows) if return_rows else loss


def compute_dsa_indexer_loss_splitk(index_scores, topk_indices, query, key, softmax_scale, loss_coeff,
                                    sparse_loss, pg_collection=None):
    """Drop-in for ``compute_dsa_indexer_loss_splitk`` (scalar f32 = coeff * mean KL)."""
    return indexer_kl_loss(index_scores, topk_indices, query, key, softmax_scale, loss_coeff, sparse_loss)
