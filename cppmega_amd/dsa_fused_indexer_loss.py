"""Fused DSA indexer loss on gfx950: Megatron's ``FusedDSAIndexerLoss`` drop-in.

Megatron trains the DSA indexer through ``dsa.FusedDSAIndexerLoss.apply``,
which cppmega replaces with the lemyx kernel in
cppmega/megatron/lemyx_dsa_warmup.py:86-178 (same call:
``apply(q, weights, k, query, key, softmax_scale, topk, loss_coeff, mask,
sparse_loss, pg_collection, varlen_starts, varlen_ends, key_positions,
query_valid_rows, use_relu) -> (topk_indices, loss)``; the gradient of the loss
flows to the indexer's q, weights and k, while query / key are the detached
attention inputs).  Here the chain is three gfx950 pieces, all on the device:

  1. index scores of q / weights / k with the mask or varlen windows added
     (``fused_qk_topk_naive``'s window-mode indexer; differentiable through
     ``IndexScores``), and the deterministic top-k of those scores;
  2. the KL loss between the causal (sparse: top-k-masked) head-mean attention
     of query / key and the softmax of the scores (``indexer_kl_loss``, the
     definition of Megatron's compute_dsa_indexer_loss, differentiable with
     respect to the scores);
  3. in backward, the KL gradient to the scores [b, sq, sk] (written once),
     then the indexer backward to q, weights and k (dsa_indexer_scores_backward).

The [b, sq, sk] scores are materialised once (they are the loss's input, as
in Megatron) and their gradient once; the [b, np, sq, sk] attention
probabilities never are.  The attention target is causal, as the KL loss
defines it; a mask beyond causal restricts the index scores and the top-k.
"""
from __future__ import annotations

import torch

from . import dsa_topk
from .dsa_splitk_indexer_loss import indexer_kl_loss

__all__ = ["FusedDSAIndexerLoss", "apply_fused_indexer_loss_patch", "fused_dsa_indexer_loss"]

# The Megatron dsa module this drop-in was installed into.  The top-k is looked
# up on it at call time (cppmega/megatron/lemyx_dsa_warmup.py:166-176 imports
# ``fused_qk_topk_naive`` from the dsa module inside ``apply``), so whatever is
# bound there at that moment runs: the gfx950 top-k patch, or IndexCache's
# capture wrapper around it while a Full layer's forward is running.
_DSA_MODULE = None


def _topk_fn():
    fn = getattr(_DSA_MODULE, "fused_qk_topk_naive", None) if _DSA_MODULE is not None else None
    return fn if fn is not None else dsa_topk.fused_qk_topk_naive


def fused_dsa_indexer_loss(q, weights, k, query, key, softmax_scale, topk, loss_coeff, mask=None,
                           sparse_loss=False, pg_collection=None, varlen_starts=None, varlen_ends=None,
                           key_positions=None, query_valid_rows=None, use_relu=True):
    """(topk_indices [b, sq, k] int64, loss 0-dim f32): the indexer's top-k and its
    KL training loss; ``loss.backward()`` reaches q, weights and k.

    q [sq, b, h_idx, d] bf16, weights [sq, b, h_idx] (f32 or bf16), k [sk, b, d]
    bf16; query [sq, b, np, hn] / key [sk, b, np or a divisor, hn] bf16 (the
    attention inputs; no gradient).  ``query_valid_rows`` and ``pg_collection``
    are accepted and not used, as in the lemyx drop-in
    (cppmega/megatron/lemyx_dsa_warmup.py:86-178, which takes
    ``query_valid_rows`` and never reads it) and cppmega's split-K loss.

    The scores and top-k come from ``fused_qk_topk_naive`` as bound on the dsa
    module that ``apply_fused_indexer_loss_patch`` installed this into, looked
    up at call time; without one, from this package's gfx950 implementation.
    """
    del query_valid_rows, pg_collection
    scores, topk_indices = _topk_fn()(q, k, weights, topk, mask=mask, varlen_starts=varlen_starts,
                                      varlen_ends=varlen_ends, key_positions=key_positions, use_relu=use_relu)
    loss = indexer_kl_loss(scores, topk_indices, query.detach(), key.detach(), softmax_scale, loss_coeff,
                           sparse_loss)
    return topk_indices, loss


class FusedDSAIndexerLoss:
    """Drop-in for Megatron's ``dsa.FusedDSAIndexerLoss``: ``apply`` has its
    signature and returns (topk_indices, loss).  Not an autograd.Function
    itself: autograd runs through IndexScores and the KL loss."""

    @staticmethod
    def apply(q, weights, k, query, key, softmax_scale, topk, loss_coeff, mask, sparse_loss, pg_collection,
              varlen_starts=None, varlen_ends=None, key_positions=None, query_valid_rows=None, use_relu=True):
        return fused_dsa_indexer_loss(q, weights, k, query, key, softmax_scale, topk, loss_coeff, mask=mask,
                                      sparse_loss=sparse_loss, pg_collection=pg_collection,
                                      varlen_starts=varlen_starts, varlen_ends=varlen_ends,
                                      key_positions=key_positions, query_valid_rows=query_valid_rows,
                                      use_relu=use_relu)


_MARKER = "__cppmega_amd_fused_indexer_loss__"
setattr(FusedDSAIndexerLoss, _MARKER, True)


def apply_fused_indexer_loss_patch(*, force: bool = False, dsa_module=None) -> bool:
    """Install ``FusedDSAIndexerLoss`` as Megatron's ``dsa.FusedDSAIndexerLoss``
    (what cppmega's apply_lemyx_dsa_patch does for its kernel,
    cppmega/megatron/lemyx_dsa_warmup.py:188-207).  Idempotent; raises when the
    attribute is absent (Megatron version mismatch).  From then on the loss
    takes its top-k from ``dsa_module.fused_qk_topk_naive``, resolved per call."""
    global _DSA_MODULE
    if dsa_module is None:
        from megatron.core.transformer.experimental_attention_variant import dsa as dsa_module
    existing = getattr(dsa_module, "FusedDSAIndexerLoss", None)
    if existing is None:
        raise RuntimeError("dsa.FusedDSAIndexerLoss not found - Megatron version mismatch?")
    _DSA_MODULE = dsa_module
    if getattr(existing, _MARKER, False) and not force:
        return True
    dsa_module.FusedDSAIndexerLoss = FusedDSAIndexerLoss
    return True
