"""IndexCache: cross-layer reuse of DSA top-k indices (arXiv:2603.12201).

Drop-in for cppmega/megatron/index_cache_patch.py:37-278.  DSA layers are
numbered in construction order ("DSA ranks").  Full ranks (default 0,3,6 from
CPPMEGA_INDEX_CACHE_FULL_LAYERS) run the indexer and cache their top-k
indices; Shared ranks skip the indexer and reuse the indices of the nearest
preceding Full rank; a Shared rank with no preceding Full rank in the cache is
promoted to Full (:168-184).  The cache is cleared when the lowest Full rank
runs, i.e. once per micro-batch (:115-117).

The schedule itself lives in ``IndexCacheSchedule`` (no Megatron needed);
``apply_index_cache_patch`` wires it into Megatron's ``DSAttention`` the same
way the reference does, re-deriving Full-layer indices with this package's
deterministic indexer + top-k.
"""
from __future__ import annotations

import logging
import os

import torch

log = logging.getLogger(__name__)


def parse_full_ranks(spec: str | None = None) -> set[int]:
    spec = os.environ.get("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0,3,6") if spec is None else spec
    return {int(x.strip()) for x in spec.split(",") if x.strip()}


class IndexCacheSchedule:
    """Full / Shared bookkeeping of IndexCache, independent of Megatron."""

    def __init__(self, full_ranks=None):
        self.full_ranks = parse_full_ranks() if full_ranks is None else set(full_ranks)
        self.min_full = min(self.full_ranks) if self.full_ranks else 0
        self.cache: dict[int, torch.Tensor] = {}
        self.step = -1
        self.promoted: set[int] = set()

    def is_full(self, rank: int) -> bool:
        return rank in self.full_ranks or rank in self.promoted

    def begin_layer(self, rank: int) -> None:
        if rank == self.min_full:
            self.step += 1
            self.cache.clear()

    def store(self, rank: int, indices: torch.Tensor) -> None:
        self.cache[rank] = indices

    def lookup(self, rank: int):
        """Indices of the nearest preceding cached rank, or None (caller promotes)."""
        for r in range(rank - 1, -1, -1):
            if r in self.cache:
                return self.cache[r]
        return None

    def promote(self, rank: int) -> None:
        self.promoted.add(rank)


_SCHEDULE: IndexCacheSchedule | None = None


def get_schedule() -> IndexCacheSchedule:
    global _SCHEDULE
    if _SCHEDULE is None:
        _SCHEDULE = IndexCacheSchedule()
    return _SCHEDULE


def apply_index_cache_patch(force: bool = False, dsa_module=None) -> bool:
    """Monkey-patch Megatron ``DSAttention`` (or ``dsa_module.DSAttention``) for IndexCache."""
    if dsa_module is None:
        from megatron.core.transformer.experimental_attention_variant import dsa as dsa_module
    from .dsa_topk import fused_qk_topk_naive

    cls = getattr(dsa_module, "DSAttention", None)
    assert cls is not None, "DSAttention not found in dsa module"
    marker = "__cppmega_amd_index_cache__"
    if getattr(cls, marker, False) and not force:
        return True

    sched = get_schedule()
    sched.full_ranks = parse_full_ranks()
    sched.min_full = min(sched.full_ranks) if sched.full_ranks else 0
    counter = [0]
    orig_init = cls.__init__
    orig_forward = cls.forward
    run_sparse = getattr(dsa_module, "_run_sparse_attention", None)

    def _ic_init(self, *args, **kwargs):
        orig_init(self, *args, **kwargs)
        self._ic_dsa_rank = counter[0]
        counter[0] += 1

    def _ic_forward(self, query, key, value, attention_mask, x, qr, position_ids=None, attn_mask_type=None,
                    attention_bias=None, packed_seq_params=None, up_v_weight=None):
        rank = self._ic_dsa_rank
        sched.begin_layer(rank)
        kw = dict(position_ids=position_ids, attn_mask_type=attn_mask_type, attention_bias=attention_bias,
                  packed_seq_params=packed_seq_params, up_v_weight=up_v_weight)
        cached = None if sched.is_full(rank) else sched.lookup(rank)
        if cached is None:
            if not sched.is_full(rank):
                sched.promote(rank)
                log.info("IndexCache: DSA rank %d promoted to FULL (no preceding Full rank)", rank)
            result = orig_forward(self, query, key, value, attention_mask, x, qr, **kw)
            with torch.no_grad():
                q_idx, k_idx, w_idx = self.indexer.forward_before_topk(x.detach(), qr.detach(), packed_seq_params)
                _, idx = fused_qk_topk_naive(q_idx, k_idx, w_idx, self.indexer.index_topk, mask=None,
                                             use_relu=getattr(self.config, "dsa_indexer_scoring_relu", True))
                sched.store(rank, idx)
            return result
        if run_sparse is None:
            raise RuntimeError("dsa module has no _run_sparse_attention for the Shared fast path")
        output, _ = run_sparse(query=query, key=key, value=value, up_v_weight=up_v_weight,
                               topk_indices=cached, softmax_scale=self.softmax_scale, config=self.config)
        return output

    cls.__init__ = _ic_init
    cls.forward = _ic_forward
    setattr(cls, marker, True)
    log.info("IndexCache installed: Full ranks %s", sorted(sched.full_ranks))
    return True


__all__ = ["IndexCacheSchedule", "apply_index_cache_patch", "get_schedule", "parse_full_ranks"]
