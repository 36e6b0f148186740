"""IndexCache: cross-layer reuse of DSA top-k indices (arXiv:2603.12201).

Drop-in for cppmega/megatron/index_cache_patch.py:37-278.  DSA layers are
numbered in construction order ("DSA ranks").  Full ranks (default 0,3,6 from
CPPMEGA_INDEX_CACHE_FULL_LAYERS, :68-69) run the original forward and cache
their top-k indices; Shared ranks skip the indexer and run sparse attention
with the indices of the nearest preceding cached rank (:160-166); a Shared
rank with nothing cached before it is promoted to Full for good (:168-184).
The cache is cleared when the lowest Full rank runs, i.e. once per
micro-batch (:115-117).

The schedule itself lives in ``IndexCacheSchedule`` (no Megatron needed);
``apply_index_cache_patch`` wires it into Megatron's ``DSAttention``.  The
reference runs a Full layer's original forward and then derives the indices a
second time (``forward_before_topk`` + an unmasked ``fused_qk_topk_naive``,
:136-154), because the forward does not expose the ones it computed.  Here the
Full layer computes them once: while its original forward runs, the dsa
module's ``fused_qk_topk_naive`` and ``FusedDSAIndexerLoss.apply`` (the
indexer-loss path, which returns the top-k indices beside the loss) are
wrapped so the indices the layer itself selected (with its own mask, on its
own inputs) are captured and cached.  Only when the forward calls neither does
the layer fall back to the reference's re-derivation, done with this package's
deterministic gfx950 indexer + top-k and with the layer's own attention mask
(``_build_dsattention_forward_mask``), so both routes cache the same picks.

Deviation from the reference: the cached indices are the Full layer's masked
picks (the ones its own sparse attention used), where the reference caches an
unmasked ``mask=None`` top-k (index_cache_patch.py:148-153) whose rows may pick
future keys that the Shared layers' mask then discards.
Context-parallel gathers go through Megatron's
``gather_from_sequence_parallel_region`` exactly where the reference calls it.
"""
from __future__ import annotations

import logging
import os

import torch

from .dsa_topk import fused_qk_topk_naive

log = logging.getLogger(__name__)

_MARKER = "__cppmega_amd_index_cache__"


def parse_full_ranks(spec: str | None = None) -> set[int]:
    """"0,3,6" -> {0, 3, 6} (index_cache_patch.py:67-69)."""
    spec = os.environ.get("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0,3,6") if spec is None else spec
    return {int(x.strip()) for x in spec.split(",") if x.strip()}


class IndexCacheSchedule:
    """Full / Shared bookkeeping of IndexCache, independent of Megatron.

    ``cache`` maps DSA rank -> topk_indices [b, sq, topk] (index_cache_patch.py:33-34);
    ``step`` counts micro-batches (the reference's _CACHE_STEP).
    """

    def __init__(self, full_ranks=None):
        self.set_full_ranks(parse_full_ranks() if full_ranks is None else full_ranks)
        self.cache: dict[int, torch.Tensor] = {}
        self.step = -1
        self.promoted: set[int] = set()
        self.captured = 0    # Full-layer forwards whose own top-k indices were cached
        self.rederived = 0   # Full-layer forwards that fell back to a second indexer + top-k pass

    def set_full_ranks(self, ranks) -> None:
        self.full_ranks = set(ranks)
        self.min_full = min(self.full_ranks) if self.full_ranks else 0

    def is_full(self, rank: int) -> bool:
        return rank in self.full_ranks or rank in self.promoted

    def begin_layer(self, rank: int) -> None:
        """Called at the top of every DSA forward: the lowest Full rank starts a micro-batch."""
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

    def savings(self, n_layers: int = 9) -> tuple[int, int, int]:
        """(full, shared, percent of indexer work saved) for n_layers DSA layers (:264-267)."""
        n_full = len(self.full_ranks)
        n_shared = n_layers - n_full
        return n_full, n_shared, int(n_shared / n_layers * 100)


_SCHEDULE: IndexCacheSchedule | None = None


def get_schedule() -> IndexCacheSchedule:
    global _SCHEDULE
    if _SCHEDULE is None:
        _SCHEDULE = IndexCacheSchedule()
    return _SCHEDULE


def _cp_info(indexer):
    cp_group = getattr(getattr(indexer, "pg_collection", None), "cp", None)
    size = cp_group.size() if cp_group is not None else 1
    rank = cp_group.rank() if cp_group is not None else 0
    return cp_group, size, rank


def apply_index_cache_patch(force: bool = False, dsa_module=None) -> bool:
    """Monkey-patch Megatron ``DSAttention`` (or ``dsa_module.DSAttention``) for IndexCache.

    Mirrors cppmega/megatron/index_cache_patch.py:37-278: same marker
    semantics (a second call is a no-op unless ``force``), same Full / Shared
    / promote flow, same helpers taken from the dsa module for the Shared
    fast path (_run_sparse_attention, _ensure_sbhd,
    _normalize_dsattention_output_rank, _build_dsattention_forward_mask,
    _normalize_cp_comm_type).
    """
    if dsa_module is None:
        from megatron.core.transformer.experimental_attention_variant import dsa as dsa_module

    cls = getattr(dsa_module, "DSAttention", None)
    assert cls is not None, "DSAttention not found in dsa module"
    if getattr(cls, _MARKER, False) and not force:
        return True

    run_sparse = dsa_module._run_sparse_attention
    ensure_sbhd = dsa_module._ensure_sbhd
    normalize_rank = dsa_module._normalize_dsattention_output_rank
    build_mask = dsa_module._build_dsattention_forward_mask
    normalize_cp = dsa_module._normalize_cp_comm_type
    try:
        from megatron.core.tensor_parallel.mappings import gather_from_sequence_parallel_region as cp_gather
    except ImportError:
        cp_gather = None

    sched = get_schedule()
    sched.set_full_ranks(parse_full_ranks())
    log.info("IndexCache: Full DSA layer ranks: %s", sorted(sched.full_ranks))
    counter = [0]
    orig_init = cls.__init__
    orig_forward = cls.forward

    def _layer_mask(self, sq, skv, b, device, attention_mask, attn_mask_type, position_ids, packed_seq_params):
        """The layer's attention mask as Megatron builds it for sparse attention:
        (float_mask, varlen_starts, varlen_ends, key_positions)."""
        cp_group, cp_size, cp_rank = _cp_info(self.indexer)
        float_mask, varlen = build_mask(
            sq=sq, skv=skv, b=b, device=device, cp_size=cp_size, cp_rank=cp_rank,
            cp_comm_type=normalize_cp(getattr(self, "cp_comm_type", None)), cp_group=cp_group,
            attn_mask_type=attn_mask_type, attention_mask=attention_mask, position_ids=position_ids,
            packed_seq_params=packed_seq_params, packed_query_positions=None)
        starts, ends, key_positions = varlen if varlen is not None else (None, None, None)
        return float_mask, starts, ends, key_positions

    def _ic_init(self, *args, **kwargs):
        orig_init(self, *args, **kwargs)
        self._ic_dsa_rank = counter[0]
        self._ic_is_full = counter[0] in sched.full_ranks
        counter[0] += 1

    def _ic_forward(self, query, key, value, attention_mask, x, qr, position_ids=None, attn_mask_type=None,
                    attention_bias=None, packed_seq_params=None, up_v_weight=None):
        rank = self._ic_dsa_rank
        sched.begin_layer(rank)
        kw = dict(position_ids=position_ids, attn_mask_type=attn_mask_type, attention_bias=attention_bias,
                  packed_seq_params=packed_seq_params, up_v_weight=up_v_weight)
        cached = None
        if not (self._ic_is_full or sched.is_full(rank)):
            cached = sched.lookup(rank)
            if cached is None:
                self._ic_is_full = True
                sched.promote(rank)
                log.info("IndexCache: DSA rank %d auto-promoted to FULL (no preceding Full rank)", rank)
        if cached is None:
            # compute once: keep what the layer's own top-k call returns, through
            # the plain top-k or through the indexer-loss path
            captured = []
            inner = getattr(dsa_module, "fused_qk_topk_naive", None)
            inner_loss = getattr(dsa_module, "FusedDSAIndexerLoss", None)
            if inner is not None:
                def _capture(*a, **k):
                    res = inner(*a, **k)
                    captured.append(res[1])
                    return res

                dsa_module.fused_qk_topk_naive = _capture
            if inner_loss is not None:
                class _CaptureLoss:
                    @staticmethod
                    def apply(*a, **k):
                        res = inner_loss.apply(*a, **k)
                        captured.append(res[0])
                        return res

                dsa_module.FusedDSAIndexerLoss = _CaptureLoss
            try:
                result = orig_forward(self, query, key, value, attention_mask, x, qr, **kw)
            finally:
                if inner is not None:
                    dsa_module.fused_qk_topk_naive = inner
                if inner_loss is not None:
                    dsa_module.FusedDSAIndexerLoss = inner_loss
            if captured:
                sched.store(rank, captured[-1].detach())
                sched.captured += 1
                return result
            sched.rederived += 1
            with torch.no_grad():
                q_idx, k_idx, w_idx = self.indexer.forward_before_topk(x.detach(), qr.detach(), packed_seq_params)
                cp_group, cp_size, cp_rank = _cp_info(self.indexer)
                q_sbhd, _ = ensure_sbhd(query, "query")
                k_sbhd, _ = ensure_sbhd(key, "key")
                sq_local, b = q_sbhd.size(0), q_sbhd.size(1)
                skv = k_sbhd.size(0)
                if cp_size > 1 and cp_gather is not None:
                    if k_idx.size(0) == sq_local:
                        k_idx = cp_gather(k_idx, group=cp_group)
                    if skv == sq_local:
                        skv *= cp_size
                float_mask, starts, ends, key_positions = _layer_mask(
                    self, sq_local, skv, b, x.device, attention_mask, attn_mask_type, position_ids,
                    packed_seq_params)
                _, idx = fused_qk_topk_naive(q_idx, k_idx, w_idx, self.indexer.index_topk, mask=float_mask,
                                             varlen_starts=starts, varlen_ends=ends, key_positions=key_positions,
                                             use_relu=getattr(self.config, "dsa_indexer_scoring_relu", False))
                sched.store(rank, idx)
            return result

        # Shared fast path: sparse attention on the cached indices, no indexer, no indexer loss
        query, _ = ensure_sbhd(query, "query")
        key, _ = ensure_sbhd(key, "key")
        if value is not None:
            value, _ = ensure_sbhd(value, "value")
        if up_v_weight is not None:
            up_v_weight = up_v_weight.to(device=query.device, dtype=query.dtype).contiguous()
        latent = int(getattr(self.config, "kv_lora_rank", 0) or 0)
        pos = int(getattr(self.config, "qk_pos_emb_head_dim", 0) or 0)
        absorbed = (latent > 0 and latent + pos > 0 and key.size(2) == 1
                    and query.size(-1) == key.size(-1) == latent + pos)
        sq, b = query.size(0), query.size(1)
        cp_group, cp_size, cp_rank = _cp_info(self.indexer)
        if cp_size > 1 and cp_gather is not None:
            if key.size(0) == sq:
                key = cp_gather(key, group=cp_group)
            if value is not None and value.size(0) == sq:
                value = cp_gather(value, group=cp_group)
        float_mask, starts, ends, key_positions = _layer_mask(
            self, sq, key.size(0), b, x.device, attention_mask, attn_mask_type, position_ids, packed_seq_params)
        output, _ = run_sparse(absorbed_mla=absorbed, query=query, key=key, value=value, up_v_weight=up_v_weight,
                               topk_indices=cached, softmax_scale=self.softmax_scale, config=self.config,
                               mask=float_mask, varlen_starts=starts, varlen_ends=ends,
                               key_positions=key_positions)
        return normalize_rank(output, x.ndim)

    cls.__init__ = _ic_init
    cls.forward = _ic_forward
    setattr(cls, _MARKER, True)
    n_full, n_shared, pct = sched.savings()
    log.info("IndexCache installed: %d Full + %d Shared = %d%% indexer savings", n_full, n_shared, pct)
    return True


__all__ = ["IndexCacheSchedule", "apply_index_cache_patch", "get_schedule", "parse_full_ranks"]
