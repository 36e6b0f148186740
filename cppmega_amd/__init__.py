"""cppmega_amd — MI355X (gfx950) DeepSeek Sparse Attention hot path.

Host code mirrors cppmega's Python surface (``sparse_mla_ops``,
``dsa_indexer_fused_patch``, top-k, ``index_cache_patch``,
``dsa_splitk_indexer_loss``, ``dsa_index_mask``) and calls the
hand-written HIP kernels of ``_lib/libdsa_hip.so`` through the C-ABI declared
in ``include/dsa_hip.h``.
"""
from . import _lib
from .dsa_fused_indexer_loss import FusedDSAIndexerLoss, apply_fused_indexer_loss_patch, fused_dsa_indexer_loss
from .dsa_indexer_fused_patch import (IndexScores, apply_dsa_indexer_fused_patch, compute_index_scores_fused_bf16,
                                      index_scores, index_scores_backward)
from .dsa_index_mask import scatter_topk_into_index_mask, topk_index_mask
from .dsa_splitk_indexer_loss import compute_dsa_indexer_loss_splitk, indexer_kl_loss, indexer_kl_loss_backward
from .dsa_topk import apply_dsa_topk_patch, fused_qk_topk_naive, indexer_topk, indexer_topk_streaming, topk_indices
from .index_cache_patch import IndexCacheSchedule, apply_index_cache_patch

__all__ = [
    "FusedDSAIndexerLoss",
    "IndexCacheSchedule",
    "IndexScores",
    "apply_dsa_indexer_fused_patch",
    "apply_dsa_topk_patch",
    "apply_fused_indexer_loss_patch",
    "apply_index_cache_patch",
    "compute_dsa_indexer_loss_splitk",
    "compute_index_scores_fused_bf16",
    "fused_dsa_indexer_loss",
    "fused_qk_topk_naive",
    "index_scores",
    "index_scores_backward",
    "indexer_kl_loss",
    "indexer_kl_loss_backward",
    "indexer_topk",
    "indexer_topk_streaming",
    "scatter_topk_into_index_mask",
    "topk_index_mask",
    "topk_indices",
]
