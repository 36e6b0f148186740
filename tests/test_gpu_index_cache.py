"""IndexCache on the GPU with a stand-in for Megatron's DSAttention whose
forward calls the dsa module's fused_qk_topk_naive (patched to the gfx950 one)
and SparseMLA, as Megatron's does.

Checked: every Full layer runs the indexer + top-k exactly once (no second
derivation pass), the cached indices are bit-identical to the causal
indexer_topk path on the same inputs, and a Shared layer's output equals the
SparseMLA output on the Full layer's indices.
"""
import types

import pytest
import torch

from cppmega_amd import index_cache_patch as icp
from cppmega_amd import synthetic
from cppmega_amd.dsa_topk import apply_dsa_topk_patch, indexer_topk
from cppmega_amd.sparse_mla_ops import sparse_mla_as_unfused_dsa

pytestmark = pytest.mark.gpu


class _Indexer:
    index_topk = 64
    pg_collection = None

    def __init__(self, qi, ki, wi):
        self.qi, self.ki, self.wi = qi, ki, wi

    def forward_before_topk(self, x, qr, packed):
        raise AssertionError("IndexCache must not re-derive the indices")


def _module(dev, S, calls):
    ninf = float("-inf")
    causal = torch.full((S, S), ninf, device=dev).triu(1)

    def megatron_topk(*a, **k):
        raise AssertionError("Megatron's torch top-k must not run")

    mod = types.SimpleNamespace(fused_qk_topk_naive=megatron_topk)
    apply_dsa_topk_patch(dsa_module=mod)

    class DSAttention:
        def __init__(self, indexer):
            self.indexer = indexer
            self.config = types.SimpleNamespace(kv_lora_rank=0, qk_pos_emb_head_dim=0, dsa_indexer_scoring_relu=True)
            self.softmax_scale = 128 ** -0.5

        def forward(self, query, key, value, attention_mask, x, qr, **kw):
            ix = self.indexer
            _, idx = mod.fused_qk_topk_naive(ix.qi, ix.ki, ix.wi, ix.index_topk, mask=causal, use_relu=True)
            calls.append(("full", idx))
            return sparse_mla_as_unfused_dsa(query, key, value, idx, self.softmax_scale)

    def run_sparse(**kw):
        calls.append(("shared", kw["topk_indices"]))
        out = sparse_mla_as_unfused_dsa(kw["query"], kw["key"], kw["value"], kw["topk_indices"], kw["softmax_scale"])
        return out, None

    mod.DSAttention = DSAttention
    mod._run_sparse_attention = run_sparse
    mod._ensure_sbhd = lambda t, name: (t, None)
    mod._normalize_dsattention_output_rank = lambda out, nd: out
    mod._build_dsattention_forward_mask = lambda **kw: (causal, None)
    mod._normalize_cp_comm_type = lambda t: t
    return mod


def test_index_cache_computes_once_and_shares(dev, monkeypatch):
    S, B, H, D, DV = 256, 2, 32, 128, 64
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0,3")
    monkeypatch.setattr(icp, "_SCHEDULE", None)
    ii = synthetic.indexer_inputs(B, S, 16, 64, seed=61)
    qi, ki, wi = ii["q"].to(dev), ii["k"].to(dev), ii["w"].to(dev)
    calls = []
    mod = _module(dev, S, calls)
    assert icp.apply_index_cache_patch(dsa_module=mod)
    layers = [mod.DSAttention(_Indexer(qi, ki, wi)) for _ in range(6)]
    g = torch.Generator().manual_seed(62)
    query = (torch.randn((S, B, H, D), generator=g) * 0.5).to(torch.bfloat16).to(dev)
    key = (torch.randn((S, B, 1, D), generator=g) * 0.5).to(torch.bfloat16).to(dev).expand(S, B, H, D)
    value = key[..., :DV]
    x = torch.zeros(S, B, 8, device=dev)
    outs = [layer.forward(query, key, value, None, x, x) for layer in layers]
    kinds = [c[0] for c in calls]
    assert kinds == ["full", "shared", "shared", "full", "shared", "shared"]
    ref = indexer_topk(qi, ki, wi, 64, causal=True).to(torch.int64)
    full_idx = calls[0][1]
    assert torch.equal(full_idx, ref)
    for c in calls[1:3] + calls[4:]:
        assert c[1] is calls[0][1] or torch.equal(c[1], full_idx)
    for o in outs[1:]:
        assert torch.equal(o, outs[0])          # same indices, same inputs: same attention output
    sched = icp.get_schedule()
    assert sched.captured == 2 and sched.rederived == 0


def test_index_cache_with_the_indexer_loss_path(dev, monkeypatch):
    """Megatron's training path: the Full layer takes its indices from
    dsa.FusedDSAIndexerLoss.apply, with this package's top-k, indexer-loss and
    IndexCache patches all installed.  Each Full layer runs one masked indexer +
    top-k (captured, nothing re-derived), the cached picks are bit-identical
    to the causal indexer_topk, the Shared layers' outputs equal SparseMLA on
    those picks, and the loss's gradient reaches the indexer inputs."""
    from cppmega_amd import dsa_fused_indexer_loss as fil

    S, B, H, D, DV = 256, 2, 32, 128, 64
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0,3")
    monkeypatch.setattr(icp, "_SCHEDULE", None)
    monkeypatch.setattr(fil, "_DSA_MODULE", None)
    ii = synthetic.indexer_inputs(B, S, 16, 64, seed=63)
    qi = ii["q"].to(dev).requires_grad_()
    ki = ii["k"].to(dev).requires_grad_()
    wi = ii["w"].to(dev).requires_grad_()
    calls = []
    mod = _module(dev, S, calls)
    causal = mod._build_dsattention_forward_mask()[0]
    mod.FusedDSAIndexerLoss = type("MegatronFusedDSAIndexerLoss", (), {})
    losses = []

    def forward(self, query, key, value, attention_mask, x, qr, **kw):
        ix = self.indexer
        idx, loss = mod.FusedDSAIndexerLoss.apply(ix.qi, ix.wi, ix.ki, query, key, self.softmax_scale,
                                                  ix.index_topk, 1.0, causal, True, None)
        losses.append(loss)
        calls.append(("full", idx))
        return sparse_mla_as_unfused_dsa(query, key, value, idx, self.softmax_scale)

    mod.DSAttention.forward = forward
    assert fil.apply_fused_indexer_loss_patch(dsa_module=mod)
    assert icp.apply_index_cache_patch(dsa_module=mod)
    layers = [mod.DSAttention(_Indexer(qi, ki, wi)) for _ in range(6)]
    g = torch.Generator().manual_seed(64)
    query = (torch.randn((S, B, H, D), generator=g) * 0.5).to(torch.bfloat16).to(dev)
    key = (torch.randn((S, B, 1, D), generator=g) * 0.5).to(torch.bfloat16).to(dev).expand(S, B, H, D)
    value = key[..., :DV]
    x = torch.zeros(S, B, 8, device=dev)
    outs = [layer.forward(query, key, value, None, x, x) for layer in layers]
    assert [c[0] for c in calls] == ["full", "shared", "shared", "full", "shared", "shared"]
    sched = icp.get_schedule()
    assert sched.captured == 2 and sched.rederived == 0
    with torch.no_grad():
        ref = indexer_topk(qi.detach(), ki.detach(), wi.detach(), 64, causal=True).to(torch.int64)
    full_idx = calls[0][1]
    assert torch.equal(full_idx, ref)
    for c in calls[1:3] + calls[4:]:
        assert torch.equal(c[1], full_idx)
    on_picks = sparse_mla_as_unfused_dsa(query, key, value, full_idx, 128 ** -0.5)
    for o in outs:
        assert torch.equal(o, on_picks)
    assert len(losses) == 2 and all(bool(torch.isfinite(l)) for l in losses)
    losses[0].backward()
    for t in (qi, ki, wi):
        assert t.grad is not None and bool(torch.isfinite(t.grad.float()).all()) and bool(t.grad.abs().sum() > 0)
    assert mod.FusedDSAIndexerLoss is fil.FusedDSAIndexerLoss
