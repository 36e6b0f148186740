"""One DSA layer step (indexer, top-k, SparseMLA fwd + bwd) captured in a HIP
graph: every replay, with eager steps and synchronisations in between, must
reproduce the eager outputs bit for bit (the kernels are deterministic and
use no memset nodes)."""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.dsa_indexer_fused_patch import CAUSAL_LOWER, index_scores
from cppmega_amd.dsa_topk import topk_indices
from cppmega_amd.sparse_mla_ops import sparse_mla_bwd, sparse_mla_fwd_interface

pytestmark = pytest.mark.gpu


def test_layer_step_graph_replays_match_eager(dev):
    B, S, H, D, DV, K = 1, 512, 32, 128, 64, 64
    mla = synthetic.sparse_mla_inputs(B, S, H, D, DV, K, std=0.5, seed=77)
    ix = synthetic.indexer_inputs(B, S, 16, 64, seed=78)
    q, kv, idx, do = (mla[k].to(dev) for k in ("q", "kv", "indices", "do"))
    iq, ik, iw = ix["q"].to(dev), ix["k"].to(dev), ix["w"].to(dev)
    scale = D ** -0.5

    def step():
        scores = index_scores(iq, iw, ik, use_relu=True, causal=CAUSAL_LOWER)
        sel = topk_indices(scores, K, causal=True)
        out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=scale, d_v=DV)
        dq, dkv = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale)
        return sel, out, lse, dq, dkv

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = step()
    for _ in range(4):
        eager = step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(gout, eager):
            assert torch.equal(a, b)
