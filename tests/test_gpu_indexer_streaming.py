"""GPU tests of the streaming indexer + top-k (dsa_indexer_topk_streaming):
query rows in chunks through a bounded scratch, no [b, sq, sk] score matrix.

Bar: bit-exact.  The indices equal the deterministic top-k of the full score
matrix (topk_indices over index_scores, itself bit-exact with the oracle on
identical fp32 scores), whatever the chunk size, and the returned top-k
scores equal the full matrix's entries at those indices.
"""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.dsa_indexer_fused_patch import CAUSAL_LOWER, CAUSAL_NONE, index_scores
from cppmega_amd.dsa_topk import indexer_topk_streaming, topk_indices
from cppmega_amd.sparse_mla_ops import tensorwise_quantize

pytestmark = pytest.mark.gpu


def _full(q, k, w, K, causal, q_scale=None, k_scale=None):
    sc = index_scores(q, w, k, causal=CAUSAL_LOWER if causal else CAUSAL_NONE, q_scale=q_scale, k_scale=k_scale,
                      out=torch.full((q.shape[1], q.shape[0], k.shape[0]), float("-inf"), device=q.device))
    return sc, topk_indices(sc, K, causal=causal)


def _gathered(sc, idx):
    v = sc.gather(-1, idx.clamp(min=0).long())
    return torch.where(idx >= 0, v, torch.full_like(v, float("-inf")))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("chunk_rows", [1, 7, 64, 10000])
def test_streaming_equals_full(dev, causal, chunk_rows):
    S, B, H, D, K = 300, 2, 16, 64, 64
    inp = synthetic.indexer_inputs(B, S, H, D, seed=91)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    sc, ref = _full(q, k, w, K, causal)
    idx, vals = indexer_topk_streaming(q, k, w, K, causal=causal, return_scores=True, chunk_rows=chunk_rows)
    assert idx.dtype == torch.int32 and idx.shape == (B, S, K)
    assert torch.equal(idx, ref)
    assert torch.equal(vals, _gathered(sc, ref))


def test_streaming_long_keys(dev):
    """Keys past one top-k pass (40000 > 32768): each chunk's top-k runs its
    segment passes in the scratch after the chunk's scores; equal to the full
    matrix's top-k, itself checked against the oracle here."""
    import numpy as np
    from oracle import topk as otk
    Sq, Sk, B, H, D, K = 40, 40000, 2, 16, 64, 512
    inp = synthetic.indexer_inputs(B, Sk, H, D, seed=93)
    q, k, w = inp["q"][:Sq].to(dev), inp["k"].to(dev), inp["w"][:Sq].to(dev)
    sc, ref = _full(q.contiguous(), k, w.contiguous(), K, False)
    np.testing.assert_array_equal(ref.cpu().reshape(B * Sq, K).numpy(),
                                  otk.topk_ascending(sc.cpu().reshape(B * Sq, Sk).numpy(), K))
    for chunk_rows in (7, 40):
        idx, vals = indexer_topk_streaming(q.contiguous(), k, w.contiguous(), K, causal=False, return_scores=True,
                                           chunk_rows=chunk_rows)
        assert torch.equal(idx, ref)
        assert torch.equal(vals, _gathered(sc, ref))


def test_streaming_e4m3_wide_heads(dev):
    """cfg5's indexer form (e4m3, h = 64, d = 128) at a small length, in 3-row chunks."""
    S, B, H, D, K = 200, 1, 64, 128, 96
    inp = synthetic.indexer_inputs(B, S, H, D, seed=92)
    q8, qs = tensorwise_quantize(inp["q"].to(dev))
    k8, ks = tensorwise_quantize(inp["k"].to(dev))
    w = inp["w"].to(dev)
    sc, ref = _full(q8, k8, w, K, True, q_scale=qs, k_scale=ks)
    idx = indexer_topk_streaming(q8, k8, w, K, q_scale=qs, k_scale=ks, chunk_rows=3)
    assert torch.equal(idx, ref)


def test_cfg3_streaming_full_scale(dev):
    """cfg3 (b=2, s=4096, h=16, d=64, top-256) through a 16 MiB scratch (512-row
    chunks): bit-exact with the full lower-triangle scores + top-k."""
    S, B, H, D, K = 4096, 2, 16, 64, 256
    inp = synthetic.indexer_inputs(B, S, H, D, seed=1235)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    sc, ref = _full(q, k, w, K, True)
    del sc
    idx = indexer_topk_streaming(q, k, w, K, max_scratch_bytes=16 << 20)
    assert torch.equal(idx, ref)


def test_cfg5_streaming_without_the_score_matrix(dev):
    """cfg5 indexer (b=1, s=16384, h=64, d=128, e4m3, top-2048) through a
    64 MiB scratch: the peak allocation stays far below the 1 GiB score matrix,
    and three 256-row slices (first, middle, last) are bit-exact with the full
    rows scored separately and selected in the causal window."""
    S, B, H, D, K = 16384, 1, 64, 128, 2048
    gen = torch.Generator(device=dev).manual_seed(55)
    q = torch.randn((S, B, H, D), generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn((S, B, D), generator=gen, device=dev).to(torch.bfloat16)
    w = torch.randn((S, B, H), generator=gen, device=dev) / H ** 0.5
    q8, qs = tensorwise_quantize(q)
    k8, ks = tensorwise_quantize(k)
    del q, k
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    idx = indexer_topk_streaming(q8, k8, w, K, q_scale=qs, k_scale=ks, max_scratch_bytes=64 << 20)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    assert peak < 200 << 20, f"peak {peak >> 20} MiB"
    for r0 in (0, 8000, S - 256):
        sub = index_scores(q8[r0:r0 + 256], w[r0:r0 + 256], k8, causal=CAUSAL_NONE, q_scale=qs, k_scale=ks)
        ref = topk_indices(sub, K, causal=True, causal_offset=r0, seq_q=256)
        assert torch.equal(idx[:, r0:r0 + 256], ref), f"rows {r0}..{r0 + 256}"


def test_streaming_replays_in_a_graph(dev):
    """Several chunks (several launches) captured once; three replays after eager
    calls on other inputs equal the eager result."""
    S, B, H, D, K = 512, 2, 16, 64, 64
    inp = synthetic.indexer_inputs(B, S, H, D, seed=93)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    ref = indexer_topk_streaming(q, k, w, K, chunk_rows=100)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        indexer_topk_streaming(q, k, w, K, chunk_rows=100)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = indexer_topk_streaming(q, k, w, K, chunk_rows=100)
    other = synthetic.indexer_inputs(B, S, H, D, seed=94)
    for _ in range(3):
        indexer_topk_streaming(other["q"].to(dev), other["k"].to(dev), other["w"].to(dev), K, chunk_rows=100)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
