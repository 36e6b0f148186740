"""GPU tests of the fused indexer + top-k (dsa_indexer_topk_fused): each query
row's running top-k kept on chip while its keys are scored, no score matrix.

Bar: bit-exact.  The indices equal the deterministic top-k of the full score
matrix (topk_indices over index_scores, itself bit-exact with the oracle on
identical fp32 scores), and the returned scores equal the full matrix's
entries at those indices.  The row lists overflow and run their selection
only on rows longer than the list capacity (896 candidates at h = 16, 1792 at
h = 32, 3584 at h = 64), so the long-row cases below are the ones that
exercise it, including at the largest top-k each shape takes.
"""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.dsa_indexer_fused_patch import CAUSAL_LOWER, CAUSAL_NONE, index_scores
from cppmega_amd.dsa_topk import indexer_topk_fused, indexer_topk_fused_max_topk, indexer_topk_streaming, topk_indices
from cppmega_amd.sparse_mla_ops import tensorwise_quantize

pytestmark = pytest.mark.gpu


def _full(q, k, w, K, causal, q_scale=None, k_scale=None):
    sc = index_scores(q, w, k, causal=CAUSAL_LOWER if causal else CAUSAL_NONE, q_scale=q_scale, k_scale=k_scale,
                      out=torch.full((q.shape[1], q.shape[0], k.shape[0]), float("-inf"), device=q.device))
    return sc, topk_indices(sc, K, causal=causal)


def _gathered(sc, idx):
    v = sc.gather(-1, idx.clamp(min=0).long())
    return torch.where(idx >= 0, v, torch.full_like(v, float("-inf")))


def _check(q, k, w, K, causal, **kw):
    sc, ref = _full(q, k, w, K, causal, **kw)
    idx, vals = indexer_topk_fused(q, k, w, K, causal=causal, return_scores=True, **kw)
    assert idx.dtype == torch.int32 and idx.shape == ref.shape
    bad = (idx != ref).any(dim=-1)
    assert not bad.any(), f"{int(bad.sum())} rows differ; first (b, t) {bad.nonzero()[0].tolist()}"
    assert torch.equal(vals, _gathered(sc, ref))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H,D,K", [(16, 64, 64), (32, 64, 200), (64, 128, 96), (16, 128, 300)])
def test_fused_equals_full(dev, causal, H, D, K):
    S, B = 300, 2
    inp = synthetic.indexer_inputs(B, S, H, D, seed=191)
    _check(inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev), K, causal)


@pytest.mark.parametrize("H,D", [(16, 64), (32, 64), (64, 128)])
@pytest.mark.parametrize("kind", ["small", "max"])
def test_fused_long_rows_select(dev, H, D, kind):
    """Rows of 7000 keys: each row's list overflows and runs its selection
    several times (at the largest top-k, every 64 new candidates)."""
    Sq, Sk, B = 24, 7000, 2
    K = 64 if kind == "small" else indexer_topk_fused_max_topk(H, D)
    inp = synthetic.indexer_inputs(B, Sk, H, D, seed=193)
    q, k, w = inp["q"][:Sq].contiguous().to(dev), inp["k"].to(dev), inp["w"][:Sq].contiguous().to(dev)
    _check(q, k, w, K, False)


def test_fused_ties_prefer_lower_columns(dev):
    """Keys repeating 5 distinct rows give every row runs of exactly equal
    scores, across selections: ties go to the lower column as in topk_indices."""
    Sq, Sk, B, H, D, K = 16, 2500, 1, 16, 64, 100
    inp = synthetic.indexer_inputs(B, Sk, H, D, seed=195)
    k = inp["k"][:5].repeat(Sk // 5, 1, 1).contiguous()
    q, w = inp["q"][:Sq].contiguous(), inp["w"][:Sq].contiguous()
    _check(q.to(dev), k.to(dev), w.to(dev), K, False)


def test_fused_negative_weights_and_zero_scores(dev):
    """Weights of both signs, and q / k shifted so that the ReLU zeroes about
    85% of the head products: several percent of the scores are exactly +0 or
    -0, which rank equal (ties to the lower column)."""
    Sq, Sk, B, H, D, K = 40, 3000, 2, 16, 64, 256
    inp = synthetic.indexer_inputs(B, Sk, H, D, seed=197)
    q = (inp["q"][:Sq].float() - 0.3).to(torch.bfloat16).contiguous()
    k = (inp["k"].float() + 0.5).to(torch.bfloat16).contiguous()
    w = inp["w"][:Sq].contiguous()
    sc, _ = _full(q.to(dev), k.to(dev), w.to(dev), K, False)
    assert (sc == 0).float().mean() > 0.02
    _check(q.to(dev), k.to(dev), w.to(dev), K, False)


def test_fused_e4m3(dev):
    """cfg5's indexer form (e4m3, h = 64, d = 128), causal, rows past the list capacity."""
    S, B, H, D, K = 4000, 1, 64, 128, 512
    inp = synthetic.indexer_inputs(B, S, H, D, seed=192)
    q8, qs = tensorwise_quantize(inp["q"].to(dev))
    k8, ks = tensorwise_quantize(inp["k"].to(dev))
    _check(q8, k8, inp["w"].to(dev), K, True, q_scale=qs, k_scale=ks)


def test_fused_short_rows_pad(dev):
    """Fewer keys than top-k: every key, then -1 (and -inf scores)."""
    Sq, Sk, B, H, D, K = 10, 40, 2, 32, 64, 64
    inp = synthetic.indexer_inputs(B, Sk, H, D, seed=198)
    q, k, w = inp["q"][:Sq].contiguous().to(dev), inp["k"].to(dev), inp["w"][:Sq].contiguous().to(dev)
    _check(q, k, w, K, False)
    _check(q, k, w, K, True)


def test_cfg3_fused_full_scale(dev):
    """cfg3 (b=2, s=4096, h=16, d=64, top-256): bit-exact with the full
    lower-triangle scores + top-k, scores included."""
    S, B, H, D, K = 4096, 2, 16, 64, 256
    inp = synthetic.indexer_inputs(B, S, H, D, seed=1235)
    _check(inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev), K, True)


def test_fused_replays_in_a_graph(dev):
    """One capture; three replays after eager calls on other inputs equal the eager result."""
    S, B, H, D, K = 1200, 2, 16, 64, 64
    inp = synthetic.indexer_inputs(B, S, H, D, seed=93)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    ref = indexer_topk_fused(q, k, w, K)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        indexer_topk_fused(q, k, w, K)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = indexer_topk_fused(q, k, w, K)
    other = synthetic.indexer_inputs(B, S, H, D, seed=94)
    for _ in range(3):
        indexer_topk_fused(other["q"].to(dev), other["k"].to(dev), other["w"].to(dev), K)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, ref)


def test_fused_nan_and_inf_scores(dev):
    """Without the ReLU (which zeroes NaN products here), a key row of +inf and one
    of NaN make scores +inf and NaN; NaN ranks as +inf with ties to the lower
    column, as in topk_indices."""
    Sq, Sk, B, H, D, K = 12, 2000, 1, 16, 64, 64
    inp = synthetic.indexer_inputs(B, Sk, H, D, seed=199)
    k = inp["k"].clone()
    k[700] = float("inf")
    k[1300] = float("nan")
    q, w = inp["q"][:Sq].contiguous().abs().to(dev), inp["w"][:Sq].contiguous().abs().to(dev)
    k = k.to(dev)
    sc = index_scores(q, w, k, use_relu=False, causal=CAUSAL_NONE)
    assert torch.isnan(sc).any() and torch.isinf(sc).any()
    ref = topk_indices(sc, K, causal=False)
    idx, vals = indexer_topk_fused(q, k, w, K, use_relu=False, causal=False, return_scores=True)
    assert torch.equal(idx, ref)
    g = _gathered(sc, ref)
    assert torch.equal(vals.isnan(), g.isnan()) and torch.equal(vals.nan_to_num(), g.nan_to_num())


def test_streaming_without_scratch_is_fused(dev):
    """indexer_topk_streaming(max_scratch_bytes=0) takes the fused path (same
    result), and refuses a top-k the fused path cannot hold."""
    S, B, H, D, K = 600, 2, 16, 64, 100
    inp = synthetic.indexer_inputs(B, S, H, D, seed=201)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    _, ref = _full(q, k, w, K, True)
    assert torch.equal(indexer_topk_streaming(q, k, w, K, max_scratch_bytes=0), ref)
    with pytest.raises(ValueError):
        indexer_topk_streaming(q, k, w, indexer_topk_fused_max_topk(H, D) + 1, max_scratch_bytes=0)
