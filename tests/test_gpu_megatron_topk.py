"""GPU tests of the Megatron top-k binding: fused_qk_topk_naive with masks,
varlen windows and key positions, its graph capture, and apply_dsa_topk_patch.

Bars: the returned scores equal the unmasked indexer scores plus the mask,
bit for bit, on every admissible element and are -inf elsewhere; the indices
are bit-exact with the oracle's deterministic top-k over the admissible
columns of those same scores; graph replays equal the eager call.
"""
import types

import numpy as np
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.dsa_indexer_fused_patch import CAUSAL_LOWER, CAUSAL_NONE, index_scores
from cppmega_amd.dsa_topk import apply_dsa_topk_patch, fused_qk_topk_naive, indexer_topk
from oracle import indexer as oix
from oracle import topk as otk

pytestmark = pytest.mark.gpu

NINF = float("-inf")


def _inputs(dev, S, B=2, H=16, D=64, seed=21, Sk=None):
    inp = synthetic.indexer_inputs(B, S, H, D, seed=seed)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    if Sk is not None and Sk != S:
        g = torch.Generator().manual_seed(seed + 1)
        k = torch.randn((Sk, B, D), generator=g).to(torch.bfloat16).to(dev)
    return q, k, w


def _check(scores, idx, full, admissible, K):
    """scores == full + mask on admissible elements (bit for bit), -inf elsewhere;
    idx == the oracle's top-K over the admissible columns of `scores`."""
    B, S, Sk = scores.shape
    sc = scores.cpu()
    adm = admissible.expand(B, S, Sk)
    assert torch.isneginf(sc[~adm]).all(), "non-admissible elements must be -inf"
    assert torch.equal(sc[adm], full.cpu()[adm]), "admissible scores differ from indexer + mask"
    ref = otk.topk_ascending(sc.numpy().reshape(B * S, Sk), K, admissible=adm.reshape(B * S, Sk).numpy())
    np.testing.assert_array_equal(idx.cpu().numpy().reshape(B * S, K), ref)


def test_causal_mask_is_the_lower_triangle_path(dev):
    """A causal float mask: scores equal the lower-triangle indexer's bit for
    bit (same MFMA order), -inf above the diagonal, and the indices equal the
    causal indexer_topk path's."""
    S, K = 300, 64
    q, k, w = _inputs(dev, S)
    mask = torch.full((S, S), NINF, device=dev).triu(1)
    scores, idx = fused_qk_topk_naive(q, k, w, K, mask=mask)
    assert idx.dtype == torch.int64 and idx.shape == (2, S, K)
    low, idx_low = indexer_topk(q, k, w, K, causal=True, return_scores=True)
    tri = torch.ones(S, S, dtype=torch.bool).tril()
    assert torch.equal(scores.cpu()[:, tri], low.cpu()[:, tri])
    assert torch.isneginf(scores.cpu()[:, ~tri]).all()
    assert torch.equal(idx.cpu(), idx_low.cpu().to(torch.int64))
    ref = oix.compute_index_scores(*(t.cpu() for t in (q, w, k)))
    err = (scores.cpu()[:, tri] - ref[:, tri]).abs().max() / ref[:, tri].abs().max()
    assert float(err) < 1e-3


@pytest.mark.parametrize("S,Sk,H,D", [(200, 200, 16, 64), (130, 257, 32, 64), (96, 96, 64, 128)])
def test_mask_with_holes_and_bias(dev, S, Sk, H, D):
    """A mask with random -inf holes, finite biases, rows with fewer admissible
    columns than K (holes inside the span must not be picked) and an all -inf row."""
    K = 48
    q, k, w = _inputs(dev, S, H=H, D=D, Sk=Sk, seed=S + H)
    g = torch.Generator().manual_seed(S)
    mask = torch.randn((S, Sk), generator=g) * 0.5
    mask[torch.rand((S, Sk), generator=g) < 0.4] = NINF
    mask[5, :] = NINF                       # nothing admissible
    mask[7, :] = NINF
    mask[7, 3:40:3] = 0.0                   # 13 admissible columns, holes between them
    mask = mask.to(dev)
    scores, idx = fused_qk_topk_naive(q, k, w, K, mask=mask)
    full = index_scores(q, w, k, causal=CAUSAL_NONE) + mask
    _check(scores, idx, full, torch.isfinite(mask.cpu())[None], min(K, S))
    assert (idx[:, 5] == -1).all()
    assert (idx[:, 7, 13:] == -1).all() and (idx[:, 7, :13] >= 0).all()


def test_batched_mask(dev):
    """A [b, 1, sq, sk] mask (one per batch) is applied per batch."""
    S, K = 160, 32
    q, k, w = _inputs(dev, S)
    m0 = torch.full((S, S), NINF).triu(1)
    m1 = torch.full((S, S), NINF).triu(1) + torch.full((S, S), NINF).tril(-50)   # sliding window of 50
    mask = torch.stack([m0, m1]).unsqueeze(1).to(dev)
    scores, idx = fused_qk_topk_naive(q, k, w, K, mask=mask)
    full = index_scores(q, w, k, causal=CAUSAL_NONE) + mask[:, 0]
    _check(scores, idx, full, torch.isfinite(mask[:, 0].cpu()), K)


def test_varlen_windows_and_key_positions(dev):
    """Packed sequences: varlen windows per query row (three sequences, causal
    inside each), then the same windows through permuted key positions."""
    S, K = 240, 40
    q, k, w = _inputs(dev, S)
    bounds = [0, 70, 171, 240]
    starts = torch.zeros(S, dtype=torch.int32)
    ends = torch.zeros(S, dtype=torch.int32)
    for a, e in zip(bounds[:-1], bounds[1:]):
        starts[a:e] = a
        ends[a:e] = torch.arange(a + 1, e + 1, dtype=torch.int32)
    scores, idx = fused_qk_topk_naive(q, k, w, K, varlen_starts=starts.to(dev), varlen_ends=ends.to(dev))
    col = torch.arange(S)
    adm = (col[None, :] >= starts[:, None].long()) & (col[None, :] < ends[:, None].long())
    full = index_scores(q, w, k, causal=CAUSAL_NONE)
    _check(scores, idx, full, adm[None], K)
    # key positions: column s holds position perm[s]; admissible iff start <= perm[s] < end
    perm = torch.randperm(S, generator=torch.Generator().manual_seed(3))
    scores_p, idx_p = fused_qk_topk_naive(q, k, w, K, varlen_starts=starts.to(dev), varlen_ends=ends.to(dev),
                                          key_positions=perm.to(dev))
    adm_p = (perm[None, :] >= starts[:, None].long()) & (perm[None, :] < ends[:, None].long())
    _check(scores_p, idx_p, full, adm_p[None], K)


def test_no_mask_keeps_every_column(dev):
    S, K = 96, 40
    q, k, w = _inputs(dev, S)
    scores, idx = fused_qk_topk_naive(q, k, w, K)
    assert torch.equal(scores, index_scores(q, w, k, causal=CAUSAL_NONE))
    ref = otk.topk_ascending(scores.cpu().numpy().reshape(2 * S, S), K)
    np.testing.assert_array_equal(idx.cpu().numpy().reshape(2 * S, K), ref)


def test_masked_call_replays_in_a_graph(dev):
    """No host synchronisation: the masked call captures in a HIP graph; three
    replays, each after an eager call on other inputs, equal the eager result."""
    S, K = 256, 64
    q, k, w = _inputs(dev, S)
    mask = torch.full((S, S), NINF, device=dev).triu(1)
    mask[:, 10:20] = NINF
    ref_scores, ref_idx = fused_qk_topk_naive(q, k, w, K, mask=mask)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fused_qk_topk_naive(q, k, w, K, mask=mask)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        g_scores, g_idx = fused_qk_topk_naive(q, k, w, K, mask=mask)
    q2, k2, w2 = _inputs(dev, S, seed=99)
    for _ in range(3):
        fused_qk_topk_naive(q2, k2, w2, K, mask=mask)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_scores, ref_scores) and torch.equal(g_idx, ref_idx)


def test_apply_dsa_topk_patch_rebinds_the_module(dev):
    calls = []

    def megatron_naive(*a, **kw):
        calls.append(1)
        raise AssertionError("the torch top-k must not run after the patch")

    mod = types.SimpleNamespace(fused_qk_topk_naive=megatron_naive)
    assert apply_dsa_topk_patch(dsa_module=mod)
    assert apply_dsa_topk_patch(dsa_module=mod)          # idempotent
    S, K = 128, 32
    q, k, w = _inputs(dev, S)
    mask = torch.full((S, S), NINF, device=dev).triu(1)
    scores, idx = mod.fused_qk_topk_naive(q, k, w, K, mask=mask, use_relu=True)
    ref_s, ref_i = fused_qk_topk_naive(q, k, w, K, mask=mask)
    assert torch.equal(scores, ref_s) and torch.equal(idx, ref_i) and not calls


def test_nam56r_full_square_indexer(dev):
    """The full-square mode Megatron's _compute_index_scores runs, at the
    reference test's NAM56R shape (tests/test_dsa_indexer_fused_patch.py:74-92:
    h=32, d=64, sq=sk=4096, bf16 weights, rel < 5e-3), on 128 sampled rows of
    each batch against the oracle, plus finiteness of the whole matrix."""
    S, B, H, D = 4096, 2, 32, 64
    inp = synthetic.indexer_inputs(B, S, H, D, seed=74, w_dtype=torch.bfloat16)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    got = index_scores(q, w, k, causal=CAUSAL_NONE)
    assert bool(torch.isfinite(got).all())
    rows = torch.randperm(S, generator=torch.Generator().manual_seed(1))[:128].sort().values
    ref = oix.compute_index_scores(inp["q"][rows], inp["w"][rows], inp["k"])
    g = got[:, rows].cpu()
    rel = float((g - ref).abs().max() / ref.abs().max())
    assert rel < 5e-3, rel
    low = index_scores(q, w, k, causal=CAUSAL_LOWER, out=torch.zeros_like(got))
    tri = torch.ones(S, S, dtype=torch.bool, device=dev).tril()
    assert torch.equal(low[:, tri], got[:, tri])


@pytest.mark.parametrize("R,B,S,Sk", [(1, 2, 96, 128), (2, 2, 64, 77), (1, 3, 40, 300)])
def test_mask_windows_kernel_matches_oracle(dev, R, B, S, Sk):
    """dsa_mask_windows: first / one-past-last finite column and the plain flag
    of every row, bit-exact with the oracle, over causal rows, sliding windows,
    holes, finite biases, -0.0, +inf / NaN entries and all -inf rows, for one
    shared mask and one per batch, 16-byte (Sk % 4 == 0) and scalar rows."""
    from cppmega_amd.dsa_topk import mask_windows

    g = torch.Generator().manual_seed(R * 100 + S + Sk)
    m = torch.full((R, S, Sk), NINF)
    for r in range(R):
        for t in range(S):
            kind = int(torch.randint(0, 6, (1,), generator=g))
            a = int(torch.randint(0, Sk, (1,), generator=g))
            e = int(torch.randint(a, Sk + 1, (1,), generator=g))
            if kind == 0:
                m[r, t, :min(t + 1, Sk)] = 0.0                 # causal, plain
            elif kind == 1:
                m[r, t, a:e] = 0.0                              # window, plain (possibly empty)
            elif kind == 2:
                m[r, t, a:e] = 0.0
                if e - a > 2:
                    m[r, t, (a + e) // 2] = NINF                # a hole
            elif kind == 3:
                m[r, t, a:e] = torch.randn(e - a, generator=g)  # finite biases
            elif kind == 4:
                m[r, t, a:e] = 0.0
                m[r, t, a] = -0.0                               # -0.0 is not +0.0
                if e < Sk:
                    m[r, t, e] = float("nan") if t % 2 else float("inf")
            # kind 5: all -inf
    st, en, pl = mask_windows(m.to(dev), B, S, Sk)
    rs, re_, rp = otk.mask_windows(m.numpy())
    exp = (lambda a: np.broadcast_to(a, (B, S))) if R == 1 else (lambda a: a)
    np.testing.assert_array_equal(st.cpu().numpy(), exp(rs))
    np.testing.assert_array_equal(en.cpu().numpy(), exp(re_))
    np.testing.assert_array_equal(pl.cpu().numpy(), exp(rp))


def test_topk_finalize_matches_oracle(dev):
    """dsa_topk_finalize: int32 picks -> int64, with -inf picks dropped (the rest
    ascending, -1 padded) on rows not flagged plain, and plain rows copied."""
    from cppmega_amd.dsa_topk import finalize_picks, topk_indices

    B, S, Sk, K = 2, 70, 150, 24
    g = torch.Generator().manual_seed(7)
    scores = torch.randn((B, S, Sk), generator=g)
    scores[torch.rand((B, S, Sk), generator=g) < 0.7] = NINF     # many rows with fewer finite than K
    scores[0, 3] = NINF
    plain = (torch.rand((B, S), generator=g) < 0.3).to(torch.int32)
    idx = topk_indices(scores.to(dev), K, causal=False)
    out = finalize_picks(scores.to(dev), idx, plain.to(dev))
    assert out.dtype == torch.int64
    ref = otk.drop_masked_picks(scores.numpy().reshape(B * S, Sk), idx.cpu().numpy().reshape(B * S, K),
                                plain=plain.numpy().reshape(-1))
    np.testing.assert_array_equal(out.cpu().numpy().reshape(B * S, K), ref)
    out2 = finalize_picks(scores.to(dev), idx)                   # no flags: every row checked
    ref2 = otk.drop_masked_picks(scores.numpy().reshape(B * S, Sk), idx.cpu().numpy().reshape(B * S, K))
    np.testing.assert_array_equal(out2.cpu().numpy().reshape(B * S, K), ref2)


def test_causal_mask_path_reads_no_mask_and_matches_lower_triangle(dev):
    """Megatron's causal float mask: every row is plain, so the window-mode
    indexer does not read the mask; scores equal the lower-triangle indexer's
    (-inf above the diagonal) and the picks equal the causal indexer_topk, bit
    for bit; the same call with a mask that has one finite bias (not plain)
    still adds it."""
    S, K = 256, 64
    q, k, w = _inputs(dev, S, seed=31)
    causal = torch.full((S, S), NINF, device=dev).triu(1)
    scores, idx = fused_qk_topk_naive(q, k, w, K, mask=causal)
    low = index_scores(q, w, k, causal=CAUSAL_LOWER)
    tri = torch.ones(S, S, dtype=torch.bool, device=dev).tril()
    assert torch.equal(scores[:, tri], low[:, tri]) and torch.isneginf(scores[:, ~tri]).all()
    assert torch.equal(idx, indexer_topk(q, k, w, K, causal=True).to(torch.int64))
    biased = causal.clone()
    biased[100, 50] = 0.25
    s2, _ = fused_qk_topk_naive(q, k, w, K, mask=biased)
    assert torch.equal(s2[:, 100, 50], low[:, 100, 50] + 0.25)
    assert torch.equal(s2[:, 101:], scores[:, 101:])
