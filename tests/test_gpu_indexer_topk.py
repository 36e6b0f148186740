"""GPU parity of the indexer-score, top-k and FP8-quantiser HIP kernels.

Bars: indexer scores within fp32 reassociation error of the oracle
(rel 1e-3 of the row scale, as the reference test uses); top-k indices
bit-exact against the oracle given the same fp32 scores; e4m3 quantisation
bit-exact (data and scale_inv) against the oracle.
"""
import numpy as np
import pytest
import torch

from cppmega_amd import compute_index_scores_fused_bf16, index_scores, indexer_topk, topk_indices
from cppmega_amd.dsa_topk import fused_qk_topk_naive
from cppmega_amd.sparse_mla_ops import tensorwise_quantize
from cppmega_amd import synthetic
from oracle import fp8 as ofp8
from oracle import indexer as oix
from oracle import topk as otk

pytestmark = pytest.mark.gpu


def _rel_err(a, e):
    a, e = a.float().cpu(), e.float().cpu()
    fin = torch.isfinite(e)
    return float((a[fin] - e[fin]).abs().max() / e[fin].abs().max().clamp_min(1e-6))


@pytest.mark.parametrize("S,B,H,D,wdt", [
    (128, 2, 8 * 2, 64, torch.bfloat16),
    (200, 1, 16, 64, torch.float32),
    (96, 2, 32, 64, torch.float32),
    (64, 1, 64, 64, torch.float32),
    (72, 1, 16, 128, torch.float32),
    (130, 1, 64, 128, torch.bfloat16),
])
def test_indexer_scores_match_oracle(dev, S, B, H, D, wdt):
    inp = synthetic.indexer_inputs(B, S, H, D, seed=3, w_dtype=wdt)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    got = compute_index_scores_fused_bf16(q, w, k, use_relu=True)
    ref = oix.compute_index_scores(inp["q"], inp["w"], inp["k"], use_relu=True)
    assert got.shape == (B, S, S) and got.dtype == torch.float32
    assert _rel_err(got, ref) < 1e-3
    got_nr = compute_index_scores_fused_bf16(q, w, k, use_relu=False)
    ref_nr = oix.compute_index_scores(inp["q"], inp["w"], inp["k"], use_relu=False)
    assert _rel_err(got_nr, ref_nr) < 1e-3


def test_indexer_causal_modes(dev):
    S, B, H, D = 300, 2, 16, 64
    inp = synthetic.indexer_inputs(B, S, H, D, seed=5)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    ref = oix.compute_index_scores(inp["q"], inp["w"], inp["k"])
    neg = index_scores(q, w, k, causal=1).cpu()
    assert _rel_err(neg, oix.causal_mask_(ref.clone())) < 1e-3
    assert torch.isneginf(neg[:, torch.ones(S, S, dtype=torch.bool).triu(1)]).all()
    sentinel = torch.full((B, S, S), 7.0, device=dev)
    low = index_scores(q, w, k, causal=2, out=sentinel).cpu()
    tri = torch.ones(S, S, dtype=torch.bool).tril()
    assert _rel_err(low[:, tri], ref[:, tri]) < 1e-3
    assert (low[:, ~tri] == 7.0).all()


@pytest.mark.parametrize("Sq,Sk,B,H,D,fp8", [
    (33, 33, 1, 16, 64, False),       # one token block pair, partial sub-tiles
    (517, 517, 2, 32, 64, False),     # odd block count: the middle block has no partner
    (1000, 1040, 1, 64, 128, True),   # keys past the last query are never visible
    (700, 660, 1, 16, 128, False),    # rows below Sk see every key
    (2064, 2064, 1, 16, 64, False),   # long rows: interior and diagonal tiles, several pieces
])
def test_indexer_lower_triangle_shapes(dev, Sq, Sk, B, H, D, fp8):
    """Lower-triangle mode splits paired token blocks (long row + short row)
    into equal pieces; every computed score must match the oracle and every
    score above the diagonal must be left untouched."""
    g = torch.Generator().manual_seed(Sq * 7 + Sk)
    q = torch.randn((Sq, B, H, D), generator=g).to(torch.bfloat16)
    k = torch.randn((Sk, B, D), generator=g).to(torch.bfloat16)
    w = torch.randn((Sq, B, H), generator=g) / H ** 0.5
    kw = {}
    if fp8:
        q, qs = ofp8.tensorwise_quantize(q)
        k, ks = ofp8.tensorwise_quantize(k)
        kw = dict(q_scale=qs.to(dev), k_scale=ks.to(dev))
        ref = oix.compute_index_scores(q.float(), w, k.float(), q_scale=qs, k_scale=ks)
    else:
        ref = oix.compute_index_scores(q, w, k)
    sentinel = torch.full((B, Sq, Sk), 7.0, device=dev)
    low = index_scores(q.to(dev), w.to(dev), k.to(dev), causal=2, out=sentinel, **kw).cpu()
    tri = torch.ones(Sq, Sk, dtype=torch.bool).tril()
    assert _rel_err(low[:, tri], ref[:, tri]) < 1e-3
    assert (low[:, ~tri] == 7.0).all()
    neg = index_scores(q.to(dev), w.to(dev), k.to(dev), causal=1, **kw).cpu()
    assert _rel_err(neg[:, tri], ref[:, tri]) < 1e-3
    assert torch.isneginf(neg[:, ~tri]).all()


def test_indexer_fp8(dev):
    S, B, H, D = 128, 1, 64, 128
    inp = synthetic.indexer_inputs(B, S, H, D, seed=9)
    q8, qs = ofp8.tensorwise_quantize(inp["q"])
    k8, ks = ofp8.tensorwise_quantize(inp["k"])
    got = index_scores(q8.to(dev), inp["w"].to(dev), k8.to(dev), q_scale=qs.to(dev), k_scale=ks.to(dev))
    ref = oix.compute_index_scores(q8.float(), inp["w"], k8.float(), q_scale=qs, k_scale=ks)
    assert _rel_err(got, ref) < 1e-3


def _tie_heavy_scores(rows, n, seed):
    g = np.random.default_rng(seed)
    s = g.standard_normal((rows, n)).astype(np.float32)
    s[:, ::3] = 0.0                                   # exact-zero ties (ReLU)
    s[:, 1::7] = -0.0                                 # negative zero equals zero
    s[g.random((rows, n)) < 0.05] = 1.5               # repeated positive value
    s[g.random((rows, n)) < 0.01] = np.nan            # NaN ranks as +inf
    s[g.random((rows, n)) < 0.01] = -np.inf
    s[g.random((rows, n)) < 0.01] = np.inf
    return s


@pytest.mark.parametrize("rows,n,topk,causal", [
    (300, 1000, 64, True),
    (257, 4096, 256, True),
    (64, 4096, 256, False),
    (40, 5000, 300, False),
    (16, 16384, 2048, False),
    (8, 20000, 2048, True),
])
def test_topk_bit_exact(dev, rows, n, topk, causal):
    s = _tie_heavy_scores(rows, n, seed=rows + n)
    seq_q = rows if causal else 1
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=causal, seq_q=seq_q if causal else None).cpu()
    st, en = otk.causal_windows(rows, seq_q, n) if causal else (None, None)
    ref = otk.topk_ascending(s, topk, st, en)
    assert got.dtype == torch.int32
    np.testing.assert_array_equal(got.numpy(), ref)


def _adversarial_scores(rows, n, seed):
    """Rows that stress the adaptive radix rounds: near-equal values a few ulps
    apart, one huge outlier squeezing the range, mostly -inf, sign-mixed tiny
    values, many exact ties right at the k-th value."""
    g = np.random.default_rng(seed)
    s = g.standard_normal((rows, n)).astype(np.float32)
    one = np.float32(1.0).view(np.int32)
    for r in range(rows):
        kind = r % 6
        if kind == 0:
            s[r] = (one + g.integers(0, 300, n)).astype(np.int32).view(np.float32)
        elif kind == 1:
            s[r, g.integers(0, n)] = 1e30
        elif kind == 2:
            s[r] = -np.inf
            s[r, g.integers(0, n, 40)] = g.standard_normal(40)
        elif kind == 3:
            s[r] = (g.standard_normal(n) * 1e-38).astype(np.float32)
        elif kind == 4:
            s[r] = np.round(s[r] * 4) / 4
        else:
            s[r, : n // 2] = 7.0
    return s


@pytest.mark.parametrize("rows,n,topk", [(36, 4096, 256), (24, 1000, 300), (12, 20000, 2048), (18, 600, 100)])
def test_topk_adversarial_rows(dev, rows, n, topk):
    s = _adversarial_scores(rows, n, seed=rows * 7 + n)
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=False).cpu()
    ref = otk.topk_ascending(s, topk)
    np.testing.assert_array_equal(got.numpy(), ref)


def _subset_bound_rows(rows, n, topk, seed):
    """Rows aimed at the wave kernel's lower bound L of the k-th largest (the
    least of 4 interleaved per-lane subset maxima; lane l holds columns 64i + l,
    item i feeds subset i % 4): exactly one large score per (lane, subset) so
    that only topk scores reach L, ties at L and scores one ulp below it (the
    same linear bucket), every subset maximum equal, NaN (ranked +inf) inside
    subsets, a subset made only of -inf (L falls back to the row minimum)."""
    g = np.random.default_rng(seed)
    s = (g.standard_normal((rows, n)) * 0.1).astype(np.float32)
    cols = np.arange(n)
    subset = (cols // 64) % 4
    lane = cols % 64
    for r in range(rows):
        kind = r % 5
        if kind in (0, 1, 2):
            big = (100.0 + g.random(256)).astype(np.float32)
            if kind == 1:
                big[:] = 5.0
            for ls in range(256):
                pick = np.flatnonzero((lane == ls // 4) & (subset == ls % 4))
                s[r, g.choice(pick)] = big[ls]
            lmin = big.min()
            if kind == 0:   # neighbours of L: equal to it, and one ulp below it
                free = np.flatnonzero(s[r] < 50)
                s[r, g.choice(free, 5, replace=False)] = lmin
                s[r, g.choice(free, 7, replace=False)] = np.nextafter(lmin, np.float32(-np.inf))
            if kind == 2:
                s[r, g.choice(n, 9, replace=False)] = np.nan
        elif kind == 3:
            s[r, (lane == 5) & (subset == 2)] = -np.inf
        else:
            s[r] = np.round(s[r] * 40) / 40
    return s


@pytest.mark.parametrize("n", [2048, 4096, 8192])
@pytest.mark.parametrize("topk", [64, 200, 256])
def test_topk_subset_bound_edges(dev, n, topk):
    s = _subset_bound_rows(30, n, topk, seed=n + topk)
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=False).cpu()
    np.testing.assert_array_equal(got.numpy(), otk.topk_ascending(s, topk))
    # the same rows as causal windows ending at every length up to n
    rows = 96
    t = np.repeat(s[:1], rows, axis=0)
    t[1::2] = s[1]
    got = topk_indices(torch.from_numpy(t).to(dev), topk, causal=True, seq_q=rows,
                       causal_offset=n - rows).cpu()
    st, en = otk.causal_windows(rows, rows, n, offset=n - rows)
    np.testing.assert_array_equal(got.numpy(), otk.topk_ascending(t, topk, st, en))


@pytest.mark.parametrize("rows,n,topk,causal", [
    (6, 70000, 2048, False),   # 3 segments of 23334 columns
    (40, 40000, 256, True),    # causal windows ending in either segment
    (5, 32769, 64, False),     # one column past a single pass
    (3, 300000, 100, False),   # 10 segments
])
def test_topk_long_rows(dev, rows, n, topk, causal):
    """Rows over 32768 columns: per-segment top-k, then one top-k over the
    segments' picks; the same contract (ties to the lower column, NaN as +inf,
    ascending, -1 padded) as one pass, against the oracle."""
    s = _tie_heavy_scores(rows, n, seed=rows + n)
    s[0, ::7] = np.nan                                   # NaN ranks +inf in every segment
    s[1 % rows] = np.float32(3.0)                         # all equal: the lowest columns win
    if rows > 3:
        s[3, : n // 2] = -np.inf                          # a -inf segment head
    seq_q, off = (rows, n // 2 - rows // 2) if causal else (1, 0)      # causal ends straddle the middle
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=causal, seq_q=seq_q if causal else None,
                       causal_offset=off).cpu()
    st, en = otk.causal_windows(rows, seq_q, n, offset=off) if causal else (None, None)
    np.testing.assert_array_equal(got.numpy(), otk.topk_ascending(s, topk, st, en))
    # explicit windows crossing the segment boundaries, some shorter than topk
    g = np.random.default_rng(n)
    starts = g.integers(0, n, rows).astype(np.int32)
    ends = np.minimum(n, starts + g.integers(0, n, rows)).astype(np.int32)
    ends[0] = min(n, starts[0] + topk // 2)
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=False,
                       starts=torch.from_numpy(starts).to(dev), ends=torch.from_numpy(ends).to(dev)).cpu()
    np.testing.assert_array_equal(got.numpy(), otk.topk_ascending(s, topk, starts, ends))


@pytest.mark.parametrize("n,off", [(16384, 8192 - 32), (20000, 8192 - 40), (12000, 8192 - 1)])
def test_topk_causal_rows_across_8192(dev, n, off):
    """Causal rows on both sides of 8192 columns in one call (two batches): the
    rows whose window fits 8192 take the wave kernel, the longer ones the
    workgroup kernel; both against the oracle."""
    rows, seq_q, topk = 128, 64, 512
    s = _tie_heavy_scores(rows, n, seed=n + off)
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=True, seq_q=seq_q, causal_offset=off).cpu()
    st, en = otk.causal_windows(rows, seq_q, n, offset=off)
    assert (en <= 8192).any() and (en > 8192).any()
    np.testing.assert_array_equal(got.numpy(), otk.topk_ascending(s, topk, st, en))


def test_topk_windows_and_all_equal(dev):
    rows, n, topk = 50, 700, 32
    s = np.zeros((rows, n), dtype=np.float32)          # all equal: lowest columns win
    s[10] = np.arange(n, dtype=np.float32)             # strictly increasing row
    g = np.random.default_rng(1)
    starts = g.integers(0, n, rows).astype(np.int32)
    ends = np.minimum(n, starts + g.integers(0, 100, rows)).astype(np.int32)
    got = topk_indices(torch.from_numpy(s).to(dev), topk, causal=False,
                       starts=torch.from_numpy(starts).to(dev), ends=torch.from_numpy(ends).to(dev)).cpu()
    ref = otk.topk_ascending(s, topk, starts, ends)
    np.testing.assert_array_equal(got.numpy(), ref)


def test_cfg3_indexer_topk_full_scale(dev):
    """cfg3: b=2 s=4096 h=16 d=64, causal top-256: GPU top-k == oracle top-k on the GPU's scores."""
    B, S, H, D, K = 2, 4096, 16, 64, 256
    inp = synthetic.indexer_inputs(B, S, H, D, seed=1234)
    inp["w"] = inp["w"] * (16 ** 0.5) / 4                # w ~ N(0,1)/4 (cfg3)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    scores, idx = indexer_topk(q, k, w, K, return_scores=True)
    sc = scores.cpu().numpy().reshape(B * S, S)
    st, en = otk.causal_windows(B * S, S, S)
    ref = otk.topk_ascending(np.where(np.arange(S)[None, :] < en[:, None], sc, 0), K, st, en)
    np.testing.assert_array_equal(idx.cpu().numpy().reshape(B * S, K), ref)
    # scores themselves vs the oracle on sampled rows
    rows = [0, 1, 255, 2048, 4095]
    ref_s = oix.compute_index_scores(inp["q"][rows], inp["w"][rows], inp["k"])
    got_s = scores.cpu()[:, rows]
    tri = torch.arange(S)[None, :] <= torch.tensor(rows)[:, None]
    assert _rel_err(got_s[:, tri], ref_s[:, tri]) < 1e-3


def test_fused_qk_topk_naive_contract(dev):
    S, B, H, D, K = 96, 2, 16, 64, 40
    inp = synthetic.indexer_inputs(B, S, H, D, seed=11)
    q, k, w = inp["q"].to(dev), inp["k"].to(dev), inp["w"].to(dev)
    scores, idx = fused_qk_topk_naive(q, k, w, K)
    assert idx.dtype == torch.int64 and idx.shape == (B, S, K)
    ref = otk.topk_ascending(scores.cpu().numpy().reshape(B * S, S), K)
    np.testing.assert_array_equal(idx.cpu().numpy().reshape(B * S, K), ref)
    mask = torch.full((S, S), float("-inf")).triu(1).to(dev)
    _, idx_c = fused_qk_topk_naive(q, k, w, K, mask=mask)
    st, en = otk.causal_windows(B * S, S, S)
    ref_c = otk.topk_ascending(scores.cpu().numpy().reshape(B * S, S), K, st, en)
    np.testing.assert_array_equal(idx_c.cpu().numpy().reshape(B * S, K), ref_c)


@pytest.mark.parametrize("n,dt", [(1, torch.float32), (1000, torch.bfloat16), (1 << 20, torch.bfloat16),
                                  (4099, torch.float32)])
def test_fp8_quantize_bit_exact(dev, n, dt):
    x = synthetic.outlier_values((n,), seed=n).to(dt)
    x8, si = tensorwise_quantize(x.to(dev))
    r8, rsi = ofp8.tensorwise_quantize(x)
    assert torch.equal(x8.cpu().view(torch.uint8), r8.view(torch.uint8))
    assert torch.equal(si.cpu(), rsi)


def test_fp8_quantize_zero_and_specials(dev):
    x = torch.zeros(64)
    x8, si = tensorwise_quantize(x.to(dev))
    assert float(si) == 1.0 and torch.all(x8.cpu().float() == 0)
    x = torch.tensor([1e-30, -1e-9, 3.0, -448.0 * 2, 5e-3, -0.0] * 8)
    x8, si = tensorwise_quantize(x.to(dev))
    r8, rsi = ofp8.tensorwise_quantize(x)
    assert torch.equal(x8.cpu().view(torch.uint8), r8.view(torch.uint8)) and torch.equal(si.cpu(), rsi)


def test_fp8_quantize_unaligned_input(dev):
    """A view starting 2 bytes into its storage takes the scalar path: same bits."""
    x = synthetic.outlier_values((4097,), seed=5).to(torch.bfloat16)
    xd = x.to(dev)[1:]
    x8, si = tensorwise_quantize(xd)
    r8, rsi = ofp8.tensorwise_quantize(x[1:])
    assert torch.equal(x8.cpu().view(torch.uint8), r8.view(torch.uint8)) and torch.equal(si.cpu(), rsi)


def test_fp8_dequantize_every_code(dev):
    """The hardware e4m3 conversion the SparseMLA kernels dequantise with equals
    the bit-field decode for all 256 codes (f32, NaN codes NaN, -0 kept), and
    the bf16 form is the RNE rounding of value * scale_inv."""
    from cppmega_amd.sparse_mla_ops import fp8_dequantize

    codes = torch.arange(256, dtype=torch.uint8)
    exp = torch.tensor([ofp8.e4m3_value(c) for c in range(256)], dtype=torch.float32)
    for n in (256, 255):   # a whole and a partial last group of four codes
        x8 = codes[:n].view(torch.float8_e4m3fn).to(dev)
        got = fp8_dequantize(x8, torch.ones(1), dtype=torch.float32).cpu()
        e = exp[:n]
        assert torch.equal(torch.isnan(got), torch.isnan(e))
        ok = ~torch.isnan(e)
        assert torch.equal(got[ok].view(torch.int32), e[ok].view(torch.int32))
    x8 = codes.view(torch.float8_e4m3fn).to(dev)
    for s in (1.0, 0.0625, 3.7e-3, 1000.0):
        si = torch.tensor([s], dtype=torch.float32)
        got = fp8_dequantize(x8, si).cpu()
        ref = (exp * si).to(torch.bfloat16)
        ok = ~torch.isnan(exp)
        assert torch.equal(got[ok].view(torch.int16), ref[ok].view(torch.int16)), s
        assert torch.isnan(got[~ok].float()).all()
    # round trip of the quantiser at its own scale
    x = synthetic.outlier_values((5000,), seed=9).to(torch.bfloat16)
    q8, qs = tensorwise_quantize(x.to(dev))
    back = fp8_dequantize(q8, qs, dtype=torch.float32).cpu()
    assert torch.equal(back, ofp8.dequantize(q8.cpu(), qs.cpu()))


def test_fp8_quantize_every_code_and_tie(dev):
    """amax = 448 makes the scale exactly 1: every e4m3 value and every midpoint
    between neighbours (round-to-nearest-even ties), both signs, and NaN map to
    the same codes as torch's float8_e4m3fn cast (x * scale never exceeds 448
    by more than rounding in a tensorwise cast, so saturation needs no test)."""
    vals = sorted({ofp8.e4m3_value(c) for c in range(128) if c != 0x7f})
    mids = [(a + b) / 2 for a, b in zip(vals[:-1], vals[1:])]
    pos = torch.tensor(vals + mids, dtype=torch.float32)
    x = torch.cat([pos, -pos, torch.tensor([448.0, float("nan"), -float("nan")])])
    x8, si = tensorwise_quantize(x.to(dev))
    assert float(si) == 1.0
    r8, _ = ofp8.tensorwise_quantize(x)
    got, ref = x8.cpu().view(torch.uint8), r8.view(torch.uint8)
    fin = ~torch.isnan(x)
    assert torch.equal(got[fin], ref[fin])
    assert torch.equal(got[~fin] & 0x7f, torch.full_like(got[~fin], 0x7f))   # NaN codes
