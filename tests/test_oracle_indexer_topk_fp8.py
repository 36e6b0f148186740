"""Pins the indexer, top-k and FP8 quantiser oracles (CPU): known-answer
fixtures, the upstream einsum form, float64 brute force, torch.topk,
torch's float8_e4m3fn cast, and hypothesis properties."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle import fp8 as of8
from oracle import indexer as oidx
from oracle import topk as otk
from tests._util import assert_close, bf16_from_bits, load_golden


# ---------------------------------------------------------------------------
# Indexer
# ---------------------------------------------------------------------------
def _golden_indexer():
    g = load_golden("indexer.npz")
    return g, bf16_from_bits(g["q_bits"]), torch.from_numpy(g["w"]), bf16_from_bits(g["k_bits"])


def test_indexer_matches_golden():
    g, q, w, k = _golden_indexer()
    expect = torch.from_numpy(g["scores"])
    assert_close(oidx.compute_index_scores(q, w, k), expect, rtol=1e-5, atol=1e-4, what="per-head loop")
    assert_close(oidx.compute_index_scores_einsum(q, w, k), expect, rtol=1e-5, atol=1e-4, what="einsum")
    assert_close(oidx.compute_index_scores_f64(q, w, k), expect.double(), rtol=1e-9, atol=1e-9, what="f64")


def test_indexer_relu_off_and_planted_mistake():
    g, q, w, k = _golden_indexer()
    a = oidx.compute_index_scores(q, w, k, use_relu=False)
    b = oidx.compute_index_scores_f64(q, w, k, use_relu=False)
    assert_close(a, b, rtol=1e-5, atol=1e-4, what="no relu")
    with pytest.raises(AssertionError):  # ReLU dropped: the fixture catches it
        assert_close(a, torch.from_numpy(g["scores"]), rtol=1e-3, atol=1e-3, what="relu dropped")
    with pytest.raises(AssertionError):  # weights of the wrong head
        assert_close(oidx.compute_index_scores(q, w.flip(-1), k), torch.from_numpy(g["scores"]),
                     rtol=1e-3, atol=1e-3, what="heads swapped")


def test_indexer_fp8_scales_dequantise():
    g, q, w, k = _golden_indexer()
    q8 = (q.float() * 8).to(torch.float8_e4m3fn)
    k8 = (k.float() * 4).to(torch.float8_e4m3fn)
    a = oidx.compute_index_scores(q8, w, k8, q_scale=0.125, k_scale=0.25)
    b = oidx.compute_index_scores_f64(q8.double() * 0.125, w, k8.double() * 0.25)
    assert_close(a, b, rtol=1e-5, atol=1e-4, what="fp8 indexer")


@pytest.mark.parametrize("relu", [True, False])
def test_indexer_backward_oracle_gradcheck(relu):
    """The float64 score loop is differentiable the way finite differences say
    (gradcheck), and its autograd gradients match the loop's value at a
    perturbed point to first order."""
    g = torch.Generator().manual_seed(7)
    q = torch.randn(5, 2, 3, 4, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(5, 2, 3, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(6, 2, 4, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b_, c: oidx.index_scores_diff(a, b_, c, relu), (q, w, k))
    grad = torch.randn(2, 5, 6, generator=g, dtype=torch.float64)
    dq, dw, dk = oidx.index_scores_backward(grad, q, w, k, use_relu=relu)
    assert dq.shape == q.shape and dw.shape == w.shape and dk.shape == k.shape
    # the float64 loop equals the fp32 oracle restatement's values
    assert torch.allclose(oidx.index_scores_diff(q, w, k, relu).float(),
                          oidx.compute_index_scores(q.float(), w.float(), k.float(), relu), atol=1e-5)


def test_indexer_backward_closed_form_and_causal():
    """One head, one query, one key: dq = G w [L > 0] k, dw = G ReLU(L),
    dk = G w [L > 0] q; a negative logit gives zero dq / dk / dw under ReLU;
    causal=True drops the gradient above the diagonal."""
    q = torch.tensor([[[[1.0, 2.0]]]], dtype=torch.float64)          # [1, 1, 1, 2]
    k = torch.tensor([[[0.5, -0.25]]], dtype=torch.float64)          # [1, 1, 2]
    w = torch.tensor([[[3.0]]], dtype=torch.float64)
    G = torch.tensor([[[2.0]]], dtype=torch.float64)
    L = float((q[0, 0, 0] * k[0, 0]).sum())                        # 0.5 - 0.5 = 0: ReLU' is 0 at 0
    assert L == 0.0
    k = torch.tensor([[[0.5, 0.25]]], dtype=torch.float64)
    L = float((q[0, 0, 0] * k[0, 0]).sum())                        # 1.0
    dq, dw, dk = oidx.index_scores_backward(G, q, w, k)
    assert torch.allclose(dq[0, 0, 0], 2.0 * 3.0 * k[0, 0]) and float(dw) == 2.0 * L
    assert torch.allclose(dk[0, 0], 2.0 * 3.0 * q[0, 0, 0])
    dq, dw, dk = oidx.index_scores_backward(G, q, w, -k)              # L < 0: ReLU blocks everything
    assert float(dq.abs().sum() + dw.abs().sum() + dk.abs().sum()) == 0.0
    gen = torch.Generator().manual_seed(3)
    q2 = torch.randn(3, 1, 2, 4, dtype=torch.float64, generator=gen)
    k2 = torch.randn(3, 1, 4, dtype=torch.float64, generator=gen)
    w2 = torch.randn(3, 1, 2, dtype=torch.float64, generator=gen)
    G2 = torch.zeros(1, 3, 3, dtype=torch.float64)
    G2[0, 0, 2] = 1.0                                                 # above the diagonal only
    dq, dw, dk = oidx.index_scores_backward(G2, q2, w2, k2, use_relu=False, causal=True)
    assert float(dq.abs().sum() + dw.abs().sum() + dk.abs().sum()) == 0.0
    dq, dw, dk = oidx.index_scores_backward(G2, q2, w2, k2, use_relu=False, causal=False)
    assert float(dk[2].abs().sum()) > 0 and float(dk[:2].abs().sum()) == 0.0


def test_causal_mask_and_flops():
    s = torch.zeros(2, 4, 4)
    oidx.causal_mask_(s)
    assert torch.isinf(s).sum() == 2 * 6 and torch.all(s.tril() == 0)
    assert oidx.flops_causal(2, 4096, 16, 64) == 34_368_126_976


# ---------------------------------------------------------------------------
# Top-k
# ---------------------------------------------------------------------------
def test_topk_matches_golden():
    g = load_golden("topk.npz")
    k = int(g["topk"])
    out = otk.topk_ascending(g["scores"], k, g["starts"], g["ends"])
    np.testing.assert_array_equal(out, g["out"])
    for r in range(len(g["out"])):
        row = otk.topk_bruteforce_row(g["scores"][r], k, int(g["starts"][r]), int(g["ends"][r]))
        assert row == list(g["out"][r])


def test_topk_vs_torch_topk_on_distinct_rows():
    gen = torch.Generator().manual_seed(3)
    s = torch.randn(64, 500, generator=gen)
    for k in (1, 7, 64, 499, 500):
        mine = otk.topk_ascending(s.numpy(), k)
        ref = torch.topk(s, k, dim=-1).indices.sort(-1).values.numpy()
        np.testing.assert_array_equal(mine, ref)


def test_topk_causal_windows_and_padding():
    rows, n, k = 12, 10, 4
    starts, ends = otk.causal_windows(rows, seq_q=6, row_len=n)
    assert list(ends[:6]) == [1, 2, 3, 4, 5, 6] and list(ends[6:]) == [1, 2, 3, 4, 5, 6]
    s = np.arange(rows * n, dtype=np.float32).reshape(rows, n)
    out = otk.topk_ascending(s, k, starts, ends)
    assert list(out[0]) == [0, -1, -1, -1]            # t + 1 < k: padded with -1
    assert list(out[5]) == [2, 3, 4, 5]               # largest in the window, ascending
    _, e2 = otk.causal_windows(4, seq_q=4, row_len=8, offset=2)
    assert list(e2) == [3, 4, 5, 6]


def test_topk_bytes():
    assert otk.topk_bytes(2, 4096, 256) == 75_513_856


_score = st.one_of(st.sampled_from([0.0, -0.0, 1.0, -1.0, 2.5, math.inf, -math.inf, math.nan]),
                   st.floats(-4, 4, width=32))


@settings(max_examples=200, deadline=None)
@given(st.lists(_score, min_size=1, max_size=40), st.integers(1, 45), st.data())
def test_topk_property_bruteforce(row, k, data):
    n = len(row)
    start = data.draw(st.integers(0, n))
    end = data.draw(st.integers(start, n))
    arr = np.array([row], dtype=np.float32)
    out = otk.topk_ascending(arr, k, np.array([start]), np.array([end]))[0]
    assert list(out) == otk.topk_bruteforce_row(arr[0], k, start, end)
    sel = [i for i in out if i >= 0]
    assert sel == sorted(sel) and len(set(sel)) == len(sel)
    assert len(sel) == min(k, end - start) and all(start <= i < end for i in sel)


@settings(max_examples=200, deadline=None)
@given(st.lists(st.tuples(_score, st.booleans()), min_size=1, max_size=40), st.integers(1, 45), st.data())
def test_topk_admissible_property_bruteforce(cells, k, data):
    """Admissible-set restriction (the masked candidates of fused_qk_topk_naive)
    against the pure-Python brute force, inside random windows."""
    n = len(cells)
    row = [c[0] for c in cells]
    adm = [c[1] for c in cells]
    start = data.draw(st.integers(0, n))
    end = data.draw(st.integers(start, n))
    arr = np.array([row], dtype=np.float32)
    out = otk.topk_ascending(arr, k, np.array([start]), np.array([end]), admissible=np.array([adm]))[0]
    assert list(out) == otk.topk_bruteforce_row(arr[0], k, start, end, admissible=adm)
    sel = [i for i in out if i >= 0]
    assert len(sel) == min(k, sum(adm[start:end])) and all(adm[i] for i in sel)


def test_mask_windows_and_masked_pick_repair():
    """Oracle pieces of the sync-free fused_qk_topk_naive: per-row spans of the
    finite mask entries (first / last finite column, (0, 0) for an all -inf
    row), the plain flag (the span holds only +0.0), and the repair that turns
    picks on -inf holes into trailing -1 padding."""
    ninf = float("-inf")
    m = np.array([[[0, 0, ninf, ninf],          # prefix, plain
                   [ninf, 0, ninf, 0],          # span with a hole
                   [ninf, ninf, ninf, ninf],    # nothing admissible (plain: adds nothing)
                   [ninf, ninf, ninf, 0.5]]],   # last column only, finite bias
                 dtype=np.float32)
    st_, en_, pl = otk.mask_windows(m)
    assert st_[0].tolist() == [0, 1, 0, 3] and en_[0].tolist() == [2, 4, 0, 4]
    assert pl[0].tolist() == [1, 0, 1, 0]
    neg0 = np.array([[[0.0, -0.0, ninf]]], dtype=np.float32)        # -0.0 is not +0.0
    assert otk.mask_windows(neg0)[2].tolist() == [[0]]
    causal = np.triu(np.full((5, 5), ninf, dtype=np.float32), 1)[None]
    cs, ce, cp = otk.mask_windows(causal)
    assert cs[0].tolist() == [0] * 5 and ce[0].tolist() == [1, 2, 3, 4, 5] and cp[0].tolist() == [1] * 5
    scores = np.array([[1.0, ninf, 3.0, ninf, 5.0]], dtype=np.float32)
    assert otk.drop_masked_picks(scores, [[0, 1, 2, 3]]).tolist() == [[0, 2, -1, -1]]
    assert otk.drop_masked_picks(scores, [[4, -1, -1]]).tolist() == [[4, -1, -1]]
    assert otk.drop_masked_picks(scores, [[0, 1, 2, 3]], plain=[1]).tolist() == [[0, 1, 2, 3]]


@settings(max_examples=200, deadline=None)
@given(st.lists(st.sampled_from([0.0, -0.0, 0.5, -2.0, float("-inf"), float("inf"), float("nan")]),
                min_size=1, max_size=12))
def test_mask_windows_matches_bruteforce(row):
    st_, en_, pl = otk.mask_windows(np.array([[row]], dtype=np.float32))
    assert (int(st_[0, 0]), int(en_[0, 0]), int(pl[0, 0])) == otk.mask_windows_bruteforce(row)


# ---------------------------------------------------------------------------
# FP8 e4m3fn
# ---------------------------------------------------------------------------
def test_e4m3_decode_all_codes_vs_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float()
    for c in range(256):
        v = of8.e4m3_value(c)
        r = float(ref[c])
        assert (math.isnan(v) and math.isnan(r)) or (v == r and math.copysign(1, v) == math.copysign(1, r)), c


def test_quantize_matches_golden_and_torch_cast():
    g = load_golden("fp8.npz")
    x = torch.from_numpy(g["x"])
    y, scale_inv = of8.tensorwise_quantize(x)
    codes = y.view(torch.uint8).numpy()
    np.testing.assert_array_equal(codes, g["codes"])
    assert float(scale_inv) == float(g["scale_inv"])
    # every finite code round-trips through decode / encode
    vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    finite = torch.isfinite(vals)
    back = vals[finite].to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(back, torch.arange(256, dtype=torch.uint8)[finite])


def test_quantize_special_cases():
    y, si = of8.tensorwise_quantize(torch.zeros(16))
    assert float(si) == 1.0 and torch.all(y.float() == 0)
    x = torch.tensor([1.0, float("nan"), -3.0, 0.5])
    y, si = of8.tensorwise_quantize(x)
    assert float(si) == pytest.approx(3.0 / 448.0, rel=1e-7)   # NaN does not enter amax
    assert float(y[2].float()) == -448.0
    assert torch.isnan(y[1].float())
    back = of8.dequantize(y, si)
    assert float(back[2]) == pytest.approx(-3.0, rel=1e-6)
    # saturation: values beyond 448 after scaling clamp to +-448
    assert float(torch.tensor([1e9]).clamp(-448, 448).to(torch.float8_e4m3fn).float()) == 448.0
