"""Pinning of the CPU oracle for the DSA indexer KL loss (oracle/indexer_loss.py).

The reference (cppmega/megatron/dsa_splitk_indexer_loss.py:328-468) is a
Triton kernel; its test (tests/test_dsa_splitk_indexer_loss.py:29-83) defines
the loss by a pure-PyTorch clone of Megatron's compute_dsa_indexer_loss, which
the oracle restates.  These checks pin that restatement independently of its
own code: a pure-Python fixture, closed forms, torch's kl_div, and planted
mistakes that the fixture must catch.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import indexer_loss as okl
from tests._util import bf16_from_bits, load_golden

FIXTURES = ("indexer_loss_h4.npz", "indexer_loss_g2.npz")


def _inputs(z, which="any"):
    q = bf16_from_bits(z["q_bits"])
    k = bf16_from_bits(z["k_bits"])
    sc = torch.from_numpy(z["index_scores"])
    topk = torch.from_numpy(z[f"topk_{which}"])
    return sc, topk, q, k, float(z["scale"])


def _same(a, e, tol=1e-9):
    a, e = np.asarray(a, dtype=np.float64), np.asarray(e, dtype=np.float64)
    assert a.shape == e.shape
    assert np.array_equal(np.isnan(a), np.isnan(e)), "NaN rows differ"
    ok = ~np.isnan(e)
    assert np.allclose(a[ok], e[ok], rtol=tol, atol=tol), float(np.abs(a[ok] - e[ok]).max())


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_matches_fixture(name):
    z = load_golden(name)
    sc, topk_any, q, k, scale = _inputs(z, "any")
    _same(okl.indexer_kl_rows(sc, topk_any, q, k, scale, False), z["rows_dense"])
    _same(okl.indexer_kl_rows(sc, topk_any, q, k, scale, True), z["rows_sparse_any"])
    _, topk_c, _, _, _ = _inputs(z, "causal")
    _same(okl.indexer_kl_rows(sc, topk_c, q, k, scale, True), z["rows_sparse_causal"])
    # the fixture exercises the NaN rule (rows with no top-k column <= t)
    assert np.isnan(z["rows_sparse_any"]).any() and not np.isnan(z["rows_sparse_causal"]).any()


def test_scalar_is_coeff_times_row_mean():
    z = load_golden("indexer_loss_g2.npz")
    sc, topk, q, k, scale = _inputs(z, "causal")
    for coeff in (1.0, 0.5, 2.0):
        loss = okl.compute_dsa_indexer_loss(sc, topk, q, k, scale, coeff, True)
        assert math.isclose(float(loss), coeff * float(np.mean(z["rows_sparse_causal"])), rel_tol=1e-12)
    l1 = okl.compute_dsa_indexer_loss(sc, topk, q, k, scale, 1.0, False)
    l2 = okl.compute_dsa_indexer_loss(sc, topk, q, k, scale, 2.0, False)
    assert math.isclose(float(l2), 2 * float(l1), rel_tol=1e-12)


def test_closed_form_uniform_target_constant_index():
    """q = 0 makes every head uniform over s <= t; constant index scores make Q
    uniform over all sk columns: KL_t = log(sk / (t + 1)) (up to the 1e-10 terms)."""
    sq, sk, b, h, d = 12, 17, 2, 3, 16
    q = torch.zeros(sq, b, h, d, dtype=torch.bfloat16)
    k = torch.randn(sk, b, h, d).to(torch.bfloat16)
    sc = torch.full((b, sq, sk), 0.7)
    topk = torch.zeros(b, sq, 1, dtype=torch.int64)
    rows = okl.indexer_kl_rows(sc, topk, q, k, 0.25, False)
    expect = torch.tensor([math.log(sk / (t + 1)) for t in range(sq)], dtype=torch.float64)
    assert torch.allclose(rows, expect.expand(b, sq), atol=1e-8)


def test_zero_when_index_equals_single_head_attention():
    """One head, index scores = its causal logits (-inf above the diagonal): P == Q, KL == 0."""
    sq, b, d = 10, 1, 32
    q = torch.randn(sq, b, 1, d).to(torch.bfloat16)
    k = torch.randn(sq, b, 1, d).to(torch.bfloat16)
    scale = 0.3
    logits = torch.einsum("tbd,sbd->bts", q[:, :, 0].double(), k[:, :, 0].double()) * scale
    logits = logits.masked_fill(torch.ones(sq, sq, dtype=torch.bool).triu(1), float("-inf"))
    rows = okl.indexer_kl_rows(logits, torch.zeros(b, sq, 1, dtype=torch.int64), q, k, scale, False)
    assert float(rows.abs().max()) < 1e-8


def test_matches_torch_kl_div():
    z = load_golden("indexer_loss_h4.npz")
    sc, _, q, k, scale = _inputs(z)
    sq, b, h, d = q.shape
    att = torch.einsum("tbhd,sbhd->bhts", q.double(), k.double()) * scale
    att = att.masked_fill(torch.ones(sq, sq, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.softmax(att, -1).mean(1)
    logq = torch.log_softmax(sc.double(), -1)
    kl = torch.nn.functional.kl_div(logq, p, reduction="none").sum(-1)   # sum p (log p - log q)
    rows = okl.indexer_kl_rows(sc, torch.zeros(b, sq, 1, dtype=torch.int64), q, k, scale, False)
    # the 1e-10 terms shift entries by at most ~1e-9 relative to the exact KL
    assert torch.allclose(rows, kl, atol=1e-6)


def _planted(kind, sc, topk, q, k, scale, sparse):
    """Oracle variants with one plausible mistake each (CPU only)."""
    sq, b, h, d = q.shape
    sk = k.shape[0]
    g = k.shape[2]
    qq = q.double().permute(1, 2, 0, 3)
    kk = k.double().repeat_interleave(h // g, dim=2).permute(1, 2, 3, 0)
    att = torch.matmul(qq, kk) * scale
    mask = okl.sparse_mask(topk, sk) if sparse else None
    if sparse:
        att = att + mask.unsqueeze(1)
    if kind != "no_causal":
        att = att + torch.triu(torch.full((sq, sk), float("-inf"), dtype=torch.float64), 1)
    probs = torch.softmax(att, -1)
    target = probs.sum(1) if kind == "sum_heads" else probs.mean(1)
    idx = sc.double() + (mask if sparse else 0)
    if kind == "causal_index":
        idx = idx + torch.triu(torch.full((sq, sk), float("-inf"), dtype=torch.float64), 1)
    qprob = torch.softmax(idx, -1)
    if kind == "log2":
        kl = target * (torch.log2(target + okl.EPS) - torch.log2(qprob + okl.EPS))
    else:
        kl = target * (torch.log(target + okl.EPS) - torch.log(qprob + okl.EPS))
    return kl.sum(-1)


@pytest.mark.parametrize("kind", ["no_causal", "causal_index", "sum_heads", "log2"])
def test_planted_mistakes_are_caught(kind):
    z = load_golden("indexer_loss_g2.npz")
    sc, topk, q, k, scale = _inputs(z, "causal")
    for sparse, key in ((False, "rows_dense"), (True, "rows_sparse_causal")):
        rows = _planted(kind, sc, topk, q, k, scale, sparse).numpy()
        assert not np.allclose(rows, z[key], rtol=1e-3, atol=1e-3), f"{kind} (sparse={sparse}) not caught"
    # and the unplanted variant reproduces the fixture
    _same(_planted("none", sc, topk, q, k, scale, True).numpy(), z["rows_sparse_causal"])


def test_rows_at_matches_full_form():
    z = load_golden("indexer_loss_g2.npz")
    sc, topk, q, k, scale = _inputs(z, "any")
    pos = [(b, t) for b in range(2) for t in range(20)]
    for sparse in (False, True):
        full = okl.indexer_kl_rows(sc, topk, q, k, scale, sparse)
        at = okl.indexer_kl_rows_at(sc, topk, q, k, scale, sparse, pos)
        _same(at.numpy(), full.flatten().numpy())


# ---- gradient with respect to the index scores ----

def _grad_case(seed, sq=6, sk=6, b=1, np_=2, hn=4, topk=3):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(sq, b, np_, hn, generator=gen).to(torch.bfloat16)
    k = torch.randn(sk, b, np_, hn, generator=gen).to(torch.bfloat16)
    z = torch.randn(b, sq, sk, generator=gen, dtype=torch.float64)
    # causal top-k (every row keeps column 0, so no row is empty)
    ti = torch.stack([torch.cat([torch.zeros(1, dtype=torch.long),
                                 torch.randint(0, t + 1, (topk - 1,), generator=gen)]) for t in range(sq)] * b)
    return q, k, z, ti.reshape(b, sq, topk)


@pytest.mark.parametrize("sparse", [False, True], ids=["dense", "sparse"])
def test_grad_matches_finite_differences(sparse):
    q, k, z, ti = _grad_case(5)
    f = lambda zz: okl.compute_dsa_indexer_loss(zz, ti, q, k, 0.5, 0.7, sparse)
    assert torch.autograd.gradcheck(f, (z.clone().requires_grad_(True),), eps=1e-6, atol=1e-8)
    g = okl.indexer_kl_grad(z, ti, q, k, 0.5, 0.7, sparse, grad_loss=1.0)
    gd = torch.zeros_like(z)
    for idx in np.ndindex(*z.shape):  # central differences of the loss itself
        e = torch.zeros_like(z)
        e[idx] = 1e-6
        gd[idx] = (f(z + e) - f(z - e)) / 2e-6
    assert torch.allclose(g, gd, atol=1e-8, rtol=1e-5)


@pytest.mark.parametrize("sparse", [False, True], ids=["dense", "sparse"])
def test_grad_invariants(sparse):
    q, k, z, ti = _grad_case(9, sq=12, sk=12, np_=3, topk=4)
    z[0, 3, 7] = float("-inf")  # a masked score: Q = 0 there
    g = okl.indexer_kl_grad(z, ti, q, k, 0.3, 1.0, sparse, grad_loss=2.0)
    # a softmax gradient sums to zero over every row
    assert g.sum(-1).abs().max() < 1e-15
    # zero wherever Q = 0
    assert g[0, 3, 7] == 0.0
    if sparse:
        keep = torch.isfinite(okl.sparse_mask(ti, 12))
        assert (g[~keep] == 0).all()
    # linear in the upstream gradient and in loss_coeff
    g1 = okl.indexer_kl_grad(z, ti, q, k, 0.3, 0.5, sparse, grad_loss=1.0)
    assert torch.allclose(g, 4.0 * g1, rtol=1e-12, atol=0)


def test_grad_nan_rows():
    q, k, z, _ = _grad_case(2, sq=5, sk=5)
    ti = torch.full((1, 5, 2), 4, dtype=torch.long)  # only column 4: rows t < 4 have no admissible column
    g = okl.indexer_kl_grad(z, ti, q, k, 0.5, 1.0, True)
    assert torch.isnan(g[0, :4]).all() and torch.isfinite(g[0, 4]).all()
