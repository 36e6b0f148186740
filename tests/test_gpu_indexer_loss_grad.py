"""GPU parity of the KL indexer loss's gradient with respect to the index scores
(dsa_indexer_kl_loss_backward through the C-ABI, and the autograd path of
indexer_kl_loss / compute_dsa_indexer_loss_splitk).

The reference's split-K loss (cppmega/megatron/dsa_splitk_indexer_loss.py:328-468)
is forward-only; the gradient it stands in for is autograd through Megatron's
compute_dsa_indexer_loss, whose clone the oracle restates
(tests/test_dsa_splitk_indexer_loss.py:29-83).  Oracle: float64 autograd of
that loss, pinned by finite differences on the CPU.  Bar: every element within
2e-3 of the largest |gradient| of the tensor (the closed form's two terms
cancel where P ~ Q, so the error is relative to the term size, not to the
element), exact zeros where Q = 0, NaN on exactly the oracle's NaN rows.
"""
import math

import pytest
import torch

from cppmega_amd import compute_dsa_indexer_loss_splitk, indexer_kl_loss, indexer_kl_loss_backward
from oracle import indexer_loss as okl

pytestmark = pytest.mark.gpu

GRAD_REL = 2e-3


def _inputs(sq, sk, b, np_, hn, seed, g=None):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    g = np_ if g is None else g
    query = torch.randn(sq, b, np_, hn, generator=gen, dtype=torch.bfloat16)
    key = torch.randn(sk, b, g, hn, generator=gen, dtype=torch.bfloat16)
    sc = torch.randn(b, sq, sk, generator=gen, dtype=torch.float32)
    return query, key, sc


def _causal_topk(sc, topk):
    sq, sk = sc.shape[-2:]
    masked = sc.masked_fill(torch.ones(sq, sk, dtype=torch.bool).triu(1), float("-inf"))
    return masked.topk(min(topk, sk), dim=-1).indices


def _check_grad(got, ref, what, zeros=True):
    got = got.detach().double().cpu()
    assert got.shape == ref.shape, f"{what}: shape {tuple(got.shape)} != {tuple(ref.shape)}"
    assert torch.equal(torch.isnan(got), torch.isnan(ref)), f"{what}: NaN pattern differs"
    ok = ~torch.isnan(ref)
    if zeros:
        assert torch.equal(got[ok] == 0, ref[ok] == 0), f"{what}: zero pattern differs"
    scale = ref[ok].abs().max()
    err = (got[ok] - ref[ok]).abs().max()
    assert err <= GRAD_REL * scale, f"{what}: max err {float(err):.3g} > {GRAD_REL} x {float(scale):.3g}"


@pytest.mark.parametrize("sparse", [False, True], ids=["dense", "sparse"])
@pytest.mark.parametrize("sq,sk,b,np_,g,hn,topk,seed", [
    (128, 128, 1, 4, 4, 64, 32, 42),     # the reference test's small case
    (128, 128, 2, 8, 8, 64, 32, 99),     # multi-head, b = 2
    (200, 300, 1, 8, 8, 128, 40, 5),     # sk > sq, sk % 4 != 0 (scalar paths), partial blocks
    (160, 160, 1, 8, 2, 192, 24, 6),     # grouped key heads, 64-key chunks
    (96, 130, 1, 4, 4, 256, 8, 7),       # hn = 256
    (300, 150, 2, 4, 1, 64, 16, 9),      # sk < sq: rows t >= sk clamp their last key to sk - 1
])
def test_grad_matches_oracle(dev, sparse, sq, sk, b, np_, g, hn, topk, seed):
    query, key, sc = _inputs(sq, sk, b, np_, hn, seed, g=g)
    ctk = _causal_topk(sc, topk)
    scale, coeff = 1.0 / math.sqrt(hn), 0.7
    ref = okl.indexer_kl_grad(sc, ctk, query, key, scale, coeff, sparse, grad_loss=1.5)
    got = indexer_kl_loss_backward(torch.tensor(1.5), sc.to(dev), ctk.to(dev), query.to(dev), key.to(dev), scale,
                                   coeff, sparse)
    assert got.dtype == torch.float32
    _check_grad(got, ref, f"{(sq, sk, b, np_, g, hn)} sparse={sparse}")
    # the rows of a softmax gradient sum to zero
    rs = got.double().sum(-1).abs().max()
    assert rs <= 1e-4 * got.double().abs().sum(-1).max()


def test_grad_padding_masked_scores_and_nan_rows(dev):
    """-1 padding and repeated top-k columns, -inf index scores (Q = 0: zero
    gradient), and rows without an admissible column (NaN on the row only)."""
    sq, sk, b, np_, hn, topk = 150, 150, 1, 4, 64, 20
    query, key, sc = _inputs(sq, sk, b, np_, hn, seed=8)
    ctk = _causal_topk(sc, topk)
    padded = ctk.clone()
    padded[:, ::3, -5:] = -1
    padded[:, 1::3, -2] = padded[:, 1::3, 0]
    masked = sc.masked_fill(torch.ones(sq, sk, dtype=torch.bool).triu(1), float("-inf"))
    args = (query.to(dev), key.to(dev), 0.125, 1.0)
    for z, tk, sparse, what in ((masked, padded, True, "padded top-k"), (masked, ctk, False, "causally masked")):
        ref = okl.indexer_kl_grad(z, tk, query, key, 0.125, 1.0, sparse)
        got = indexer_kl_loss_backward(1.0, z.to(dev), tk.to(dev), *args, sparse)
        _check_grad(got, ref, what)
    # top-k holding columns 100 and 120 only: rows t < 100 have no target (NaN
    # rows); a row t >= 120 whose target equals its index softmax has a
    # gradient of rounding size on both sides, so no zero-pattern check here
    only = torch.tensor([100, 120]).expand(b, sq, 2).contiguous()
    ref = okl.indexer_kl_grad(sc, only, query, key, 0.125, 1.0, True)
    got = indexer_kl_loss_backward(1.0, sc.to(dev), only.to(dev), *args, True)
    assert torch.isnan(ref[0, :100]).all() and torch.isfinite(ref[0, 100:]).all()
    _check_grad(got, ref, "NaN rows", zeros=False)


def test_autograd_path(dev):
    """loss.backward() through indexer_kl_loss and the drop-in gives the same
    bits as the direct backward call; without requires_grad no graph is built."""
    query, key, sc = _inputs(128, 128, 1, 4, 64, seed=3)
    ctk = _causal_topk(sc, 16).to(dev)
    qd, kd = query.to(dev), key.to(dev)
    for sparse in (False, True):
        z = sc.to(dev).requires_grad_(True)
        loss = compute_dsa_indexer_loss_splitk(z, ctk, qd, kd, 0.125, 0.5, sparse, None)
        assert loss.requires_grad
        (2.0 * loss).backward()
        direct = indexer_kl_loss_backward(2.0, sc.to(dev), ctk, qd, kd, 0.125, 0.5, sparse)
        assert torch.equal(z.grad, direct)
        plain = indexer_kl_loss(sc.to(dev), ctk, qd, kd, 0.125, 0.5, sparse)
        assert not plain.requires_grad
        assert torch.equal(plain, loss.detach())


def test_full_size_grad_properties(dev):
    """b = 2, s = 4096, 32 heads of 128, top-256: finite, zero row sums, zeros
    off the top-k set (sparse) and above the diagonal's -inf scores,
    bitwise-identical reruns."""
    sq, b, np_, hn, topk = 4096, 2, 32, 128, 256
    gen = torch.Generator().manual_seed(21)
    query = (torch.randn(sq, b, np_, hn, generator=gen) * 0.5).to(torch.bfloat16).to(dev)
    key = (torch.randn(sq, b, np_, hn, generator=gen) * 0.5).to(torch.bfloat16).to(dev)
    sc = torch.randn(b, sq, sq, generator=gen).to(dev)
    masked = sc.masked_fill(torch.ones(sq, sq, dtype=torch.bool, device=dev).triu(1), float("-inf"))
    ctk = masked.topk(topk, dim=-1).indices
    for sparse in (False, True):
        g1 = indexer_kl_loss_backward(1.0, masked, ctk, query, key, 1.0 / math.sqrt(hn), 1.0, sparse)
        g2 = indexer_kl_loss_backward(1.0, masked, ctk, query, key, 1.0 / math.sqrt(hn), 1.0, sparse)
        assert torch.equal(g1, g2)
        assert torch.isfinite(g1).all()
        assert (g1.masked_select(torch.ones(sq, sq, dtype=torch.bool, device=dev).triu(1)) == 0).all()
        if sparse:
            keep = torch.zeros_like(g1, dtype=torch.bool).scatter_(-1, ctk, True)
            assert (g1[~keep] == 0).all()
        rs = g1.double().sum(-1).abs().max()
        assert rs <= 1e-4 * g1.double().abs().sum(-1).max()
        del g1, g2
