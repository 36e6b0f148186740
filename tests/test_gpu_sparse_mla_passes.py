"""GPU parity of the SparseMLA backward when it runs in several passes.

dsa_sparse_mla_bwd works through contiguous token ranges sized so that each
pass's partial dKV rows fit a cap (4 GiB by default, set small here through the calls'
pass_bytes argument): whole batches per pass, or one batch split
into 32-token multiples whose kv-row sums are carried in fp32 between passes.
Each case checks dq / dkv against the oracle at the usual bar, dq bitwise
against the one-pass call (dq does not depend on the passes), dkv against the
one-pass call at a tight bound (only the association of the fp32 sums
differs), and bitwise repeatability at the same cap.
"""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.sparse_mla_ops import sparse_mla_bwd, sparse_mla_bwd_fp8, sparse_mla_fwd_fp8_interface, \
    sparse_mla_fwd_interface
from oracle import sparse_mla as orc
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _per_token_bytes(H, D, topk, fp32_rows=False):
    ntiles = (H + 31) // 32
    return topk * ntiles * (D * (4 if fp32_rows else 2) + 1)


def _close_to_one_pass(a, b, what):
    a, b = a.float().cpu(), b.float().cpu()
    scale = float(b.abs().max())
    err = float((a - b).abs().max())
    assert err <= 4e-3 * scale + 1e-6, f"{what}: max diff {err:.3e} vs scale {scale:.3e}"


@pytest.mark.parametrize("B,S,H,D,DV,topk,tokens_per_pass", [
    (3, 96, 32, 128, 64, 64, 192),    # two whole batches per pass, then one
    (2, 200, 32, 128, 64, 64, 64),    # each batch in passes of 64, 64, 64, 8 tokens
    (1, 130, 64, 128, 64, 80, 32),    # two head tiles, five passes (the last of 2 tokens)
    (1, 96, 32, 192, 128, 48, 40),    # d_qk = 192: passes of 32 tokens
])
def test_bwd_passes_narrow(dev, B, S, H, D, DV, topk, tokens_per_pass):
    inp = synthetic.sparse_mla_inputs(B, S, H, D, DV, topk, std=0.5, seed=S + H)
    q, kv, idx, do = (inp[k].to(dev) for k in ("q", "kv", "indices", "do"))
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=inp["scale"], d_v=DV)
    dq1, dkv1 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"])
    cap = tokens_per_pass * _per_token_bytes(H, D, topk)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"], pass_bytes=cap)
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], inp["indices"], lse.cpu(),
                                   inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    assert torch.equal(dq, dq1), "dq depends on the passes"
    _close_to_one_pass(dkv, dkv1, "dkv vs one pass")
    dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"], pass_bytes=cap)
    assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2), "not bitwise repeatable"


def test_bwd_passes_repeated_rows(dev):
    """Unsorted slots and rows repeated inside a token (serial CSR placement) in a split batch."""
    B, S, H, D, DV, topk = 1, 160, 32, 128, 64, 64
    inp = synthetic.sparse_mla_inputs(B, S, H, D, DV, topk, std=0.5, seed=5)
    g = torch.Generator().manual_seed(5)
    idx = torch.gather(inp["indices"], -1, torch.argsort(torch.rand(B, S, 1, topk, generator=g), dim=-1))
    idx[0, 40, 0, 10:20] = idx[0, 40, 0, 0]
    idx[0, 130, 0, :] = 7
    idx = idx.contiguous()
    q, kv, idxd, do = inp["q"].to(dev), inp["kv"].to(dev), idx.to(dev), inp["do"].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idxd, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"],
                             pass_bytes=64 * _per_token_bytes(H, D, topk))
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], idx, lse.cpu(), inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")


@pytest.mark.parametrize("fp32_rows", [False, True], ids=["fp16_rows", "fp32_rows"])
@pytest.mark.parametrize("B,S,H,topk,tokens_per_pass", [(1, 72, 64, 48, 32), (2, 40, 32, 33, 40)])
def test_bwd_passes_wide(dev, B, S, H, topk, tokens_per_pass, fp32_rows):
    """d_qk = 576 / d_v = 512: a split batch, and whole batches per pass, with
    fp16 (default) and fp32 partial rows."""
    D, DV = 576, 512
    inp = synthetic.sparse_mla_inputs(B, S, H, D, DV, topk, std=0.5, seed=H + topk)
    q, kv, idx, do = (inp[k].to(dev) for k in ("q", "kv", "indices", "do"))
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=inp["scale"], d_v=DV)
    dq1, dkv1 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"], fp32_partials=fp32_rows)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"], fp32_partials=fp32_rows,
                             pass_bytes=tokens_per_pass * _per_token_bytes(H, D, topk, fp32_rows))
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], inp["indices"], lse.cpu(),
                                   inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    assert torch.equal(dq, dq1)
    _close_to_one_pass(dkv, dkv1, "dkv vs one pass")


def test_bwd_passes_fp8_per_token_scales(dev):
    """e4m3 codes with distinct per-token q scales and per-row kv scales: every
    pass must read the scales of its own tokens and kv rows."""
    B, S, H, D, DV, topk = 2, 96, 32, 128, 64, 64
    g = torch.Generator().manual_seed(11)
    q8 = torch.randn((B, S, H, D), generator=g).to(torch.float8_e4m3fn)
    k8 = torch.randn((B, S, 1, D), generator=g).to(torch.float8_e4m3fn)
    qsv = torch.exp2(torch.randint(-3, 1, (B, S), generator=g).float())
    ksv = torch.exp2(torch.randint(-3, 1, (B, S), generator=g).float())
    idx = synthetic.causal_indices(B, S, topk, seed=12)
    do = torch.randn((B, S, H, DV), generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    out, lse = sparse_mla_fwd_fp8_interface(q8.to(dev), k8.to(dev), idx.to(dev), q_scale=qsv.to(dev),
                                            kv_scale=ksv.to(dev), sm_scale=scale, d_v=DV)
    args = (q8.to(dev), k8.to(dev), qsv.to(dev), ksv.to(dev), out, do.to(dev), idx.to(dev), lse)
    dq1, dkv1 = sparse_mla_bwd_fp8(*args, sm_scale=scale)
    dq, dkv = sparse_mla_bwd_fp8(*args, sm_scale=scale, pass_bytes=32 * _per_token_bytes(H, D, topk))
    rdq, rdkv = orc.sparse_mla_bwd(q8, k8, out.cpu(), do, idx, lse.cpu(), scale, DV, q_scale=qsv, kv_scale=ksv)
    assert_close(dq, rdq, what="fp8 dq")
    assert_close(dkv, rdkv, what="fp8 dkv")
    assert torch.equal(dq, dq1), "dq depends on the passes"
    _close_to_one_pass(dkv, dkv1, "fp8 dkv vs one pass")
