"""GPU parity of the SparseMLA HIP kernels against the CPU oracle.

Bar: bf16 out, LSE (log2 units) and gradients within 2e-2 relative / 1e-2
absolute of the oracle (which restates the reference kernels, including the
bf16 rounding of P and dS); dKV bitwise identical across repeated calls.
"""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.sparse_mla_ops import (SparseMLA, sparse_mla_as_unfused_dsa, sparse_mla_bwd,
                                        sparse_mla_fwd_interface)
from oracle import sparse_mla as orc
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _fwd(inp, dev, d_v):
    q, kv, idx = inp["q"].to(dev), inp["kv"].to(dev), inp["indices"].to(dev)
    return sparse_mla_fwd_interface(q, kv, idx, sm_scale=inp["scale"], d_v=d_v)


def _inputs(B, S, H, D, DV, topk, G=1, seed=7, std=0.5, S_kv=None):
    inp = synthetic.sparse_mla_inputs(B, S, H, D, DV, topk, std=std, seed=seed, S_kv=S_kv)
    if G > 1:
        g = torch.Generator().manual_seed(seed + 99)
        S_kv = inp["kv"].shape[1]
        inp["kv"] = (torch.randn((B, S_kv, G, D), generator=g) * std).to(torch.bfloat16)
        idx = [synthetic.causal_indices(B, S, topk, seed=seed + 10 * gg, S_kv=S_kv) for gg in range(G)]
        inp["indices"] = torch.cat(idx, dim=2).contiguous()
    return inp


def test_fwd_cfg1_matches_oracle(dev):
    inp = synthetic.sparse_mla_inputs(1, 512, 16, 128, 64, 64, std=0.5, seed=1234, grad=False)
    inp["scale"] = 1.0 / 128 ** 0.5
    out, lse = _fwd(inp, dev, 64)
    ro, rl = orc.sparse_mla_fwd(inp["q"], inp["kv"], inp["indices"], inp["scale"], 64)
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32
    assert_close(out, ro, what="out")
    assert_close(lse, rl, what="lse2")


@pytest.mark.parametrize("B,S,H,G,D,DV,topk", [
    (2, 128, 32, 1, 128, 64, 64),
    (1, 200, 64, 1, 128, 64, 100),
    (1, 96, 128, 1, 128, 64, 40),
    (1, 80, 40, 1, 128, 64, 72),
    (1, 64, 32, 2, 128, 128, 32),
    (1, 64, 16, 1, 64, 32, 48),
    (1, 72, 32, 1, 192, 128, 96),
])
def test_fwd_shapes(dev, B, S, H, G, D, DV, topk):
    inp = _inputs(B, S, H, D, DV, topk, G=G)
    out, lse = _fwd(inp, dev, DV)
    ro, rl = orc.sparse_mla_fwd(inp["q"], inp["kv"], inp["indices"], inp["scale"], DV)
    assert_close(out, ro, what="out")
    assert_close(lse, rl, what="lse2")


def test_fwd_edge_indices(dev):
    B, S, H, D, DV, topk = 1, 64, 32, 128, 64, 64
    inp = _inputs(B, S, H, D, DV, topk)
    idx = inp["indices"].clone()
    idx[0, 5, 0, :] = -1                       # all masked
    idx[0, 6, 0, :8] = 3                       # duplicates count per occurrence
    idx[0, 7, 0, 10:20] = -7                   # other negatives are masked
    idx[0, 8, 0, 0:4] = torch.tensor([S, S + 5, 10 ** 6, -(2 ** 31)], dtype=torch.int32)  # out of range
    idx[0, 9, 0, :] = -1
    idx[0, 9, 0, 33] = 2                       # single valid slot, in the second block
    inp["indices"] = idx
    out, lse = _fwd(inp, dev, DV)
    ro, rl = orc.sparse_mla_fwd(inp["q"], inp["kv"], idx, inp["scale"], DV)
    assert_close(out, ro, what="out")
    assert_close(lse, rl, what="lse2")
    assert torch.all(out[0, 5] == 0) and torch.all(torch.isneginf(lse[0, 5]))
    # single valid slot: out = V[idx] exactly (P = 1), lse2 = scale * q.k * log2(e)
    v = inp["kv"][0, 2, 0, :DV].float()
    assert_close(out[0, 9].float().cpu(), v.expand(H, DV), rtol=0, atol=0, what="single-slot out")


def _bwd_case(dev, B, S, H, D, DV, topk, G=1, seed=7):
    inp = _inputs(B, S, H, D, DV, topk, G=G, seed=seed)
    q, kv, idx, do = (inp[k].to(dev) for k in ("q", "kv", "indices", "do"))
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"])
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], inp["indices"], lse.cpu(),
                                   inp["scale"], DV)
    return inp, (q, kv, idx, do, out, lse), (dq, dkv), (rdq, rdkv)


@pytest.mark.parametrize("B,S,H,G,D,DV,topk", [
    (1, 128, 32, 1, 128, 64, 64),
    (2, 96, 64, 1, 128, 64, 80),
    (1, 64, 16, 1, 128, 64, 40),
    (1, 64, 32, 2, 128, 128, 32),
    (1, 64, 16, 1, 64, 32, 48),
    (1, 72, 32, 1, 192, 128, 96),
])
def test_bwd_matches_oracle(dev, B, S, H, G, D, DV, topk):
    _, _, (dq, dkv), (rdq, rdkv) = _bwd_case(dev, B, S, H, D, DV, topk, G=G)
    assert dq.dtype == torch.bfloat16 and dkv.dtype == torch.bfloat16
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")


def test_bwd_bitwise_deterministic(dev):
    _, (q, kv, idx, do, out, lse), (dq, dkv), _ = _bwd_case(dev, 1, 256, 32, 128, 64, 64)
    for _ in range(2):
        dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idx, lse)
        assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2)


def test_bwd_edge_indices(dev):
    B, S, H, D, DV, topk = 1, 64, 32, 128, 64, 64
    inp = _inputs(B, S, H, D, DV, topk)
    idx = inp["indices"].clone()
    idx[0, 5, 0, :] = -1
    idx[0, 6, 0, :8] = 3
    idx[0, 8, 0, 0:4] = torch.tensor([S, S + 5, 10 ** 6, -3], dtype=torch.int32)
    q, kv, idxd, do = inp["q"].to(dev), inp["kv"].to(dev), idx.to(dev), inp["do"].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idxd, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], idx, lse.cpu(), inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    assert torch.all(dq[0, 5] == 0)


@pytest.mark.parametrize("D,DV,H,topk", [(128, 64, 32, 160), (576, 512, 64, 96)])
def test_bwd_last_valid_block(dev, D, DV, H, topk):
    """The block loops end after the last block that holds a valid slot: rows
    whose valid slots stop early, -1 scattered before valid slots, a wholly
    masked row, a row whose only valid slot is the last one, and out-of-range
    entries past the last valid slot (narrow and d_qk = 576 kernels)."""
    B, S = 1, 96
    inp = _inputs(B, S, H, D, DV, topk, seed=D + topk)
    g = torch.Generator().manual_seed(5)
    idx = torch.full((B, S, 1, topk), -1, dtype=torch.int32)
    for t in range(S):
        n = int(torch.randint(0, topk + 1, (1,), generator=g))
        pos = torch.randperm(topk, generator=g)[:n].sort().values
        idx[0, t, 0, pos] = torch.randint(0, t + 1, (n,), generator=g, dtype=torch.int32)
    idx[0, 10] = -1                                   # wholly masked
    idx[0, 11] = -1
    idx[0, 11, 0, topk - 1] = 7                       # only the last slot is valid
    idx[0, 12] = -1
    idx[0, 12, 0, 3] = 2                              # only the first block holds a valid slot
    idx[0, 12, 0, 40:] = S + 3                        # out of range past it (masked)
    q, kv, idxd, do = inp["q"].to(dev), inp["kv"].to(dev), idx.to(dev), inp["do"].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idxd, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], idx, lse.cpu(), inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    assert torch.all(dq[0, 10] == 0)


def test_bwd_unsorted_and_duplicate_indices(dev):
    """Unsorted slot order and repeated rows inside a token take the serial CSR path."""
    B, S, H, D, DV, topk = 2, 96, 32, 128, 64, 64
    inp = _inputs(B, S, H, D, DV, topk, seed=3)
    g = torch.Generator().manual_seed(3)
    perm = torch.argsort(torch.rand(B, S, 1, topk, generator=g), dim=-1)
    idx = torch.gather(inp["indices"], -1, perm)
    idx[0, 50, 0, 10:20] = idx[0, 50, 0, 0]
    idx[1, 70, 0, :] = 5
    q, kv, idxd, do = inp["q"].to(dev), inp["kv"].to(dev), idx.contiguous().to(dev), inp["do"].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idxd, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], idx, lse.cpu(), inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    assert torch.equal(dkv, dkv2) and torch.equal(dq, dq2)


def test_bwd_fp32_partials(dev):
    """fp32 dKV rows: same parity bar, deterministic, and at least as close to the oracle."""
    _, (q, kv, idx, do, out, lse), (dq, dkv), (rdq, rdkv) = _bwd_case(dev, 1, 256, 32, 128, 64, 128)
    dq32, dkv32 = sparse_mla_bwd(q, kv, out, do, idx, lse, fp32_partials=True)
    assert_close(dkv32, rdkv, what="dkv fp32 partials")
    assert torch.equal(dq32, dq)
    dq32b, dkv32b = sparse_mla_bwd(q, kv, out, do, idx, lse, fp32_partials=True)
    assert torch.equal(dkv32, dkv32b)
    err16 = float((dkv.float().cpu() - rdkv).abs().mean())
    err32 = float((dkv32.float().cpu() - rdkv).abs().mean())
    assert err32 <= err16 * 1.05 + 1e-6, (err32, err16)


def test_autograd_and_adapter(dev):
    B, S, H, D, DV, topk = 2, 64, 16, 128, 64, 32
    inp = _inputs(B, S, H, D, DV, topk)
    q = inp["q"].to(dev).requires_grad_()
    kv = inp["kv"].to(dev).requires_grad_()
    out, lse = SparseMLA.apply(q, kv, inp["indices"].to(dev), inp["scale"], DV)
    out.backward(inp["do"].to(dev))
    ro, rl = orc.sparse_mla_fwd(inp["q"], inp["kv"], inp["indices"], inp["scale"], DV)
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.detach().cpu(), inp["do"], inp["indices"],
                                   lse.detach().cpu(), inp["scale"], DV)
    assert_close(out, ro, what="out")
    assert_close(q.grad, rdq, what="dq")
    assert_close(kv.grad, rdkv, what="dkv")
    # Megatron unfused_dsa_fn layout: query [sq,b,np,hn], key [sk,b,np,hn], topk [b,sq,topk] int64
    query = inp["q"].permute(1, 0, 2, 3).contiguous()
    key = inp["kv"].permute(1, 0, 2, 3).expand(S, B, H, D).contiguous()
    value = key[..., :DV].contiguous()
    topk_idx = inp["indices"][:, :, 0, :].to(torch.int64)
    res = sparse_mla_as_unfused_dsa(query.to(dev), key.to(dev), value.to(dev), topk_idx.to(dev), inp["scale"])
    assert res.shape == (S, B, H * DV)
    assert_close(res, ro.permute(1, 0, 2, 3).reshape(S, B, H * DV), what="unfused adapter")


def test_three_dim_inputs(dev):
    inp = _inputs(1, 64, 32, 128, 64, 32)
    q, kv, idx = inp["q"][0].to(dev), inp["kv"][0].to(dev), inp["indices"][0].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=inp["scale"], d_v=64)
    assert out.shape == (64, 32, 64) and lse.shape == (64, 32)
    ro, rl = orc.sparse_mla_fwd(inp["q"], inp["kv"], inp["indices"], inp["scale"], 64)
    assert_close(out, ro[0], what="out")


def test_cfg2_full_scale(dev):
    """cfg2 at full size: sampled tokens vs the oracle, sampled kv rows of dKV vs
    the oracle restricted to the tokens that reference them, determinism."""
    B, S, H, D, DV, topk = 2, 4096, 32, 128, 64, 256
    inp = synthetic.sparse_mla_inputs(B, S, H, D, DV, topk, std=0.5, seed=1234)
    q, kv, idx, do = (inp[k].to(dev) for k in ("q", "kv", "indices", "do"))
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"])
    dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=inp["scale"])
    assert torch.equal(dkv, dkv2) and torch.equal(dq, dq2)
    outc, lsec = out.cpu(), lse.cpu()
    b = 1
    toks = torch.tensor([0, 1, 255, 256, 1000, 2047, 3000, 4095])
    sub = lambda x: x[b:b + 1, toks].contiguous()
    ro, rl = orc.sparse_mla_fwd(sub(inp["q"]), inp["kv"][b:b + 1], sub(inp["indices"]), inp["scale"], DV)
    assert_close(outc[b:b + 1, toks], ro, what="out (sampled)")
    assert_close(lsec[b:b + 1, toks], rl, what="lse2 (sampled)")
    rdq, _ = orc.sparse_mla_bwd(sub(inp["q"]), inp["kv"][b:b + 1], sub(outc), sub(inp["do"]),
                                sub(inp["indices"]), sub(lsec), inp["scale"], DV)
    assert_close(dq.cpu()[b:b + 1, toks], rdq, what="dq (sampled)")
    rows = torch.tensor([0, 7, 100, 2048, 4000])
    ref_tok = (inp["indices"][b, :, 0, :, None] == rows[None, None, :]).any(-1).any(-1).nonzero()[:, 0]
    _, rdkv = orc.sparse_mla_bwd(inp["q"][b:b + 1, ref_tok].contiguous(), inp["kv"][b:b + 1],
                                 outc[b:b + 1, ref_tok].contiguous(), inp["do"][b:b + 1, ref_tok].contiguous(),
                                 inp["indices"][b:b + 1, ref_tok].contiguous(), lsec[b:b + 1, ref_tok].contiguous(),
                                 inp["scale"], DV)
    assert_close(dkv.cpu()[b, rows], rdkv[0, rows], what="dkv (sampled rows)")
    # size-independent checks over every token and row: every token has at least one
    # valid slot (index 0), so all outputs are finite; summing dKV over all rows, the
    # rope tail (d >= d_v) is scale * sum_{t,h} q * sum_slot dS = 0 and the V part is
    # sum_{t,h} dO because each softmax row sums to one
    assert torch.isfinite(out).all() and torch.isfinite(lse).all() and torch.isfinite(dq).all()
    vmax = kv[..., :DV].float().abs().amax()
    assert float(out.float().abs().amax()) <= float(vmax) * 1.01      # convex combinations of V rows
    col = dkv.double().sum(dim=(0, 1, 2)).cpu()
    expect_v = do.double().sum(dim=(0, 1, 2)).cpu()
    scale_v = float(expect_v.norm() / DV ** 0.5)
    assert float((col[:DV] - expect_v).abs().max()) <= 2e-2 * scale_v, "sum_j dKV_j[:d_v] != sum dO"
    assert float(col[DV:].abs().max()) <= 2e-2 * scale_v, "sum_j dKV_j[d_v:] != 0"


@pytest.mark.parametrize("B,S,H,G,D,DV,topk,dup", [
    (1, 100, 32, 2, 128, 128, 300, False),   # > 256 slots per segment, partial last token chunk, 2 groups
    (2, 70, 32, 2, 128, 128, 40, True),      # a row repeated inside (token, group): serial chunk path
    (1, 33, 16, 1, 128, 64, 520, True),      # topk > S_kv: many masked slots plus repeats
])
def test_bwd_inverse_index_paths(dev, B, S, H, G, D, DV, topk, dup):
    """The inverse index's chunk paths: several 256-slot parts per (token, group),
    a token chunk cut short by S, kv groups, and repeated rows (exact counts and
    serial placement), all against the oracle and bitwise repeatable."""
    inp = _inputs(B, S, H, D, DV, topk, G=G, seed=S + topk)
    idx = inp["indices"].clone()
    if dup:
        g = torch.Generator().manual_seed(S)
        t = torch.randint(0, S, (5,), generator=g)
        for tt in t.tolist():
            n = min(tt + 1, topk)
            idx[0, tt, G - 1, : min(4, n)] = idx[0, tt, G - 1, 0]   # same row several times
    q, kv, idxd, do = inp["q"].to(dev), inp["kv"].to(dev), idx.contiguous().to(dev), inp["do"].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idxd, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], idx, lse.cpu(), inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2)


@pytest.mark.parametrize("S,G,S_kv,topk,dup", [
    (64, 1, 40000, 256, False),    # more kv rows than one LDS histogram held (32768)
    (40, 2, 20000, 128, True),     # 40000 rows over two groups, repeats in one row part
    (16, 1, 270000, 64, False),    # rows split by LDS size (17 parts), not only to fill the GPU
])
def test_bwd_long_kv_rows(dev, S, G, S_kv, topk, dup):
    """Backward with S_kv * G well past 32768 rows: the inverse index splits every
    32-token chunk's rows into parts (one workgroup and one LDS slice each);
    indices spread over the whole kv range, checked against the oracle and
    bitwise repeatable."""
    B, H, D, DV = 1, 32, 128, 64
    inp = _inputs(B, S, H, D, DV, topk, G=G, seed=S_kv + S, S_kv=S_kv)
    g = torch.Generator().manual_seed(S_kv)
    idx = torch.stack([torch.rand((S, S_kv), generator=g).topk(topk, dim=-1).indices.sort(dim=-1).values
                       for _ in range(G)], dim=1).to(torch.int32)[None]          # [1, S, G, topk]
    if dup:
        idx[0, 3, G - 1, :3] = idx[0, 3, G - 1, 0]
        idx[0, S - 1, 0, 1] = idx[0, S - 1, 0, 0]
    q, kv, idxd, do = inp["q"].to(dev), inp["kv"].to(dev), idx.contiguous().to(dev), inp["do"].to(dev)
    out, lse = sparse_mla_fwd_interface(q, kv, idxd, sm_scale=inp["scale"], d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    rdq, rdkv = orc.sparse_mla_bwd(inp["q"], inp["kv"], out.cpu(), inp["do"], idx, lse.cpu(), inp["scale"], DV)
    assert_close(dq, rdq, what="dq")
    assert_close(dkv, rdkv, what="dkv")
    dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idxd, lse, sm_scale=inp["scale"])
    assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2)
