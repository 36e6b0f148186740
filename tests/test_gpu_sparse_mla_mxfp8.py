"""GPU parity of the MXFP8 block-scaled SparseMLA forward (dsa_sparse_mla_fwd
with DSA_DTYPE_MXFP8) and of its backward through dequantisation.

Reference: sparse_mla_blockscaled_mxfp8_fwd_interface / _backward
(cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_blockscaled_fused.py:248-418,
694-793, 1015-1051).  Bars: out, LSE within the bf16 bar (2e-2 rel / 1e-2 abs)
of the MXFP8 oracle on the same e4m3 payloads and scales; the block-scaled
dequantisation bit-exact; the backward within the bf16 bar of the oracle's
bf16 backward on the dequantised tensors.
"""
import os

import pytest
import torch

from cppmega_amd import _lib, synthetic
from cppmega_amd.sparse_mla_ops import (mxfp8_dequantize, sparse_mla_blockscaled_mxfp8_backward,
                                        sparse_mla_blockscaled_mxfp8_forward,
                                        sparse_mla_blockscaled_mxfp8_fwd_interface)
from oracle import sparse_mla as orc
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def _inputs(B, S, H, D, G, K, seed, spread=True, pow2=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, S, H, D), generator=g) * 0.5
    kv = torch.randn((B, S, G, D), generator=g) * 0.5
    if spread:
        # q channel blocks 10^4 apart in magnitude make every score depend on
        # the right q / kv block scale; kv (whose first channels are V) varies
        # mildly, since the P-rounding error of any bf16 PV grows with |V|
        # rather than with |out| (a x100 V fails the output-relative bar for
        # the bf16 kernel against the bf16 oracle too)
        q = q * torch.logspace(-2, 2, D)
        kv = kv * torch.logspace(0.3, -0.3, D)
    q8, qs = orc.mxfp8_quantize(q)
    kv8, ks = orc.mxfp8_quantize(kv)
    if not pow2:  # arbitrary f32 block scales (the ABI takes any)
        qs = qs * (1.0 + torch.rand(qs.shape, generator=g))
        ks = ks * (1.0 + torch.rand(ks.shape, generator=g))
    idx = synthetic.causal_indices(B, S, K, seed=seed + 1).expand(B, S, G, K).contiguous()
    return q8, qs, kv8, ks, idx


@pytest.mark.parametrize("B,S,H,D,DV,G,K,pow2", [
    (1, 128, 32, 128, 64, 1, 64, True),
    (2, 96, 16, 128, 64, 1, 40, False),
    (1, 64, 64, 128, 64, 2, 48, True),
    (1, 80, 32, 192, 128, 1, 64, False),
    # d_qk = 576 (the wide kernel: four waves split d_qk, so blocks 4 and 13
    # are each scaled half in one wave and half in the next)
    (1, 48, 32, 576, 512, 1, 64, True),
    (2, 40, 16, 576, 512, 1, 40, False),
    (1, 36, 64, 576, 512, 2, 48, False),
    (1, 24, 96, 576, 512, 1, 40, False),   # two head tiles per workgroup, one empty
])
def test_mxfp8_fwd_matches_oracle(dev, B, S, H, D, DV, G, K, pow2):
    q8, qs, kv8, ks, idx = _inputs(B, S, H, D, G, K, seed=S + D, pow2=pow2)
    scale = D ** -0.5
    out, lse = sparse_mla_blockscaled_mxfp8_fwd_interface(q8.to(dev), kv8.to(dev), qs.to(dev), ks.to(dev), idx.to(dev),
                                                          sm_scale=scale, d_v=DV)
    ro, rl = orc.sparse_mla_fwd_mxfp8(q8, kv8, qs, ks, idx, scale, DV)
    assert out.dtype == torch.bfloat16 and out.shape == (B, S, H, DV)
    assert_close(out, ro, what="mxfp8 out")
    assert_close(lse, rl, what="mxfp8 lse2")
    # deterministic
    out2, lse2 = sparse_mla_blockscaled_mxfp8_fwd_interface(q8.to(dev), kv8.to(dev), qs.to(dev), ks.to(dev),
                                                            idx.to(dev), sm_scale=scale, d_v=DV)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)


def _mx_fwd_blockscaled_only(q8, kv8, qs, ks, idx, scale, dv):
    """dsa_sparse_mla_fwd without a workspace: the block-scaled e4m3 kernel alone."""
    B, S, H, D = q8.shape
    _, Skv, G, _ = kv8.shape
    out = torch.empty((B, S, H, dv), dtype=torch.bfloat16, device=q8.device)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=q8.device)
    L = _lib.load()
    _lib.check(L.dsa_sparse_mla_fwd(q8.data_ptr(), kv8.data_ptr(), idx.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                    B, S, Skv, H, G, D, dv, idx.shape[-1], scale, _lib.DTYPE_MXFP8, qs.data_ptr(),
                                    ks.data_ptr(), 0), "dsa_sparse_mla_fwd(mxfp8)")
    return out, lse


@pytest.mark.parametrize("B,S,H,D,DV,G,K", [
    (1, 128, 32, 128, 64, 1, 64),
    (2, 64, 64, 128, 64, 2, 48),
    (1, 80, 32, 192, 128, 1, 64),
    (1, 48, 96, 576, 512, 1, 64),
])
def test_mxfp8_exact_path_and_fallback(dev, B, S, H, D, DV, G, K):
    """Power-of-two block scales: the call dequantises kv exactly and runs the
    bf16 kernel (q converted at load); its output matches the block-scaled
    kernel's up to the order of the fp32 score sums.  One scale that is not a
    power of two sends the same call to the block-scaled kernel, whose result
    then equals the no-workspace call's bit for bit."""
    q8, qs, kv8, ks, idx = (t.to(dev) for t in _inputs(B, S, H, D, G, K, seed=D + H))
    scale = D ** -0.5
    out, lse = sparse_mla_blockscaled_mxfp8_fwd_interface(q8, kv8, qs, ks, idx, sm_scale=scale, d_v=DV)
    ob, lb = _mx_fwd_blockscaled_only(q8, kv8, qs, ks, idx, scale, DV)
    ref_scale = float(ob.float().abs().max())
    assert float((out.float() - ob.float()).abs().max()) <= 2 ** -7 * ref_scale
    assert float((lse - lb).abs().max()) <= 1e-4 * float(lb.abs().max())
    ro, rl = orc.sparse_mla_fwd_mxfp8(q8.cpu(), kv8.cpu(), qs.cpu(), ks.cpu(), idx.cpu(), scale, DV)
    assert_close(out, ro, what="exact-path out")
    assert_close(lse, rl, what="exact-path lse2")
    for which in ("kv", "q"):   # one scale off the power-of-two grid: the block-scaled kernel
        qs2, ks2 = qs.clone(), ks.clone()
        (ks2 if which == "kv" else qs2).view(-1)[5] *= 1.5
        o2, l2 = sparse_mla_blockscaled_mxfp8_fwd_interface(q8, kv8, qs2, ks2, idx, sm_scale=scale, d_v=DV)
        ob2, lb2 = _mx_fwd_blockscaled_only(q8, kv8, qs2, ks2, idx, scale, DV)
        assert torch.equal(o2, ob2) and torch.equal(l2, lb2), which


def test_mxfp8_path_choice_in_a_graph(dev):
    """The path is chosen on the device at every replay: a captured call
    follows in-place changes of the block scales between replays."""
    B, S, H, D, DV, G, K = 1, 96, 32, 128, 64, 1, 48
    q8, qs, kv8, ks, idx = (t.to(dev) for t in _inputs(B, S, H, D, G, K, seed=7))
    scale = D ** -0.5
    ks_pow2 = ks.clone()
    ks_odd = ks.clone()
    ks_odd.view(-1)[3] *= 1.25
    eager = {}
    for name, k in (("pow2", ks_pow2), ("odd", ks_odd)):
        ks.copy_(k)
        eager[name] = [t.clone() for t in sparse_mla_blockscaled_mxfp8_fwd_interface(q8, kv8, qs, ks, idx,
                                                                                      sm_scale=scale, d_v=DV)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sparse_mla_blockscaled_mxfp8_fwd_interface(q8, kv8, qs, ks, idx, sm_scale=scale, d_v=DV)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = sparse_mla_blockscaled_mxfp8_fwd_interface(q8, kv8, qs, ks, idx, sm_scale=scale, d_v=DV)
    for name in ("pow2", "odd", "pow2", "odd"):
        ks.copy_(ks_pow2 if name == "pow2" else ks_odd)
        torch.zeros(1 << 20, device=dev).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res[0], eager[name][0]) and torch.equal(res[1], eager[name][1]), name


def test_mxfp8_dequantize_bit_exact(dev):
    q8, qs, _, _, _ = _inputs(2, 33, 8, 128, 1, 8, seed=3, pow2=False)
    for dt in (torch.bfloat16, torch.float32):
        got = mxfp8_dequantize(q8.to(dev), qs.to(dev), dtype=dt).cpu()
        ref = orc.dequantize_blockwise(q8, qs, out_dtype=dt)
        assert torch.equal(got.view(torch.int16 if dt == torch.bfloat16 else torch.int32),
                           ref.view(torch.int16 if dt == torch.bfloat16 else torch.int32))


@pytest.mark.parametrize("S,D,DV", [(96, 128, 64), (40, 576, 512)])
def test_mxfp8_public_wrappers_and_backward(dev, monkeypatch, S, D, DV):
    B, H, K = 1, 32, 48
    # unspread values, arbitrary block scales: the gradients of the bf16
    # backward scale their dS / P rounding with |q| and |dO|, so the bar is
    # stated for the N(0, 0.5)-sized tensors it is stated for elsewhere
    q8, qs, kv8, ks, idx = _inputs(B, S, H, D, 1, K, seed=11, spread=False, pow2=False)
    args = [t.to(dev) for t in (q8, kv8, qs, ks, idx)]
    monkeypatch.delenv("CPPMEGA_SPARSE_MLA_BLOCKSCALED_FUSED", raising=False)
    with pytest.raises(RuntimeError):
        sparse_mla_blockscaled_mxfp8_forward(*args, softmax_scale=None, d_v=DV)
    monkeypatch.setenv("CPPMEGA_SPARSE_MLA_BLOCKSCALED_FUSED", "1")
    out, lse = sparse_mla_blockscaled_mxfp8_forward(*args, softmax_scale=None, d_v=DV)
    do = torch.randn((B, S, H, DV), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    dq, dkv = sparse_mla_blockscaled_mxfp8_backward(args[0], args[1], args[2], args[3], out, do.to(dev), args[4], lse,
                                                    softmax_scale=None, d_v=DV)
    qd = orc.dequantize_blockwise(q8, qs)
    kvd = orc.dequantize_blockwise(kv8, ks)
    ro, rl = orc.sparse_mla_fwd(qd, kvd, idx, D ** -0.5, DV)
    rdq, rdkv = orc.sparse_mla_bwd(qd, kvd, ro.to(torch.bfloat16), do, idx, rl, D ** -0.5, DV)
    assert dq.shape == qd.shape and dkv.shape == kvd.shape
    assert_close(dq, rdq, what="mxfp8 dq")
    assert_close(dkv, rdkv, what="mxfp8 dkv")


def test_mxfp8_input_validation(dev):
    q8, qs, kv8, ks, idx = _inputs(1, 32, 16, 128, 1, 16, seed=2)
    a = [t.to(dev) for t in (q8, kv8, qs, ks, idx)]
    with pytest.raises(ValueError):   # tail_dim = 0 (the reference requires a positive tail)
        sparse_mla_blockscaled_mxfp8_fwd_interface(*a, d_v=128)
    with pytest.raises(ValueError):   # bf16 data
        sparse_mla_blockscaled_mxfp8_fwd_interface(a[0].float().to(torch.bfloat16), *a[1:], d_v=64)
    with pytest.raises(ValueError):   # wrong scale shape
        sparse_mla_blockscaled_mxfp8_fwd_interface(a[0], a[1], a[2][..., :2].contiguous(), a[3], a[4], d_v=64)
