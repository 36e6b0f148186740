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

from cppmega_amd import synthetic
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
