"""GPU tests of the SparseMLA drop-in surface Megatron calls: the FP8
unfused_dsa_fn adapter, the absorbed-MLA FP8 call site, the per-batch 3-D
SparseMLA.apply that Megatron's _fused_sparse_mla_absorbed makes (forward
and backward), zero-copy Float8Tensor input, and cfg4 (FP8 tensorwise) at
full size.

Bars: against the FP8 oracle on the same e4m3 payloads and scales, the bf16
one (2e-2 relative / 1e-2 absolute) on N(0, 0.5) data and the stated
mostly-close bar on outlier data; bf16 paths against the bf16 oracle at the
bf16 bar.
"""
import types

import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.sparse_mla_ops import (SparseMLA, SparseMLA_FP8, fp8_dequantize, fused_sparse_mla_absorbed_fp8,
                                        sparse_mla_bwd_fp8, sparse_mla_fp8_as_unfused_dsa,
                                        sparse_mla_fwd_fp8_interface, tensorwise_quantize)
from cppmega_amd.sparse_mla_ops.sparse_mla import _extract_fp8_data
from oracle import fp8 as ofp8
from oracle import sparse_mla as orc
from tests._util import assert_close, assert_mostly_close

pytestmark = pytest.mark.gpu


def _data(B, S, H, D, DV, topk, seed, std=0.5):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn((B, S, H, D), generator=g) * std).to(torch.bfloat16)
    kv = (torch.randn((B, S, 1, D), generator=g) * std).to(torch.bfloat16)
    do = torch.randn((B, S, H, DV), generator=g).to(torch.bfloat16)
    idx = synthetic.causal_indices(B, S, topk, seed=seed + 1)
    return q, kv, idx, do


def _fp8_oracle(q, kv, idx, scale, DV, do=None, out=None, lse=None):
    """Tensorwise quantisation of the whole q / kv (bit-exact with the device
    quantiser), then the FP8 oracle forward (and backward when do is given)."""
    B, S = q.shape[:2]
    q8, qs = ofp8.tensorwise_quantize(q)
    k8, ks = ofp8.tensorwise_quantize(kv)
    qsv, ksv = qs.expand(B, S).contiguous(), ks.expand(B, S).contiguous()
    ro, rl = orc.sparse_mla_fwd(q8, k8, idx, scale, DV, q_scale=qsv, kv_scale=ksv)
    if do is None:
        return ro, rl
    rdq, rdkv = orc.sparse_mla_bwd(q8, k8, out, do, idx, lse, scale, DV, q_scale=qsv, kv_scale=ksv)
    return ro, rl, rdq, rdkv


def test_fp8_unfused_dsa_adapter(dev):
    """sparse_mla_fp8_as_unfused_dsa (Megatron unfused_dsa_fn signature): SBHD
    query / key with the latent shared by every head, int64 top-k with -1 and
    out-of-range picks -> [sq, b, np * hnv], forward and backward."""
    B, S, H, D, DV, topk = 2, 96, 16, 128, 64, 48
    q, kv, idx, do = _data(B, S, H, D, DV, topk, seed=301)
    topk_idx = idx[:, :, 0, :].to(torch.int64)
    topk_idx[0, 10, :5] = S + 3          # out of range: masked like -1
    idx_ref = topk_idx.clone()
    idx_ref[(idx_ref < 0) | (idx_ref >= S)] = -1
    idx_ref = idx_ref.to(torch.int32).unsqueeze(2)
    scale = D ** -0.5
    query = q.permute(1, 0, 2, 3).contiguous().to(dev).requires_grad_()
    key_lat = kv.permute(1, 0, 2, 3).contiguous().to(dev).requires_grad_()
    key = key_lat.expand(S, B, H, D)
    value = key[..., :DV]
    res = sparse_mla_fp8_as_unfused_dsa(query, key, value, topk_idx.to(dev), scale)
    assert res.shape == (S, B, H * DV) and res.dtype == torch.bfloat16
    dres = do.permute(1, 0, 2, 3).reshape(S, B, H * DV).to(dev)
    res.backward(dres)
    out = res.detach().reshape(S, B, H, DV).permute(1, 0, 2, 3).contiguous()
    # the adapter quantises the contiguous BSHD q and the [b, sk, 1, d] latent
    ro, rl = _fp8_oracle(q, kv, idx_ref, scale, DV)
    assert_close(out, ro, what="adapter out")
    _, _, rdq, rdkv = _fp8_oracle(q, kv, idx_ref, scale, DV, do=do, out=out.cpu(), lse=_lse_of(q, kv, idx_ref, dev,
                                                                                                scale, DV))
    assert_close(query.grad.permute(1, 0, 2, 3), rdq, what="adapter dq")
    # the key gradient reaches the shared latent through the expand
    assert_close(key_lat.grad.permute(1, 0, 2, 3), rdkv, what="adapter dkv")


def _lse_of(q, kv, idx, dev, scale, DV):
    q8, qs = tensorwise_quantize(q.to(dev))
    k8, ks = tensorwise_quantize(kv.to(dev))
    B, S = q.shape[:2]
    _, lse = sparse_mla_fwd_fp8_interface(q8, k8, idx.to(dev), q_scale=qs.expand(B, S).contiguous(),
                                          kv_scale=ks.expand(B, S).contiguous(), sm_scale=scale, d_v=DV)
    return lse.cpu()


def test_fused_sparse_mla_absorbed_fp8(dev):
    """The absorbed-MLA FP8 call site (cppmega/megatron/sparse_mla_ops/sparse_mla.py:689-734):
    one SparseMLA_FP8 call per batch element on 3-D tensors, each quantised on
    its own; forward vs the FP8 oracle per batch element, gradients through
    autograd, and None for unsupported shapes."""
    B, S, H, D, DV, topk = 2, 128, 32, 128, 64, 64
    q, kv, idx, do = _data(B, S, H, D, DV, topk, seed=311)
    scale = D ** -0.5
    query = q.permute(1, 0, 2, 3).contiguous().to(dev).requires_grad_()     # [sq, b, np, d]
    key = kv.permute(1, 0, 2, 3).contiguous().to(dev).requires_grad_()      # [skv, b, 1, d]
    topk_idx = idx[:, :, 0, :].to(torch.int64).to(dev)                       # [b, sq, topk]
    out = fused_sparse_mla_absorbed_fp8(query, key, topk_idx, scale, DV)
    assert out.shape == (S, B, H, DV)
    out.backward(do.permute(1, 0, 2, 3).to(dev))
    for bi in range(B):
        qb, kb, ib, dob = q[bi:bi + 1], kv[bi:bi + 1], idx[bi:bi + 1], do[bi:bi + 1]
        ob = out.detach()[:, bi].unsqueeze(0).cpu()
        lse = _lse_of(qb, kb, ib, dev, scale, DV)
        ro, _, rdq, rdkv = _fp8_oracle(qb, kb, ib, scale, DV, do=dob, out=ob, lse=lse)
        assert_close(ob, ro, what=f"absorbed out b={bi}")
        assert_close(query.grad[:, bi].unsqueeze(0), rdq, what=f"absorbed dq b={bi}")
        assert_close(key.grad[:, bi].unsqueeze(0), rdkv, what=f"absorbed dkv b={bi}")
    assert fused_sparse_mla_absorbed_fp8(query, key, topk_idx[..., :40], scale, DV) is None   # topk % 64
    assert fused_sparse_mla_absorbed_fp8(query, key.expand(S, B, 2, D), topk_idx, scale, DV) is None


def test_three_dim_per_batch_apply_backward(dev):
    """Megatron's _fused_sparse_mla_absorbed loop (apply_dsa_cg_patches.py:238-243):
    SparseMLA.apply(q_t [sq, np, d], kv_t [skv, 1, d], idx_t [sq, 1, topk] i32,
    scale, v_channels) per batch element, forward and backward, bf16."""
    B, S, H, D, DV, topk = 2, 80, 32, 128, 64, 40
    q, kv, idx, do = _data(B, S, H, D, DV, topk, seed=321)
    scale = D ** -0.5
    for bi in range(B):
        q_t = q[bi].to(dev).requires_grad_()
        kv_t = kv[bi].to(dev).requires_grad_()
        idx_t = idx[bi].to(dev)
        out, lse = SparseMLA.apply(q_t, kv_t, idx_t, scale, DV)
        assert out.shape == (S, H, DV) and lse.shape == (S, H)
        out.backward(do[bi].to(dev))
        ro, rl = orc.sparse_mla_fwd(q[bi:bi + 1], kv[bi:bi + 1], idx[bi:bi + 1], scale, DV)
        assert_close(out, ro[0], what="3-D out")
        assert_close(lse, rl[0], what="3-D lse2")
        rdq, rdkv = orc.sparse_mla_bwd(q[bi:bi + 1], kv[bi:bi + 1], out.detach().cpu().unsqueeze(0),
                                       do[bi:bi + 1], idx[bi:bi + 1], lse.detach().cpu().unsqueeze(0), scale, DV)
        assert q_t.grad.shape == q_t.shape and kv_t.grad.shape == kv_t.shape
        assert_close(q_t.grad, rdq[0], what="3-D dq")
        assert_close(kv_t.grad, rdkv[0], what="3-D dkv")


class _FakeFloat8Tensor:
    """Duck type of a Transformer Engine Float8Tensor as SparseMLA_FP8 sees it:
    uint8 storage in _data, the dequant factor in _scale_inv and the e4m3 kind
    in _fp8_dtype (tests/test_sparse_mla_te_fp8_extract.py:89-130)."""

    def __init__(self, x):
        x8, si = tensorwise_quantize(x)
        self._data = x8.view(torch.uint8)
        self._scale_inv = si
        self._fp8_dtype = types.SimpleNamespace(name="kFloat8E4M3")
        self.shape = x.shape


def test_float8_tensor_zero_copy_extraction(dev):
    x = synthetic.outlier_values((64, 128), seed=7).to(torch.bfloat16).to(dev)
    packed = _FakeFloat8Tensor(x)
    fp8, scale = _extract_fp8_data(packed)
    assert fp8 is not None and fp8.dtype == torch.float8_e4m3fn
    assert fp8.data_ptr() == packed._data.data_ptr()             # zero copy
    assert scale is packed._scale_inv
    ref = (fp8.to(torch.float32) * scale).to(torch.bfloat16)
    assert torch.equal(fp8_dequantize(fp8, scale), ref)          # Float8Tensor.dequantize() role, exact
    assert _extract_fp8_data(torch.zeros(3, device=dev)) == (None, None)
    other = types.SimpleNamespace(_data=packed._data, _scale_inv=scale,
                                  _fp8_dtype=types.SimpleNamespace(name="kFloat8E5M2"))
    assert _extract_fp8_data(other) == (None, None)              # e5m2 payloads are not taken


def test_sparse_mla_fp8_takes_float8_tensors(dev):
    """SparseMLA_FP8 on Float8Tensor-like q / kv: the payloads are used as they
    are (no requantisation), matching the FP8 oracle on the same codes."""
    B, S, H, D, DV, topk = 1, 128, 32, 128, 64, 64
    q, kv, idx, do = _data(B, S, H, D, DV, topk, seed=331)
    scale = D ** -0.5
    pq, pk = _FakeFloat8Tensor(q.to(dev)), _FakeFloat8Tensor(kv.to(dev))
    out, lse = SparseMLA_FP8.apply(pq, pk, idx.to(dev), scale, DV)
    ro, rl = _fp8_oracle(q, kv, idx, scale, DV)
    assert_close(out, ro, what="Float8Tensor out")
    assert_close(lse, rl, what="Float8Tensor lse2")


def test_cfg4_full_scale(dev):
    """cfg4 at full size (b=2, s=4096, h=32, topk=256; q / kv N(0, 1) with 1% x20
    outliers, e4m3 tensorwise): sampled tokens of out, LSE and dq vs the FP8
    oracle, sampled dKV rows vs the oracle over the tokens that reference them,
    bitwise reruns, and the size-independent column sums of dKV."""
    B, S, H, D, DV, topk = 2, 4096, 32, 128, 64, 256
    q = synthetic.outlier_values((B, S, H, D), 41).to(torch.bfloat16)
    kv = synthetic.outlier_values((B, S, 1, D), 42).to(torch.bfloat16)
    idx = synthetic.causal_indices(B, S, topk, seed=43)
    do = torch.randn((B, S, H, DV), generator=torch.Generator().manual_seed(44)).to(torch.bfloat16)
    scale = D ** -0.5
    q8, qs = tensorwise_quantize(q.to(dev))
    k8, ks = tensorwise_quantize(kv.to(dev))
    r8, rqs = ofp8.tensorwise_quantize(q)
    rk8, rks = ofp8.tensorwise_quantize(kv)
    assert torch.equal(q8.cpu().view(torch.uint8), r8.view(torch.uint8)) and torch.equal(qs.cpu(), rqs)
    qsv, ksv = qs.expand(B, S).contiguous(), ks.expand(B, S).contiguous()
    idxd, dod = idx.to(dev), do.to(dev)
    out, lse = sparse_mla_fwd_fp8_interface(q8, k8, idxd, q_scale=qsv, kv_scale=ksv, sm_scale=scale, d_v=DV)
    dq, dkv = sparse_mla_bwd_fp8(q8, k8, qsv, ksv, out, dod, idxd, lse, sm_scale=scale)
    dq2, dkv2 = sparse_mla_bwd_fp8(q8, k8, qsv, ksv, out, dod, idxd, lse, sm_scale=scale)
    assert torch.equal(dq, dq2) and torch.equal(dkv, dkv2)
    outc, lsec = out.cpu(), lse.cpu()
    rqsv, rksv = rqs.expand(B, S).contiguous(), rks.expand(B, S).contiguous()
    b = 0
    toks = torch.tensor([0, 3, 255, 256, 1500, 2047, 3333, 4095])
    sub = lambda x: x[b:b + 1, toks].contiguous()
    ro, rl = orc.sparse_mla_fwd(sub(r8), rk8[b:b + 1], sub(idx), scale, DV, q_scale=sub(rqsv),
                                kv_scale=rksv[b:b + 1])
    assert_close(outc[b:b + 1, toks], ro, what="cfg4 out (sampled)")
    assert_close(lsec[b:b + 1, toks], rl, what="cfg4 lse2 (sampled)")
    rdq, _ = orc.sparse_mla_bwd(sub(r8), rk8[b:b + 1], sub(outc), sub(do), sub(idx), sub(lsec), scale, DV,
                                q_scale=sub(rqsv), kv_scale=rksv[b:b + 1])
    assert_mostly_close(dq.cpu()[b:b + 1, toks], rdq, what="cfg4 dq (sampled)")
    rows = torch.tensor([0, 9, 777, 2048, 4001])
    rt = (idx[b, :, 0, :, None] == rows[None, None, :]).any(-1).any(-1).nonzero()[:, 0]
    sel = lambda x: x[b:b + 1, rt].contiguous()
    _, rdkv = orc.sparse_mla_bwd(sel(r8), rk8[b:b + 1], sel(outc), sel(do), sel(idx), sel(lsec), scale, DV,
                                 q_scale=sel(rqsv), kv_scale=rksv[b:b + 1])
    assert_mostly_close(dkv.cpu()[b, rows], rdkv[0, rows], what="cfg4 dkv (sampled rows)")
    assert torch.isfinite(out).all() and torch.isfinite(dq).all() and torch.isfinite(dkv).all()
    col = dkv.double().sum(dim=(0, 1, 2)).cpu()
    expect_v = do.double().sum(dim=(0, 1, 2))
    scale_v = float(expect_v.norm() / DV ** 0.5)
    assert float((col[:DV] - expect_v).abs().max()) <= 2e-2 * scale_v, "sum_j dKV_j[:d_v] != sum dO"
