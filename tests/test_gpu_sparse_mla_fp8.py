"""GPU parity of the FP8 (e4m3 tensorwise) SparseMLA path.

Against the FP8 oracle on identical quantised inputs the bar is the bf16 one
(2e-2 relative / 1e-2 absolute); against the bf16 oracle on the unquantised
inputs (cfg4-style data with 1% x20 outliers) the looser stated bound is
checked in tests/test_oracle_sparse_mla.py on the CPU and here on the GPU.
"""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.sparse_mla_ops import (SparseMLA_FP8, per_token_cast_to_fp8, sparse_mla_bwd_fp8,
                                        sparse_mla_fwd_fp8_interface)
from oracle import fp8 as ofp8
from oracle import sparse_mla as orc
from tests._util import assert_close, assert_mostly_close

pytestmark = pytest.mark.gpu

# FP8 vs bf16 reference, stated looser bound: relative L2 (Frobenius) error of
# out <= 0.15 on cfg4-style data (1% x20 outliers; the oracle measures 0.08-0.10
# there) and <= 0.05 on N(0, 0.5) data (oracle: ~0.025).
FP8_VS_BF16_REL_L2_OUTLIERS = 0.15
FP8_VS_BF16_REL_L2_GAUSS = 0.05


def _fp8_inputs(B, S, H, D, DV, topk, seed=21, outliers=True):
    if outliers:
        q = synthetic.outlier_values((B, S, H, D), seed).to(torch.bfloat16)
        kv = synthetic.outlier_values((B, S, 1, D), seed + 1).to(torch.bfloat16)
    else:
        q = (torch.randn((B, S, H, D), generator=torch.Generator().manual_seed(seed)) * 0.5).to(torch.bfloat16)
        kv = (torch.randn((B, S, 1, D), generator=torch.Generator().manual_seed(seed + 1)) * 0.5).to(torch.bfloat16)
    idx = synthetic.causal_indices(B, S, topk, seed=seed + 2)
    do = torch.randn((B, S, H, DV), generator=torch.Generator().manual_seed(seed + 3)).to(torch.bfloat16)
    return q, kv, idx, do


@pytest.mark.parametrize("outliers", [False, True])
@pytest.mark.parametrize("B,S,H,D,DV,topk", [(1, 128, 32, 128, 64, 64), (2, 96, 16, 128, 64, 40),
                                             (1, 64, 64, 128, 128, 96)])
def test_fp8_fwd_bwd_match_fp8_oracle(dev, B, S, H, D, DV, topk, outliers):
    q, kv, idx, do = _fp8_inputs(B, S, H, D, DV, topk, outliers=outliers)
    scale = D ** -0.5
    q8, qs = ofp8.tensorwise_quantize(q)
    k8, ks = ofp8.tensorwise_quantize(kv)
    qsv = qs.expand(B, S).contiguous()
    ksv = ks.expand(B, S).contiguous()
    out, lse = sparse_mla_fwd_fp8_interface(q8.to(dev), k8.to(dev), idx.to(dev), q_scale=qsv.to(dev),
                                            kv_scale=ksv.to(dev), sm_scale=scale, d_v=DV)
    ro, rl = orc.sparse_mla_fwd(q8, k8, idx, scale, DV, q_scale=qsv, kv_scale=ksv)
    assert_close(out, ro, what="fp8 out")
    assert_close(lse, rl, what="fp8 lse2")
    dq, dkv = sparse_mla_bwd_fp8(q8.to(dev), k8.to(dev), qsv.to(dev), ksv.to(dev), out, do.to(dev), idx.to(dev),
                                 lse, sm_scale=scale)
    rdq, rdkv = orc.sparse_mla_bwd(q8, k8, out.cpu(), do, idx, lse.cpu(), scale, DV, q_scale=qsv, kv_scale=ksv)
    check = assert_mostly_close if outliers else assert_close
    check(dq, rdq, what="fp8 dq")
    check(dkv, rdkv, what="fp8 dkv")


def test_sparse_mla_fp8_autograd_quantises_on_device(dev):
    B, S, H, D, DV, topk = 1, 128, 32, 128, 64, 64
    q, kv, idx, do = _fp8_inputs(B, S, H, D, DV, topk, seed=5)
    scale = D ** -0.5
    qd = q.to(dev).requires_grad_()
    kd = kv.to(dev).requires_grad_()
    out, lse = SparseMLA_FP8.apply(qd, kd, idx.to(dev), scale, DV)
    out.backward(do.to(dev))
    # the same quantisation on the CPU oracle is bit-exact, so this is the FP8 oracle path
    q8, qs = ofp8.tensorwise_quantize(q.reshape(B * S, -1))
    k8, ks = ofp8.tensorwise_quantize(kv.reshape(B * S, -1))
    q8, k8 = q8.reshape(q.shape), k8.reshape(kv.shape)
    qsv, ksv = qs.expand(B, S).contiguous(), ks.expand(B, S).contiguous()
    ro, _ = orc.sparse_mla_fwd(q8, k8, idx, scale, DV, q_scale=qsv, kv_scale=ksv)
    assert_close(out, ro, what="SparseMLA_FP8 out")
    rdq, rdkv = orc.sparse_mla_bwd(q8, k8, out.detach().cpu(), do, idx, lse.detach().cpu(), scale, DV,
                                   q_scale=qsv, kv_scale=ksv)
    assert_mostly_close(qd.grad, rdq, what="SparseMLA_FP8 dq")
    assert_mostly_close(kd.grad, rdkv, what="SparseMLA_FP8 dkv")
    # looser bound against the bf16 reference on the unquantised inputs
    bo, _ = orc.sparse_mla_fwd(q, kv, idx, scale, DV)
    rel = float((out.detach().float().cpu() - bo).norm() / bo.norm())
    assert rel <= FP8_VS_BF16_REL_L2_OUTLIERS, rel


def test_raw_fp8_without_scale_raises(dev):
    q = torch.zeros((1, 4, 16, 128), dtype=torch.float8_e4m3fn, device=dev)
    kv = torch.zeros((1, 4, 1, 128), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((1, 4, 1, 4), dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        SparseMLA_FP8.apply(q, kv, idx, 0.1, 64)


def test_per_token_cast_broadcasts_scale(dev):
    x = torch.randn(6, 40).to(torch.bfloat16)
    x8, s = per_token_cast_to_fp8(x.to(dev))
    r8, rs = ofp8.tensorwise_quantize(x)
    assert s.shape == (6,) and torch.all(s.cpu() == rs)
    assert torch.equal(x8.cpu().view(torch.uint8), r8.view(torch.uint8))


@pytest.mark.parametrize("mx", [False, True], ids=["e4m3", "mxfp8"])
@pytest.mark.parametrize("B,S,H,G,D,DV,topk", [(2, 96, 32, 1, 128, 64, 64), (1, 80, 64, 2, 128, 128, 48),
                                               (1, 64, 32, 1, 192, 128, 40)])
def test_fwd_with_v_dequantised_once_is_bit_identical(dev, mx, B, S, H, G, D, DV, topk):
    """dsa_sparse_mla_fwd_ws (V rows dequantised to bf16 once per call into the
    workspace) returns the same bits as dsa_sparse_mla_fwd (V converted per
    gather), with per-row and per-block scales and masked slots."""
    from cppmega_amd import _lib
    L = _lib.load()
    g = torch.Generator(device=dev).manual_seed(B * S + H + D)
    q8 = torch.randn((B, S, H, D), generator=g, device=dev).to(torch.float8_e4m3fn)
    k8 = torch.randn((B, S, G, D), generator=g, device=dev).to(torch.float8_e4m3fn)
    idx = synthetic.causal_indices(B, S, topk, seed=S).to(dev).expand(B, S, G, topk).contiguous()
    idx[:, 5, :, 3:9] = -1
    if mx:
        dtype = _lib.DTYPE_MXFP8
        qs = torch.exp2(torch.randint(-3, 2, (B, S, H, D // 32), generator=g, device=dev).float()) * 1.37
        ks = torch.exp2(torch.randint(-3, 2, (B, S, G, D // 32), generator=g, device=dev).float()) * 0.61
    else:
        dtype = _lib.DTYPE_E4M3
        qs = torch.rand((B, S), generator=g, device=dev) + 0.25
        ks = torch.rand((B, S), generator=g, device=dev) + 0.25
    outs = []
    for use_ws in (False, True):
        out = torch.empty((B, S, H, DV), dtype=torch.bfloat16, device=dev)
        lse = torch.empty((B, S, H), dtype=torch.float32, device=dev)
        st = torch.cuda.current_stream().cuda_stream
        args = (q8.data_ptr(), k8.data_ptr(), idx.data_ptr(), out.data_ptr(), lse.data_ptr(), B, S, S, H, G, D, DV,
                topk, D ** -0.5, dtype, qs.data_ptr(), ks.data_ptr())
        if use_ws:
            n = int(L.dsa_sparse_mla_fwd_workspace_size(B, S, G, D, DV, dtype))
            assert n >= B * S * G * DV * 2
            ws = torch.empty(n, dtype=torch.uint8, device=dev)
            _lib.check(L.dsa_sparse_mla_fwd_ws(*args, ws.data_ptr(), n, st), "dsa_sparse_mla_fwd_ws")
        else:
            _lib.check(L.dsa_sparse_mla_fwd(*args, st), "dsa_sparse_mla_fwd")
        outs.append((out, lse))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
