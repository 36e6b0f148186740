"""GPU tests of the SparseMLA backward with its inverse index built ahead.

``build_inverse_index`` builds the backward's kv-row -> entries index from the
indices alone (on a second stream, overlapping whatever runs meanwhile) and
``sparse_mla_bwd(..., inverse_index=...)`` then runs only the main kernel and
the dKV reduction.  The result must be the same bits as the one-call backward,
through the autograd functions, and across replays of a captured HIP graph.
"""
import pytest
import torch

from cppmega_amd import synthetic
from cppmega_amd.sparse_mla_ops import (SparseMLA, SparseMLA_FP8, build_inverse_index, side_stream,
                                        sparse_mla_bwd, sparse_mla_bwd_fp8, sparse_mla_fwd_fp8_interface,
                                        sparse_mla_fwd_interface)

pytestmark = pytest.mark.gpu


def _case(dev, B, S, H, G, D, DV, topk, seed):
    inp = synthetic.sparse_mla_inputs(B, S, H, D, DV, topk, std=0.5, seed=seed)
    q, kv, idx, do = (inp[k].to(dev) for k in ("q", "kv", "indices", "do"))
    if G > 1:
        g = torch.Generator().manual_seed(seed)
        kv = (torch.randn((B, S, G, D), generator=g) * 0.5).to(torch.bfloat16).to(dev)
        idx = idx.expand(B, S, G, topk).contiguous()
    return q, kv, idx, do, inp["scale"]


@pytest.mark.parametrize("B,S,H,G,D,DV,topk", [
    (2, 160, 32, 1, 128, 64, 64),
    (1, 96, 64, 2, 128, 128, 48),
    (1, 72, 32, 1, 192, 128, 40),
    (1, 64, 64, 1, 576, 512, 48),   # wide kernel: every chunk placed by the scatter
])
def test_prebuilt_index_is_bit_identical(dev, B, S, H, G, D, DV, topk):
    q, kv, idx, do, scale = _case(dev, B, S, H, G, D, DV, topk, seed=S + H)
    idx[0, S // 2, 0, 3:9] = idx[0, S // 2, 0, 0]   # a repeated row: serial placement of that chunk
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=scale, d_v=DV)
    dq0, dkv0 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale)
    ix = build_inverse_index(q, kv, idx, DV, stream=side_stream(dev))
    assert ix is not None and ix.event is not None
    dq1, dkv1 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale, inverse_index=ix)
    assert torch.equal(dq0, dq1) and torch.equal(dkv0, dkv1)
    ix2 = build_inverse_index(q, kv, idx, DV)   # on the current stream
    assert ix2.event is None
    dq2, dkv2 = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale, inverse_index=ix2)
    assert torch.equal(dq0, dq2) and torch.equal(dkv0, dkv2)
    with pytest.raises(ValueError, match="another call"):
        sparse_mla_bwd(q, kv, out, do, idx.clone(), lse, sm_scale=scale, inverse_index=ix2)


def test_prebuilt_index_fp8(dev):
    B, S, H, D, DV, topk = 2, 128, 32, 128, 64, 64
    g = torch.Generator(device=dev).manual_seed(3)
    q8 = torch.randn((B, S, H, D), generator=g, device=dev).to(torch.float8_e4m3fn)
    k8 = torch.randn((B, S, 1, D), generator=g, device=dev).to(torch.float8_e4m3fn)
    qs = torch.rand((B, S), generator=g, device=dev) + 0.25
    ks = torch.rand((B, S), generator=g, device=dev) + 0.25
    idx = synthetic.causal_indices(B, S, topk, seed=4).to(dev)
    do = torch.randn((B, S, H, DV), generator=g, device=dev).to(torch.bfloat16)
    out, lse = sparse_mla_fwd_fp8_interface(q8, k8, idx, q_scale=qs, kv_scale=ks, sm_scale=D ** -0.5, d_v=DV)
    dq0, dkv0 = sparse_mla_bwd_fp8(q8, k8, qs, ks, out, do, idx, lse, sm_scale=D ** -0.5)
    ix = build_inverse_index(q8, k8, idx, DV, stream=side_stream(dev))
    dq1, dkv1 = sparse_mla_bwd_fp8(q8, k8, qs, ks, out, do, idx, lse, sm_scale=D ** -0.5, inverse_index=ix)
    assert torch.equal(dq0, dq1) and torch.equal(dkv0, dkv1)


def test_autograd_builds_the_index_during_the_forward(dev):
    """SparseMLA.apply builds the index on the side stream in its forward; the
    gradients equal the direct backward's bit for bit (bf16 and FP8 classes)."""
    B, S, H, D, DV, topk = 1, 192, 32, 128, 64, 64
    q, kv, idx, do, scale = _case(dev, B, S, H, 1, D, DV, topk, seed=9)
    qd, kvd = q.clone().requires_grad_(), kv.clone().requires_grad_()
    out, lse = SparseMLA.apply(qd, kvd, idx, scale, DV)
    out.backward(do)
    out2, lse2 = sparse_mla_fwd_interface(q, kv, idx, sm_scale=scale, d_v=DV)
    dq, dkv = sparse_mla_bwd(q, kv, out2, do, idx, lse2, sm_scale=scale)
    assert torch.equal(out, out2) and torch.equal(qd.grad, dq) and torch.equal(kvd.grad, dkv)
    # no grad needed: no index is built
    with torch.no_grad():
        SparseMLA.apply(q, kv, idx, scale, DV)
    qf, kvf = q.clone().requires_grad_(), kv.clone().requires_grad_()
    of, _ = SparseMLA_FP8.apply(qf, kvf, idx, scale, DV)
    of.backward(do)
    assert torch.isfinite(qf.grad).all() and torch.isfinite(kvf.grad).all()


def test_prebuilt_index_in_a_graph(dev):
    """Forward, side-stream index build and backward captured in one HIP graph:
    three replays (eager work and syncs in between) each equal the eager result."""
    B, S, H, D, DV, topk = 2, 256, 32, 128, 64, 64
    q, kv, idx, do, scale = _case(dev, B, S, H, 1, D, DV, topk, seed=21)

    def step():
        ix = build_inverse_index(q, kv, idx, DV, stream=side_stream(dev))
        out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=scale, d_v=DV)
        return sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale, inverse_index=ix)

    ref = [t.clone() for t in step()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = step()
    for _ in range(3):
        torch.zeros(1 << 20, device=dev).sum().item()   # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res[0], ref[0]) and torch.equal(res[1], ref[1])


def test_no_prebuilt_index_for_several_passes(dev):
    """A backward that runs in several passes builds its index per pass:
    build_inverse_index returns None and the plain call still works."""
    B, S, H, D, DV, topk = 1, 128, 32, 128, 64, 64
    q, kv, idx, do, scale = _case(dev, B, S, H, 1, D, DV, topk, seed=5)
    cap = 32 * topk * (2 * D + 1)
    assert build_inverse_index(q, kv, idx, DV, pass_bytes=cap) is None
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=scale, d_v=DV)
    dq, _ = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale, pass_bytes=cap)
    dq1, _ = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale)
    assert torch.equal(dq, dq1)
    # an index built for another cap (here the default, one pass) is refused, not misused
    inv = build_inverse_index(q, kv, idx, DV)
    assert inv is not None
    with pytest.raises(ValueError, match="another call"):
        sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale, inverse_index=inv, pass_bytes=cap)
