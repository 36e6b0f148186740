"""Pins the SparseMLA oracle (CPU): known-answer fixtures, float64 autograd of
the closed form, gradcheck, closed-form special cases and invariants.  A few
tests plant a mistake in the oracle's inputs and check that the same
comparison catches it."""
from __future__ import annotations

import pytest
import torch

from oracle import sparse_mla as osm
from tests._util import assert_close, bf16_from_bits, load_golden

GOLDEN = ["sparse_mla_d128.npz", "sparse_mla_d64_g2.npz"]


def _golden_inputs(name):
    g = load_golden(name)
    q = bf16_from_bits(g["q_bits"])
    kv = bf16_from_bits(g["kv_bits"])
    do = bf16_from_bits(g["do_bits"])
    idx = torch.from_numpy(g["indices"]).to(torch.int32)
    return g, q, kv, do, idx, float(g["scale"]), int(g["d_v"])


@pytest.mark.parametrize("name", GOLDEN)
def test_fwd_matches_golden_exact_math(name):
    g, q, kv, do, idx, scale, d_v = _golden_inputs(name)
    out, lse = osm.sparse_mla_fwd(q, kv, idx, sm_scale=scale, d_v=d_v, round_p_bf16=False)
    assert_close(out, torch.from_numpy(g["out"]), rtol=1e-5, atol=1e-6, what="out")
    assert_close(lse, torch.from_numpy(g["lse2"]), rtol=1e-6, atol=1e-5, what="lse2")


@pytest.mark.parametrize("name", GOLDEN)
def test_fwd_bf16_rounding_within_contract(name):
    g, q, kv, do, idx, scale, d_v = _golden_inputs(name)
    out, lse = osm.sparse_mla_fwd(q, kv, idx, sm_scale=scale, d_v=d_v)
    assert_close(out, torch.from_numpy(g["out"]), what="out (P in bf16)")
    assert_close(lse, torch.from_numpy(g["lse2"]), what="lse2")


@pytest.mark.parametrize("name", GOLDEN)
def test_bwd_matches_golden(name):
    g, q, kv, do, idx, scale, d_v = _golden_inputs(name)
    o = torch.from_numpy(g["out"])
    lse = torch.from_numpy(g["lse2"])
    dq, dkv = osm.sparse_mla_bwd(q, kv, o, do, idx, lse, sm_scale=scale, d_v=d_v, round_bf16=False)
    assert_close(dq, torch.from_numpy(g["dq"]), rtol=1e-4, atol=1e-5, what="dq")
    assert_close(dkv, torch.from_numpy(g["dkv"]), rtol=1e-4, atol=1e-5, what="dkv")
    # the reference kernels' arithmetic (bf16 O, P and dS) against exact math: dKV sums
    # many bf16-rounded terms, so its band here is atol 2e-2 (the 2e-2 / 1e-2 contract
    # applies between implementations that round the same way)
    o_b = o.to(torch.bfloat16)
    dq2, dkv2 = osm.sparse_mla_bwd(q, kv, o_b, do, idx, lse, sm_scale=scale, d_v=d_v)
    assert_close(dq2, torch.from_numpy(g["dq"]), what="dq (bf16 P/dS)")
    assert_close(dkv2, torch.from_numpy(g["dkv"]), atol=2e-2, what="dkv (bf16 P/dS)")


@pytest.mark.parametrize("name", GOLDEN)
def test_autograd_f64_matches_golden(name):
    g, q, kv, do, idx, scale, d_v = _golden_inputs(name)
    qd = q.double().requires_grad_(True)
    kvd = kv.double().requires_grad_(True)
    out, lse = osm.sparse_mla_autograd_f64(qd, kvd, idx, sm_scale=scale, d_v=d_v)
    assert_close(out, torch.from_numpy(g["out"]).double(), rtol=1e-6, atol=1e-7, what="out")
    assert_close(lse, torch.from_numpy(g["lse2"]).double(), rtol=1e-6, atol=1e-6, what="lse2")
    out.backward(do.double())
    assert_close(qd.grad, torch.from_numpy(g["dq"]).double(), rtol=1e-5, atol=1e-6, what="dq")
    assert_close(kvd.grad, torch.from_numpy(g["dkv"]).double(), rtol=1e-5, atol=1e-6, what="dkv")


@pytest.mark.parametrize("mistake", ["lse_shift", "wrong_scale", "transposed_heads", "kv_halves_swapped"])
def test_planted_mistakes_are_caught(mistake):
    """Each plausible slip (a shifted LSE, a wrong softmax scale, heads read in the
    wrong order, the latent and rope halves of kv exchanged) moves the backward
    outside the tolerance band of the known answer."""
    g, q, kv, do, idx, scale, d_v = _golden_inputs("sparse_mla_d128.npz")
    o = torch.from_numpy(g["out"])
    lse = torch.from_numpy(g["lse2"])
    if mistake == "lse_shift":
        lse = lse + 0.25
    elif mistake == "wrong_scale":
        scale = scale * 1.1
    elif mistake == "transposed_heads":
        q = q.flip(2).contiguous()
    elif mistake == "kv_halves_swapped":
        kv = torch.cat([kv[..., 64:], kv[..., :64]], dim=-1).contiguous()
    dq, dkv = osm.sparse_mla_bwd(q, kv, o, do, idx, lse, sm_scale=scale, d_v=d_v, round_bf16=False)
    with pytest.raises(AssertionError):
        assert_close(dq, torch.from_numpy(g["dq"]), what="dq")
        assert_close(dkv, torch.from_numpy(g["dkv"]), what="dkv")


def _rand_case(B=2, S=6, Skv=9, H=4, G=2, D=16, d_v=8, K=7, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, D, generator=gen, dtype=torch.float64)
    kv = torch.randn(B, Skv, G, D, generator=gen, dtype=torch.float64)
    idx = torch.randint(-2, Skv + 2, (B, S, G, K), generator=gen, dtype=torch.int32)
    idx[0, 0, 0] = -1  # one fully masked (token, group)
    do = torch.randn(B, S, H, d_v, generator=gen, dtype=torch.float64)
    return q, kv, idx, do


def test_explicit_bwd_matches_f64_autograd_random():
    q, kv, idx, do = _rand_case()
    d_v = do.shape[-1]
    qd, kvd = q.clone().requires_grad_(True), kv.clone().requires_grad_(True)
    out_ref, lse_ref = osm.sparse_mla_autograd_f64(qd, kvd, idx, d_v=d_v)
    out_ref.backward(do)
    out, lse = osm.sparse_mla_fwd(q.float(), kv.float(), idx, d_v=d_v, round_p_bf16=False)
    assert_close(out, out_ref, rtol=1e-5, atol=1e-6, what="out")
    assert_close(lse, lse_ref, rtol=1e-5, atol=1e-5, what="lse2")
    dq, dkv = osm.sparse_mla_bwd(q.float(), kv.float(), out, do.float(), idx, lse, d_v=d_v, round_bf16=False)
    assert_close(dq, qd.grad, rtol=1e-4, atol=1e-5, what="dq")
    assert_close(dkv, kvd.grad, rtol=1e-4, atol=1e-5, what="dkv")
    # the fully masked (token, group) contributes nothing and gets zero gradient
    hpg = q.shape[2] // kv.shape[2]
    assert torch.all(out[0, 0, :hpg] == 0) and torch.all(torch.isneginf(lse[0, 0, :hpg]))
    assert torch.all(dq[0, 0, :hpg] == 0)


def test_gradcheck_closed_form():
    q, kv, idx, _ = _rand_case(B=1, S=3, Skv=5, H=2, G=1, D=4, d_v=3, K=4, seed=3)
    idx[0, 0, 0, 0] = 0  # keep at least one valid slot in the first row

    def f(qq, kk):
        return osm.sparse_mla_autograd_f64(qq, kk, idx, d_v=3)[0]

    assert torch.autograd.gradcheck(f, (q.requires_grad_(True), kv.requires_grad_(True)), eps=1e-6, atol=1e-6)


def test_single_valid_index_closed_form():
    q, kv, idx, _ = _rand_case(B=1, S=4, Skv=6, H=2, G=1, D=8, d_v=4, K=5, seed=5)
    idx.fill_(-1)
    idx[0, :, 0, 2] = torch.tensor([0, 3, 5, 1], dtype=torch.int32)
    out, lse = osm.sparse_mla_fwd(q.float(), kv.float(), idx, d_v=4, round_p_bf16=False)
    rows = kv[0, idx[0, :, 0, 2].long(), 0]                        # [S, D]
    assert_close(out[0], rows[:, None, :4].expand(-1, 2, -1), rtol=0, atol=1e-6, what="out = V[idx]")
    expect = (q[0] * rows[:, None, :]).sum(-1) * (8 ** -0.5) * osm.LOG2E
    assert_close(lse[0], expect, rtol=1e-6, atol=1e-5, what="lse2 = scale q.k log2e")


def test_equal_scores_give_mean_of_values_and_duplicates_count():
    q, kv, idx, _ = _rand_case(B=1, S=2, Skv=6, H=2, G=1, D=8, d_v=4, K=4, seed=7)
    q.zero_()
    idx[0, 0, 0] = torch.tensor([1, 2, 4, -1], dtype=torch.int32)
    idx[0, 1, 0] = torch.tensor([3, 3, 5, 9], dtype=torch.int32)   # duplicate 3, 9 out of range
    out, lse = osm.sparse_mla_fwd(q.float(), kv.float(), idx, d_v=4, round_p_bf16=False)
    v = kv[0, :, 0, :4]
    assert_close(out[0, 0, 0], (v[1] + v[2] + v[4]) / 3, rtol=0, atol=1e-6, what="mean of V")
    assert_close(out[0, 1, 0], (2 * v[3] + v[5]) / 3, rtol=0, atol=1e-6, what="duplicates counted")
    assert_close(lse[0, 1], torch.full((2,), torch.log2(torch.tensor(3.0)).item()), rtol=0, atol=1e-6,
                 what="lse2 = log2(n)")


def test_slot_order_invariance():
    q, kv, idx, do = _rand_case(seed=9)
    perm = torch.randperm(idx.shape[-1], generator=torch.Generator().manual_seed(1))
    a = osm.sparse_mla_fwd(q.float(), kv.float(), idx, d_v=8, round_p_bf16=False)
    b = osm.sparse_mla_fwd(q.float(), kv.float(), idx[..., perm].contiguous(), d_v=8, round_p_bf16=False)
    assert_close(a[0], b[0], rtol=1e-6, atol=1e-6, what="out")
    assert_close(a[1], b[1], rtol=1e-6, atol=1e-6, what="lse2")


def test_ds_sums_to_zero_over_slots():
    """sum_s dS_s = 0 per (token, head), seen through dq: adding the same vector c
    to the rope tail of every key (a part V does not read) shifts all scores of a
    (token, head) equally, so the softmax and dS are unchanged and
    dq' - dq = scale * (sum_s dS_s) c must vanish."""
    q, kv, idx, do = _rand_case(B=1, S=3, Skv=4, H=2, G=1, D=6, d_v=3, K=4, seed=11)
    idx[:] = torch.tensor([0, 1, 2, 3], dtype=torch.int32)  # every token sees every row once
    out, lse = osm.sparse_mla_fwd(q.float(), kv.float(), idx, d_v=3, round_p_bf16=False)
    dq, _ = osm.sparse_mla_bwd(q.float(), kv.float(), out, do.float(), idx, lse, d_v=3, round_bf16=False)
    kv2 = kv.clone()
    kv2[..., 3:] += torch.tensor([0.7, -1.3, 2.1], dtype=kv.dtype)
    out2, lse2 = osm.sparse_mla_fwd(q.float(), kv2.float(), idx, d_v=3, round_p_bf16=False)
    dq2, _ = osm.sparse_mla_bwd(q.float(), kv2.float(), out2, do.float(), idx, lse2, d_v=3, round_bf16=False)
    assert_close(out2, out, rtol=1e-5, atol=1e-6, what="softmax shift invariance")
    assert_close(dq2, dq, rtol=1e-4, atol=1e-5, what="sum_s dS_s = 0")


def test_three_dim_inputs():
    q, kv, idx, do = _rand_case(B=1, seed=13)
    out4, lse4 = osm.sparse_mla_fwd(q.float(), kv.float(), idx, d_v=8)
    out3, lse3 = osm.sparse_mla_fwd(q[0].float(), kv[0].float(), idx[0], d_v=8)
    assert out3.dim() == 3 and torch.equal(out3, out4[0]) and torch.equal(lse3, lse4[0])


def test_fp8_reduces_to_dequantised_bf16():
    """e4m3 inputs with unit scales: the fp8 oracle equals the bf16 oracle on the decoded values."""
    q, kv, idx, do = _rand_case(B=1, S=5, Skv=7, H=2, G=1, D=16, d_v=8, K=6, seed=17)
    q8 = (q * 4).float().to(torch.float8_e4m3fn)
    kv8 = (kv * 4).float().to(torch.float8_e4m3fn)
    ones_q, ones_kv = torch.ones(1, 5), torch.ones(1, 7)
    a = osm.sparse_mla_fwd(q8, kv8, idx, d_v=8, q_scale=ones_q, kv_scale=ones_kv)
    b = osm.sparse_mla_fwd(q8.float(), kv8.float().to(torch.bfloat16), idx, d_v=8)
    assert torch.equal(a[1], b[1]) and torch.equal(a[0], b[0])
    # scales enter multiplicatively: the score path sees q_scale * kv_scale
    qs, ks = torch.full((1, 5), 0.25), torch.full((1, 7), 0.5)
    c = osm.sparse_mla_fwd(q8, kv8, idx, d_v=8, q_scale=qs, kv_scale=ks)
    d = osm.sparse_mla_fwd((q8.float() * 0.25), (kv8.float() * 0.5).to(torch.bfloat16), idx, d_v=8)
    assert_close(c[1], d[1], rtol=1e-6, atol=1e-6, what="lse2 with scales")
    assert_close(c[0], d[0], rtol=1e-6, atol=1e-6, what="out with scales")


@pytest.mark.parametrize("outliers,bound", [(False, 0.05), (True, 0.15)])
def test_fp8_vs_bf16_stated_bound(outliers, bound):
    """The stated FP8 bound: relative L2 of the e4m3-tensorwise output against the
    bf16 result on the same (unquantised) inputs."""
    from cppmega_amd import synthetic
    from oracle import fp8 as of8
    B, S, H, D, DV, K = 1, 64, 16, 128, 64, 32
    if outliers:
        q = synthetic.outlier_values((B, S, H, D), 31).to(torch.bfloat16)
        kv = synthetic.outlier_values((B, S, 1, D), 32).to(torch.bfloat16)
    else:
        g = torch.Generator().manual_seed(31)
        q = (torch.randn((B, S, H, D), generator=g) * 0.5).to(torch.bfloat16)
        kv = (torch.randn((B, S, 1, D), generator=g) * 0.5).to(torch.bfloat16)
    idx = synthetic.causal_indices(B, S, K, seed=33)
    ref, _ = osm.sparse_mla_fwd(q, kv, idx, d_v=DV)
    q8, qsi = of8.tensorwise_quantize(q)
    kv8, ksi = of8.tensorwise_quantize(kv)
    out8, _ = osm.sparse_mla_fwd(q8, kv8, idx, d_v=DV, q_scale=qsi.expand(B, S), kv_scale=ksi.expand(B, S))
    rel = float((out8 - ref).norm() / ref.norm())
    assert rel <= bound, rel


def test_flop_conventions():
    # cfg2 figures quoted by the reference's benchmark scripts
    assert osm.flops_fwd(2, 4096, 32, 256, 128, 64) == 25_769_803_776
    assert osm.flops_bwd(2, 4096, 32, 256, 128, 64) == 68_719_476_736


# ---------------------------------------------------------------------------
# MXFP8 block-scaled forward
# ---------------------------------------------------------------------------
def _mx_inputs(B=1, S=24, H=16, D=128, G=1, K=20, seed=5):
    from cppmega_amd import synthetic
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, S, H, D), generator=g)
    kv = torch.randn((B, S, G, D), generator=g)
    idx = synthetic.causal_indices(B, S, K, seed=seed + 1).expand(B, S, G, K).contiguous()
    return q, kv, idx


def test_mxfp8_uniform_block_scales_equal_tensorwise():
    """Equal scales in every block reduce the block-scaled forward to the
    tensorwise FP8 forward (pinned separately) with those scales."""
    q, kv, idx = _mx_inputs()
    q8 = q.clamp(-400, 400).to(torch.float8_e4m3fn)
    kv8 = kv.clamp(-400, 400).to(torch.float8_e4m3fn)
    B, S, H, D = q.shape
    qs, ks = 0.37, 1.9
    qsb = torch.full((B, S, H, D // 32), qs)
    ksb = torch.full((B, S, 1, D // 32), ks)
    o_mx, l_mx = osm.sparse_mla_fwd_mxfp8(q8, kv8, qsb, ksb, idx, 0.1, 64)
    o_t, l_t = osm.sparse_mla_fwd(q8, kv8, idx, 0.1, 64, q_scale=torch.full((B, S), qs),
                                  kv_scale=torch.full((B, S), ks))
    assert torch.allclose(o_mx, o_t, atol=1e-6, rtol=1e-5) and torch.allclose(l_mx, l_t, atol=1e-5)


def test_mxfp8_power_of_two_scales_equal_bf16_on_dequantised_inputs():
    """With power-of-two (MX) scales the dequantised values are exact in bf16, so
    the block-scaled forward equals the bf16 forward on the dequantised tensors
    (scores up to fp32 summation order)."""
    q, kv, idx = _mx_inputs(G=2, H=32)
    q8, qs = osm.mxfp8_quantize(q)
    kv8, ks = osm.mxfp8_quantize(kv)
    o_mx, l_mx = osm.sparse_mla_fwd_mxfp8(q8, kv8, qs, ks, idx, 0.09, 64)
    qd = osm.dequantize_blockwise(q8, qs)
    kvd = osm.dequantize_blockwise(kv8, ks)
    assert torch.equal(qd.float(), osm.dequantize_blockwise(q8, qs, out_dtype=torch.float32))  # exact in bf16
    o_b, l_b = osm.sparse_mla_fwd(qd, kvd, idx, 0.09, 64)
    assert torch.allclose(o_mx, o_b, atol=2e-6, rtol=1e-5) and torch.allclose(l_mx, l_b, atol=2e-5)


def test_mxfp8_block_scale_placement_is_pinned():
    """Planted mistake: scaling every block by block 0's kv scale changes the result."""
    q, kv, idx = _mx_inputs()
    q8, qs = osm.mxfp8_quantize(q * torch.linspace(0.1, 10, 128))
    kv8, ks = osm.mxfp8_quantize(kv * torch.linspace(10, 0.1, 128))
    o, _ = osm.sparse_mla_fwd_mxfp8(q8, kv8, qs, ks, idx, 0.09, 64)
    o_bad, _ = osm.sparse_mla_fwd_mxfp8(q8, kv8, qs, ks[..., :1].expand_as(ks).contiguous(), idx, 0.09, 64)
    assert not torch.allclose(o, o_bad, atol=1e-2)


def test_mxfp8_quantizer_closed_form():
    """Shared exponent floor(log2 amax) - 8: a block with amax 3.0 gets scale 2^-7;
    values that are e4m3-representable multiples of the scale round-trip exactly."""
    x = torch.zeros(1, 64)
    x[0, :32] = torch.tensor([3.0, -1.5, 0.75, 2.0 ** -6] + [0.0] * 28)
    x[0, 32:] = 0.0
    d, s = osm.mxfp8_quantize(x)
    assert float(s[0, 0]) == 2.0 ** -7 and float(s[0, 1]) == 1.0
    back = osm.dequantize_blockwise(d, s, out_dtype=torch.float32)
    assert torch.equal(back, x)
