"""GPU kernels against the committed known-answer fixtures (tests/golden/),
which come from a float64 / pure-Python computation of the definitions and
need neither the oracle nor the reference at run time.

Bars: SparseMLA out / LSE / dq within 2e-2 rel / 1e-2 abs of exact math, dkv
within 2e-2 rel / 2e-2 abs (it sums many bf16-rounded P and dS terms, as the
reference kernels do); indexer within 1e-3 of the row scale; top-k indices
and e4m3 codes bit-exact.
"""
import numpy as np
import pytest
import torch

from cppmega_amd import index_scores, topk_indices
from cppmega_amd.sparse_mla_ops import sparse_mla_bwd, sparse_mla_fwd_interface, tensorwise_quantize
from tests._util import assert_close, bf16_from_bits, load_golden

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["sparse_mla_d128.npz", "sparse_mla_d64_g2.npz"])
def test_sparse_mla_known_answer(dev, name):
    print(f"golden {name}", flush=True)
    g = load_golden(name)
    q = bf16_from_bits(g["q_bits"]).to(dev)
    kv = bf16_from_bits(g["kv_bits"]).to(dev)
    do = bf16_from_bits(g["do_bits"]).to(dev)
    idx = torch.from_numpy(g["indices"]).to(torch.int32).to(dev)
    scale, d_v = float(g["scale"]), int(g["d_v"])
    out, lse = sparse_mla_fwd_interface(q, kv, idx, sm_scale=scale, d_v=d_v)
    assert_close(out, torch.from_numpy(g["out"]), what="out")
    assert_close(lse, torch.from_numpy(g["lse2"]), what="lse2")
    dq, dkv = sparse_mla_bwd(q, kv, out, do, idx, lse, sm_scale=scale, d_v=d_v)
    assert_close(dq, torch.from_numpy(g["dq"]), what="dq")
    assert_close(dkv, torch.from_numpy(g["dkv"]), atol=2e-2, what="dkv")


def test_indexer_known_answer(dev):
    g = load_golden("indexer.npz")
    q = bf16_from_bits(g["q_bits"]).to(dev)
    k = bf16_from_bits(g["k_bits"]).to(dev)
    w = torch.from_numpy(g["w"]).to(dev)
    got = index_scores(q, w, k).cpu().double()
    ref = torch.from_numpy(g["scores"])
    assert float((got - ref).abs().max() / ref.abs().max()) < 1e-3


def test_topk_known_answer(dev):
    g = load_golden("topk.npz")
    s = torch.from_numpy(g["scores"]).to(dev)
    st = torch.from_numpy(g["starts"]).to(dev)
    en = torch.from_numpy(g["ends"]).to(dev)
    got = topk_indices(s, int(g["topk"]), causal=False, starts=st, ends=en).cpu().numpy()
    np.testing.assert_array_equal(got, g["out"])


def test_fp8_quantize_known_answer(dev):
    g = load_golden("fp8.npz")
    x8, si = tensorwise_quantize(torch.from_numpy(g["x"]).to(dev))
    np.testing.assert_array_equal(x8.view(torch.uint8).cpu().numpy(), g["codes"])
    assert float(si) == float(g["scale_inv"])
