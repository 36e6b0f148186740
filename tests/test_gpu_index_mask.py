"""GPU parity of the top-k index mask (dsa_topk_index_mask through the C-ABI):
bit-exact against the oracle, in both the in-place scatter and the whole-row
fill form, and identical across replays of a captured HIP graph."""
import pytest
import torch

from cppmega_amd import scatter_topk_into_index_mask, topk_index_mask
from oracle import index_mask as oim
from tests._util import load_golden

pytestmark = pytest.mark.gpu


def _same(a, e):
    assert torch.equal(a.cpu(), e), f"{int((a.cpu() != e).sum())} elements differ"


def test_fixture_scatter(dev):
    z = load_golden("index_mask.npz")
    idx = torch.from_numpy(z["idx"])
    s0, s1, sk = int(z["s0"]), int(z["s1"]), int(z["s_kv"])
    for dt in (torch.int64, torch.int32):
        mask = torch.full((2, 64, sk), float("-inf"), device=dev)
        out = scatter_topk_into_index_mask(mask, idx.to(dt).to(dev), s0, s1)
        assert out.data_ptr() == mask.data_ptr()
        _same(out, torch.from_numpy(z["mask"]))


@pytest.mark.parametrize("b,sq,sk,topk", [(2, 4096, 4096, 256), (1, 300, 1001, 40), (3, 17, 5, 9)])
def test_full_mask_matches_oracle(dev, b, sq, sk, topk):
    g = torch.Generator().manual_seed(sq + sk)
    idx = torch.randint(-1, sk + 2, (b, sq, topk), generator=g)   # sentinels and past-the-row columns
    got = topk_index_mask(idx.to(dev), sk)
    _same(got, oim.topk_index_mask(idx, sk))
    # scatter into a pre-filled mask gives the same result
    pre = torch.full((b, sq, sk), float("-inf"), device=dev)
    _same(scatter_topk_into_index_mask(pre, idx.to(dev)), oim.topk_index_mask(idx, sk))


def test_scatter_leaves_other_rows(dev):
    g = torch.Generator().manual_seed(7)
    base = torch.randn(2, 40, 64, generator=g)
    idx = torch.randint(-1, 64, (2, 10, 5), generator=g)
    got = scatter_topk_into_index_mask(base.clone().to(dev), idx.to(dev), 20, 30)
    _same(got, oim.scatter_topk_into_index_mask(base, idx, 20, 30))


def test_graph_replays(dev):
    """Captured in a HIP graph and replayed (with eager work between replays):
    every replay equals the eager result (no host sync inside the call)."""
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(-1, 256, (2, 64, 8), generator=g).to(dev)
    ref = oim.topk_index_mask(idx.cpu(), 256)
    out = torch.empty((2, 64, 256), device=dev)
    topk_index_mask(idx, 256, out=out)           # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        topk_index_mask(idx, 256, out=out)
    for _ in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _same(out, ref)
