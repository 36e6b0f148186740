"""Host-side behaviour that needs no GPU: the product path refuses CPU tensors
(no fallback), the reference's assertion / error contract, the IndexCache
schedule wired into a stand-in Megatron dsa module, and bench.py's one-GPU
rule."""
from __future__ import annotations

import ast
import os
import subprocess
import sys
import types

import pytest
import torch

import cppmega_amd
from cppmega_amd import index_cache_patch as icp
from cppmega_amd.dsa_indexer_fused_patch import compute_index_scores_fused_bf16, index_scores
from cppmega_amd.dsa_topk import topk_indices
from cppmega_amd.sparse_mla_ops import (SparseMLA, SparseMLA_FP8, sparse_mla_bwd, sparse_mla_fwd_interface,
                                        sparse_mla_fwd_fp8_interface)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _inputs(B=1, S=8, H=16, D=128, K=16):
    q = torch.randn(B, S, H, D).to(torch.bfloat16)
    kv = torch.randn(B, S, 1, D).to(torch.bfloat16)
    idx = torch.zeros(B, S, 1, K, dtype=torch.int32)
    return q, kv, idx


def test_product_path_has_no_cpu_fallback():
    q, kv, idx = _inputs()
    with pytest.raises(RuntimeError, match="gfx950"):
        sparse_mla_fwd_interface(q, kv, idx, d_v=64)
    with pytest.raises(RuntimeError, match="gfx950"):
        SparseMLA.apply(q, kv, idx, 0.1, 64)
    with pytest.raises(RuntimeError, match="gfx950"):
        compute_index_scores_fused_bf16(torch.randn(8, 1, 16, 64).bfloat16(), torch.randn(8, 1, 16),
                                        torch.randn(8, 1, 64).bfloat16())
    with pytest.raises(RuntimeError, match="gfx950"):
        topk_indices(torch.randn(1, 8, 8), 4)


def test_product_package_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "cppmega_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if not f.endswith(".py"):
                continue
            tree = ast.parse(open(os.path.join(dirpath, f)).read())
            for node in ast.walk(tree):
                names = []
                if isinstance(node, ast.Import):
                    names = [a.name for a in node.names]
                elif isinstance(node, ast.ImportFrom) and node.module:
                    names = [node.module]
                assert not any(n == "oracle" or n.startswith("oracle.") for n in names), f"{f} imports oracle"


def test_reference_assertions():
    q, kv, idx = _inputs()
    with pytest.raises(AssertionError):
        sparse_mla_fwd_interface(q, kv, idx, d_v=64, return_p_sum=True)
    with pytest.raises(AssertionError):
        sparse_mla_fwd_interface(q, kv[..., :64].contiguous(), idx, d_v=64)      # dim mismatch
    with pytest.raises(AssertionError):
        sparse_mla_fwd_interface(q, kv, idx, d_v=256)                             # d_v > d_qk
    with pytest.raises(AssertionError):
        sparse_mla_fwd_interface(q, kv, idx.long(), d_v=64)                       # int64 indices
    with pytest.raises(AssertionError):
        sparse_mla_fwd_interface(q.transpose(1, 2), kv, idx, d_v=64)             # non-contiguous
    with pytest.raises(AssertionError):
        sparse_mla_bwd(q, kv, q[..., :64], q[..., :64], idx.long(), torch.zeros(1, 8, 16))


def test_raw_fp8_without_scale_is_a_value_error():
    q, kv, idx = _inputs()
    with pytest.raises(ValueError):
        SparseMLA_FP8.apply(q.float().to(torch.float8_e4m3fn), kv.float().to(torch.float8_e4m3fn), idx, 0.1, 64)
    with pytest.raises(RuntimeError, match="gfx950"):
        sparse_mla_fwd_fp8_interface(q, kv, idx, d_v=64)                          # quantises on the GPU only


def test_indexer_shape_checks():
    with pytest.raises(AssertionError):
        index_scores(torch.randn(8, 1, 16, 64).bfloat16(), torch.randn(8, 1, 16), torch.randn(8, 2, 64).bfloat16())
    with pytest.raises(TypeError):
        index_scores(torch.randn(8, 1, 16, 64), torch.randn(8, 1, 16), torch.randn(8, 1, 64))


def test_package_exports():
    from cppmega_amd import sparse_mla_ops
    for name in ("SparseMLA", "SparseMLA_FP8", "sparse_mla_fwd_interface", "sparse_mla_bwd",
                 "sparse_mla_fwd_fp8_interface", "sparse_mla_bwd_fp8", "per_token_cast_to_fp8",
                 "sparse_mla_as_unfused_dsa", "sparse_mla_fp8_as_unfused_dsa"):
        assert hasattr(sparse_mla_ops, name), name
    assert cppmega_amd is not None


def test_sparse_mla_patch_rebinds_megatron_module(monkeypatch):
    from cppmega_amd import sparse_mla_ops as smo

    def orig(*a, **k):
        return None

    mod = types.SimpleNamespace(__name__="fake_dsa", unfused_dsa_fn=orig, SparseMLA=object)
    monkeypatch.setenv("CPPMEGA_DSA_FP8_ATTENTION", "0")
    assert smo.apply_sparse_mla_patch(dsa_module=mod)
    assert mod.unfused_dsa_fn is smo.sparse_mla_as_unfused_dsa and mod.SparseMLA is smo.SparseMLA
    mod2 = types.SimpleNamespace(__name__="fake_dsa2", unfused_dsa_fn=orig, SparseMLA=object)
    assert smo.apply_sparse_mla_patch(fp8=True, dsa_module=mod2)
    assert mod2.unfused_dsa_fn is smo.sparse_mla_fp8_as_unfused_dsa and mod2.SparseMLA is smo.SparseMLA_FP8
    assert not smo.apply_sparse_mla_patch(dsa_module=types.SimpleNamespace())


# ---------------------------------------------------------------------------
# IndexCache schedule
# ---------------------------------------------------------------------------
def test_schedule_semantics():
    s = icp.IndexCacheSchedule(full_ranks={0, 3, 6})
    assert [s.is_full(r) for r in range(9)] == [r in (0, 3, 6) for r in range(9)]
    assert s.savings(9) == (3, 6, 66)
    s.begin_layer(0)
    assert s.step == 0
    s.store(0, "i0")
    assert s.lookup(1) == "i0" and s.lookup(2) == "i0"
    s.store(3, "i3")
    assert s.lookup(4) == "i3" and s.lookup(8) == "i3"
    s.begin_layer(0)                      # next micro-batch clears the cache
    assert s.step == 1 and s.lookup(5) is None
    assert icp.parse_full_ranks(" 1, 4 ,7,") == {1, 4, 7}


class _FakeIndexer:
    index_topk = 2
    pg_collection = None

    def forward_before_topk(self, x, qr, packed):
        return x, qr, packed


def _fake_dsa_module(calls):
    class DSAttention:
        def __init__(self, layer_number):
            self.layer_number = layer_number
            self.indexer = _FakeIndexer()
            self.config = types.SimpleNamespace(kv_lora_rank=0, qk_pos_emb_head_dim=0)
            self.softmax_scale = 0.5

        def forward(self, query, key, value, attention_mask, x, qr, **kw):
            calls.append(("full", self._ic_dsa_rank))
            return "full-out"

    def run_sparse(**kw):
        calls.append(("shared", kw["topk_indices"]))
        return "shared-out", "path"

    return types.SimpleNamespace(
        DSAttention=DSAttention,
        _run_sparse_attention=run_sparse,
        _ensure_sbhd=lambda t, name: (t, None),
        _normalize_dsattention_output_rank=lambda out, nd: out,
        _build_dsattention_forward_mask=lambda **kw: (None, None),
        _normalize_cp_comm_type=lambda t: t,
    )


def test_index_cache_patch_full_shared_promote(monkeypatch):
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "1,3")
    monkeypatch.setattr(icp, "_SCHEDULE", None)
    picks = []

    def fake_topk(q, k, w, topk, mask=None, use_relu=False, **kw):
        picks.append(use_relu)
        return None, f"idx-from-{int(q)}"

    monkeypatch.setattr(icp, "fused_qk_topk_naive", fake_topk)
    calls = []
    mod = _fake_dsa_module(calls)
    assert icp.apply_index_cache_patch(dsa_module=mod)
    assert icp.apply_index_cache_patch(dsa_module=mod)          # second call: no-op
    layers = [mod.DSAttention(i) for i in range(5)]
    q4 = torch.zeros(4, 1, 2, 8)
    for step in range(2):
        calls.clear()
        outs = [layer.forward(q4, q4, None, None, torch.tensor(10 * step + i), torch.tensor(0), None)
                for i, layer in enumerate(layers)]
        # rank 0 has no preceding Full rank: promoted; 1 and 3 are Full; 2 reuses 1, 4 reuses 3
        assert outs == ["full-out", "full-out", "shared-out", "full-out", "shared-out"]
        assert calls == [("full", 0), ("full", 1), ("shared", f"idx-from-{10 * step + 1}"), ("full", 3),
                         ("shared", f"idx-from-{10 * step + 3}")]
    assert layers[0]._ic_is_full and not layers[2]._ic_is_full
    assert picks and not any(picks)            # relu defaults to the config's False, as the reference


def test_index_cache_full_layer_computes_indices_once(monkeypatch):
    """When the Full layer's own forward calls the dsa module's
    fused_qk_topk_naive (as Megatron's DSAttention does), IndexCache caches the
    indices of that call: no second indexer + top-k pass, and the Shared layers
    get exactly the Full layer's (masked) picks."""
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0,3")
    monkeypatch.setattr(icp, "_SCHEDULE", None)

    def rederive(*a, **k):
        raise AssertionError("the Full layer must not run a second indexer + top-k pass")

    monkeypatch.setattr(icp, "fused_qk_topk_naive", rederive)
    calls = []
    mod = _fake_dsa_module(calls)
    topk_calls = []

    def module_topk(q, k, w, topk, mask=None, **kw):
        topk_calls.append(int(q))
        return None, torch.tensor([int(q), -1])

    mod.fused_qk_topk_naive = module_topk

    def forward(self, query, key, value, attention_mask, x, qr, **kw):
        _, idx = mod.fused_qk_topk_naive(x, qr, None, 2, mask="causal")   # Megatron's own call
        calls.append(("full", self._ic_dsa_rank))
        return "full-out"

    mod.DSAttention.forward = forward
    assert icp.apply_index_cache_patch(dsa_module=mod)
    layers = [mod.DSAttention(i) for i in range(6)]
    q4 = torch.zeros(4, 1, 2, 8)
    outs = [layer.forward(q4, q4, None, None, torch.tensor(10 + i), torch.tensor(0), None)
            for i, layer in enumerate(layers)]
    assert outs == ["full-out", "shared-out", "shared-out", "full-out", "shared-out", "shared-out"]
    assert topk_calls == [10, 13]                       # one top-k per Full layer
    shared = [c[1].tolist() for c in calls if c[0] == "shared"]
    assert shared == [[10, -1], [10, -1], [13, -1], [13, -1]]
    assert mod.fused_qk_topk_naive is module_topk        # the wrapper is removed after the forward
    sched = icp.get_schedule()
    assert sched.captured == 2 and sched.rederived == 0


def test_index_scores_patch_keeps_autograd(monkeypatch):
    """compute_index_scores_fused_bf16 (what the Megatron patch installs) returns
    a tensor with autograd history whenever grad mode is on and q, weights or k
    requires grad, and its backward runs the indexer backward; without grad it
    returns a plain tensor.  The HIP launches are replaced by CPU stand-ins
    (this checks the wiring; the GPU tests check the kernels)."""
    from cppmega_amd import dsa_indexer_fused_patch as dip
    from oracle import indexer as oix

    seen = []

    def fake_scores(q, weights, k, use_relu=True, causal=0, **kw):
        return oix.compute_index_scores(q, weights, k, use_relu)

    def fake_backward(grad, q, weights, k, use_relu=True, causal=False, starts=None, ends=None):
        assert starts is None and ends is None
        seen.append((use_relu, causal))
        dq, dw, dk = oix.index_scores_backward(grad, q, weights, k, use_relu, causal)
        return dq.to(q.dtype), dw.to(weights.dtype), dk.to(k.dtype)

    monkeypatch.setattr(dip, "index_scores", fake_scores)
    monkeypatch.setattr(dip, "index_scores_backward", fake_backward)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(6, 1, 16, 64, generator=g).to(torch.bfloat16).requires_grad_()
    w = torch.randn(6, 1, 16, generator=g).requires_grad_()
    k = torch.randn(7, 1, 64, generator=g).to(torch.bfloat16).requires_grad_()
    out = dip.compute_index_scores_fused_bf16(q, w, k)
    assert out.requires_grad and out.grad_fn is not None, "the patch must not return a detached tensor"
    out.sum().backward()
    assert seen == [(True, False)]
    assert q.grad is not None and w.grad is not None and k.grad is not None
    assert q.grad.dtype == torch.bfloat16 and w.grad.dtype == torch.float32
    with torch.no_grad():
        plain = dip.compute_index_scores_fused_bf16(q, w, k)
    assert not plain.requires_grad
    mod = types.SimpleNamespace(_compute_index_scores=lambda *a, **kw: None)
    assert dip.apply_dsa_indexer_fused_patch(dsa_module=mod)
    r = mod._compute_index_scores(q, w, k, use_relu=True)
    assert r.requires_grad


def test_fused_indexer_loss_patch_rebinds_the_module(monkeypatch):
    from cppmega_amd import dsa_fused_indexer_loss as fil

    monkeypatch.setattr(fil, "_DSA_MODULE", None)

    class Megatrons:
        @staticmethod
        def apply(*a, **kw):
            raise AssertionError("replaced")

    mod = types.SimpleNamespace(FusedDSAIndexerLoss=Megatrons)
    assert fil.apply_fused_indexer_loss_patch(dsa_module=mod)
    assert mod.FusedDSAIndexerLoss is fil.FusedDSAIndexerLoss
    assert fil.apply_fused_indexer_loss_patch(dsa_module=mod)
    assert fil._DSA_MODULE is mod
    with pytest.raises(RuntimeError):
        fil.apply_fused_indexer_loss_patch(dsa_module=types.SimpleNamespace())


def test_fused_indexer_loss_resolves_topk_at_call_time(monkeypatch):
    """The loss takes its scores and top-k from the dsa module's
    fused_qk_topk_naive as bound at call time (lemyx_dsa_warmup.py:166-176
    imports it inside apply), and accepts and ignores query_valid_rows
    (lemyx_dsa_warmup.py:101)."""
    from cppmega_amd import dsa_fused_indexer_loss as fil

    monkeypatch.setattr(fil, "_DSA_MODULE", None)
    seen = []

    def kl(scores, idx, query, key, scale, coeff, sparse):
        seen.append(("kl", scores, idx, sparse))
        return torch.tensor(0.25)

    monkeypatch.setattr(fil, "indexer_kl_loss", kl)

    def first(q, k, w, topk, mask=None, varlen_starts=None, varlen_ends=None, key_positions=None, use_relu=True):
        seen.append(("first", mask, use_relu))
        return "scores-1", "idx-1"

    def second(q, k, w, topk, **kw):
        seen.append(("second", kw["mask"]))
        return "scores-2", "idx-2"

    mod = types.SimpleNamespace(FusedDSAIndexerLoss=object, fused_qk_topk_naive=first)
    assert fil.apply_fused_indexer_loss_patch(dsa_module=mod)
    t = torch.zeros(2, 1, 1, 1)
    idx, loss = mod.FusedDSAIndexerLoss.apply(t, t, t, t, t, 0.1, 4, 1.0, "m", True, None,
                                              query_valid_rows=torch.ones(2, dtype=torch.int32), use_relu=False)
    assert (idx, float(loss)) == ("idx-1", 0.25)
    mod.fused_qk_topk_naive = second                  # rebinding after the patch takes effect on the next call
    idx, _ = mod.FusedDSAIndexerLoss.apply(t, t, t, t, t, 0.1, 4, 1.0, "m2", False, None)
    assert idx == "idx-2"
    assert seen == [("first", "m", False), ("kl", "scores-1", "idx-1", True), ("second", "m2"),
                    ("kl", "scores-2", "idx-2", False)]


def _loss_layer_module(calls, loss_cls_factory):
    """A fake dsa module whose DSAttention takes its indices from
    FusedDSAIndexerLoss.apply (Megatron's training path with the indexer loss)."""
    mod = _fake_dsa_module(calls)
    topk_calls = []

    def module_topk(q, k, w, topk, mask=None, **kw):
        topk_calls.append((int(q), mask))
        return "scores", torch.tensor([int(q), -1])

    mod.fused_qk_topk_naive = module_topk
    mod.FusedDSAIndexerLoss = loss_cls_factory(mod)

    def forward(self, query, key, value, attention_mask, x, qr, **kw):
        idx, loss = mod.FusedDSAIndexerLoss.apply(x, None, qr, query, key, 0.1, 2, 1.0, "causal", True, None)
        calls.append(("full", self._ic_dsa_rank, idx.tolist()))
        return "full-out"

    mod.DSAttention.forward = forward
    return mod, topk_calls


def test_index_cache_captures_indices_of_the_indexer_loss_path(monkeypatch):
    """Both patches installed (this package's FusedDSAIndexerLoss and
    IndexCache), the Full layers take their indices from
    FusedDSAIndexerLoss.apply: each Full layer runs one top-k, its masked
    picks are cached, nothing is re-derived."""
    from cppmega_amd import dsa_fused_indexer_loss as fil

    monkeypatch.setattr(fil, "_DSA_MODULE", None)
    monkeypatch.setattr(fil, "indexer_kl_loss", lambda *a: torch.tensor(0.5))
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0,3")
    monkeypatch.setattr(icp, "_SCHEDULE", None)

    def rederive(*a, **k):
        raise AssertionError("the Full layer must not run a second indexer + top-k pass")

    monkeypatch.setattr(icp, "fused_qk_topk_naive", rederive)
    calls = []

    def factory(mod):
        class Megatrons:
            @staticmethod
            def apply(*a, **kw):
                raise AssertionError("replaced by the gfx950 drop-in")
        return Megatrons

    mod, topk_calls = _loss_layer_module(calls, factory)
    assert fil.apply_fused_indexer_loss_patch(dsa_module=mod)
    assert icp.apply_index_cache_patch(dsa_module=mod)
    layers = [mod.DSAttention(i) for i in range(6)]
    q4 = torch.zeros(4, 1, 2, 8)
    outs = [layer.forward(q4, q4, None, None, torch.tensor(20 + i), torch.tensor(0), None)
            for i, layer in enumerate(layers)]
    assert outs == ["full-out", "shared-out", "shared-out", "full-out", "shared-out", "shared-out"]
    assert topk_calls == [(20, "causal"), (23, "causal")]        # one masked top-k per Full layer
    shared = [c[1].tolist() for c in calls if c[0] == "shared"]
    assert shared == [[20, -1], [20, -1], [23, -1], [23, -1]]
    assert mod.FusedDSAIndexerLoss is fil.FusedDSAIndexerLoss   # wrappers removed after the forward
    sched = icp.get_schedule()
    assert sched.captured == 2 and sched.rederived == 0


def test_index_cache_captures_a_loss_bound_at_import(monkeypatch):
    """An indexer loss that imported its top-k at load time (so the module's
    fused_qk_topk_naive is never called) is still captured, through the
    FusedDSAIndexerLoss.apply wrapper."""
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0")
    monkeypatch.setattr(icp, "_SCHEDULE", None)
    monkeypatch.setattr(icp, "fused_qk_topk_naive",
                        lambda *a, **k: (_ for _ in ()).throw(AssertionError("no re-derivation")))
    calls = []

    def factory(mod):
        class BoundAtImport:
            @staticmethod
            def apply(q, w, k, *rest, **kw):
                return torch.tensor([int(q), 7]), torch.tensor(0.0)
        return BoundAtImport

    mod, topk_calls = _loss_layer_module(calls, factory)
    assert icp.apply_index_cache_patch(dsa_module=mod)
    layers = [mod.DSAttention(i) for i in range(3)]
    q4 = torch.zeros(4, 1, 2, 8)
    outs = [layer.forward(q4, q4, None, None, torch.tensor(30 + i), torch.tensor(0), None)
            for i, layer in enumerate(layers)]
    assert outs == ["full-out", "shared-out", "shared-out"] and topk_calls == []
    assert [c[1].tolist() for c in calls if c[0] == "shared"] == [[30, 7], [30, 7]]
    sched = icp.get_schedule()
    assert sched.captured == 1 and sched.rederived == 0


def test_index_cache_fallback_uses_the_layer_mask(monkeypatch):
    """A Full forward that calls neither top-k entry falls back to a second
    pass, which selects with the layer's own attention mask and varlen windows
    (so it caches what the layer would have picked)."""
    monkeypatch.setenv("CPPMEGA_INDEX_CACHE_FULL_LAYERS", "0")
    monkeypatch.setattr(icp, "_SCHEDULE", None)
    seen = []

    def rederive(q, k, w, topk, mask=None, varlen_starts=None, varlen_ends=None, key_positions=None,
                 use_relu=False):
        seen.append((mask, varlen_starts, varlen_ends, key_positions, topk))
        return None, "picks"

    monkeypatch.setattr(icp, "fused_qk_topk_naive", rederive)
    calls = []
    mod = _fake_dsa_module(calls)
    built = []

    def build_mask(**kw):
        built.append((kw["sq"], kw["skv"], kw["b"]))
        return "layer-mask", ("st", "en", "kp")

    mod._build_dsattention_forward_mask = build_mask
    assert icp.apply_index_cache_patch(dsa_module=mod)
    layers = [mod.DSAttention(i) for i in range(2)]
    q = torch.zeros(5, 3, 2, 8)
    outs = [layer.forward(q, q, None, None, torch.tensor(1), torch.tensor(0), None) for layer in layers]
    assert outs == ["full-out", "shared-out"]
    assert seen == [("layer-mask", "st", "en", "kp", 2)]
    assert built[0] == (5, 5, 3)
    assert calls[-1] == ("shared", "picks")
    sched = icp.get_schedule()
    assert sched.captured == 0 and sched.rederived == 1


# ---------------------------------------------------------------------------
# bench.py: one GPU only
# ---------------------------------------------------------------------------
def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr)


def test_unwrap_quantized_looks_te_up_once(monkeypatch):
    """unwrap_quantized returns plain tensors untouched without any import, and
    looks Transformer Engine up at most once per process (a failed import is
    not cached by Python); a QuantizedTensor is dequantised."""
    import builtins

    from cppmega_amd.sparse_mla_ops import _common

    monkeypatch.setattr(_common, "_QUANTIZED_TENSOR", _common._NOT_LOOKED_UP)
    calls = []
    real_import = builtins.__import__

    def counting(name, *a, **k):
        if name.startswith("transformer_engine"):
            calls.append(name)
        return real_import(name, *a, **k)

    monkeypatch.setattr(builtins, "__import__", counting)
    t = torch.zeros(2)
    assert _common.unwrap_quantized(t) is t and calls == []

    class Sub(torch.Tensor):
        pass

    x = torch.zeros(2).as_subclass(Sub)
    for _ in range(3):
        assert _common.unwrap_quantized(x) is x
    assert len(calls) <= 1

    class FakeQuantized:
        def dequantize(self):
            return "dequantised"

    monkeypatch.setattr(_common, "_QUANTIZED_TENSOR", FakeQuantized)
    assert _common.unwrap_quantized(FakeQuantized()) == "dequantised"
