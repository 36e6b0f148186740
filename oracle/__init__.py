"""CPU oracle for the DSA hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of every function
on the DeepSeek Sparse Attention hot path of cppmega (SparseMLA forward and
backward in bf16 and FP8-tensorwise form, the indexer scores, the
deterministic top-k and the tensorwise FP8 quantiser).  Each function cites
the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or as the timed CPU
baseline.  The product package ``cppmega_amd`` never imports it: its entry
points call the HIP library and fail loudly when that library is missing.

Pinning (what checks each function beyond restating it):
  * sparse_mla.sparse_mla_fwd / sparse_mla_bwd — float64 autograd of the
    closed-form masked softmax (``sparse_mla.sparse_mla_autograd_f64``),
    ``torch.autograd.gradcheck`` on tiny shapes, closed-form special cases
    (single valid index, equal scores, duplicates, all-masked rows) and
    invariants (sum over slots of dS is zero; index-order invariance).
  * indexer.compute_index_scores — the upstream einsum form and a float64
    brute force on tiny shapes.
  * topk.topk_ascending — pure-Python brute force over tiny rows,
    ``torch.topk`` on tie-free rows, and hypothesis properties.
  * fp8.tensorwise_quantize — torch's own float8_e4m3fn cast (an independent
    library routine) and exhaustive round-trip over all 256 e4m3 codes.
  * FP8 SparseMLA — reduces to the bf16 oracle on dequantised inputs
    (checked bit-for-bit on the score path) and stays within a stated bound
    of the bf16 result on cfg4-style inputs.
"""
