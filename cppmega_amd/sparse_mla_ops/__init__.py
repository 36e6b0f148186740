"""SparseMLA on gfx950: the drop-in surface of cppmega.megatron.sparse_mla_ops.

Every entry point launches the HIP kernels of libdsa_hip.so; importing this
package does not load the library (that happens on first use), so the module
imports on hosts without a GPU and fails loudly on first call there.
"""
from .sparse_mla import (
    SparseMLA,
    SparseMLA_FP8,
    apply_sparse_mla_patch,
    fused_sparse_mla_absorbed_fp8,
    sparse_mla_as_unfused_dsa,
    sparse_mla_fp8_as_unfused_dsa,
)
from .sparse_mla_blockscaled import (
    mxfp8_dequantize,
    sparse_mla_blockscaled_mxfp8_backward,
    sparse_mla_blockscaled_mxfp8_forward,
    sparse_mla_blockscaled_mxfp8_fwd_interface,
)
from .sparse_mla_bwd import InverseIndex, build_inverse_index, side_stream, sparse_mla_bwd
from .sparse_mla_bwd_fp8 import sparse_mla_bwd_fp8
from .sparse_mla_fwd import sparse_mla_fwd_interface
from .sparse_mla_fwd_fp8 import fp8_dequantize, per_token_cast_to_fp8, sparse_mla_fwd_fp8_interface, tensorwise_quantize

__all__ = [
    "SparseMLA",
    "SparseMLA_FP8",
    "apply_sparse_mla_patch",
    "fused_sparse_mla_absorbed_fp8",
    "mxfp8_dequantize",
    "per_token_cast_to_fp8",
    "sparse_mla_as_unfused_dsa",
    "sparse_mla_blockscaled_mxfp8_backward",
    "sparse_mla_blockscaled_mxfp8_forward",
    "sparse_mla_blockscaled_mxfp8_fwd_interface",
    "sparse_mla_bwd",
    "InverseIndex",
    "build_inverse_index",
    "side_stream",
    "sparse_mla_bwd_fp8",
    "sparse_mla_fp8_as_unfused_dsa",
    "sparse_mla_fwd_fp8_interface",
    "fp8_dequantize",
    "sparse_mla_fwd_interface",
    "tensorwise_quantize",
]
