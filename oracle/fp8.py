"""CPU restatement of tensorwise (current-scaling) FP8 e4m3 quantisation.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference: per_token_cast_to_fp8 -> _te_tensorwise_cast_to_fp8
(cppmega/megatron/sparse_mla_ops/tilelang_sparse_mla_fwd_fp8.py:74-99,396-412)
calls Transformer Engine's Float8CurrentScalingQuantizer (not vendored, pin
TE 2.16.0.dev0 in STACK.lock:14-23): one fp32 amax over the whole tensor,
scale = fp8_max / amax, data = e4m3(x * scale), scale_inv = 1 / scale,
real value = data * scale_inv (sparse_mla.py:316-326).  TE's own numerics
are not available here, so the exact rounding of scale and scale_inv is
"parity unpinned" against TE; this restatement fixes it as IEEE fp32
division and torch's round-to-nearest-even float8_e4m3fn cast of values
clamped to +-448.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0


def tensorwise_quantize(x):
    """x (any float dtype) -> (fp8 float8_e4m3fn, scale_inv fp32 0-dim tensor)."""
    xf = x.float()
    # NaN entries do not take part in amax (an fmax reduction ignores them)
    amax = xf.abs().nan_to_num(nan=0.0, posinf=float("inf")).max() if xf.numel() else torch.tensor(0.0)
    amax = amax.to(torch.float32)
    if float(amax) > 0 and torch.isfinite(amax):
        scale = torch.tensor(E4M3_MAX, dtype=torch.float32) / amax
    else:
        scale = torch.tensor(1.0, dtype=torch.float32)
    y = (xf * scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    scale_inv = torch.tensor(1.0, dtype=torch.float32) / scale
    return y, scale_inv


def dequantize(x8, scale_inv):
    return x8.float() * scale_inv


def e4m3_value(code):
    """Decode one e4m3fn byte from its bit fields (bias 7, 3 mantissa bits, 0x7f/0xff NaN)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
