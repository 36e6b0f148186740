"""Shared test helpers (tolerance checks, device moves)."""
from __future__ import annotations

import torch

# Tolerance contract for bf16 SparseMLA outputs, LSE and gradients vs the oracle.
RTOL = 2e-2
ATOL = 1e-2


def assert_close(actual, expected, rtol=RTOL, atol=ATOL, what=""):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    both_inf = torch.isinf(a) & torch.isinf(e) & (torch.sign(a) == torch.sign(e))
    diff = (a - e).abs()
    bad = (diff > atol + rtol * e.abs()) & ~both_inf
    if bad.any():
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.numel()} elements outside rtol={rtol} atol={atol}; "
            f"max abs diff {float(diff[~both_inf].max()):.4g}; first bad flat index {i}: "
            f"actual {float(a.flatten()[i]):.6g} expected {float(e.flatten()[i]):.6g}")


def to_dev(d, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
