"""The allocation-free quantiser entry point (dsa_fp8_tensorwise_quantize_noalloc)
against the workspace entry point (dsa_fp8_tensorwise_quantize), through the
C-ABI: bit-identical codes and scale_inv on two calls in a row, the second on a
smaller input, with nothing allocated by the library for the call."""
import pytest
import torch

from cppmega_amd import _lib, synthetic

pytestmark = pytest.mark.gpu


def _with_workspace(x):
    L = _lib.load()
    out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    si = torch.empty(1, dtype=torch.float32, device=x.device)
    nb = int(L.dsa_fp8_quantize_workspace_size())
    ws = torch.empty(nb, dtype=torch.uint8, device=x.device)
    code = _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F32
    _lib.check(L.dsa_fp8_tensorwise_quantize(x.data_ptr(), x.numel(), code, out.data_ptr(), si.data_ptr(),
                                             ws.data_ptr(), nb, _lib.stream_ptr(x.device.index)),
               "dsa_fp8_tensorwise_quantize")
    return out, si


def _no_alloc(x, out, si):
    L = _lib.load()
    code = _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F32
    _lib.check(L.dsa_fp8_tensorwise_quantize_noalloc(x.data_ptr(), x.numel(), code, out.data_ptr(), si.data_ptr(),
                                                     _lib.stream_ptr(x.device.index)),
               "dsa_fp8_tensorwise_quantize_noalloc")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dev, dt):
    big = synthetic.outlier_values((3, 70001), seed=11).to(dt).to(dev)       # > 1024 partial blocks
    small = (synthetic.outlier_values((777,), seed=12) * 0.01).to(dt).to(dev)  # different scale, fewer blocks
    _lib.ensure_device(big)
    outs = []
    for x in (big, small):
        out = torch.full(x.shape, 0xAB, dtype=torch.uint8, device=dev)
        si = torch.full((1,), -1.0, dtype=torch.float32, device=dev)
        _no_alloc(x, out, si)
        outs.append((out, si))
    torch.cuda.synchronize()
    for x, (out, si) in zip((big, small), outs):
        ref_out, ref_si = _with_workspace(x)
        assert torch.equal(out, ref_out), "codes differ from the workspace entry point"
        assert torch.equal(si, ref_si), "scale_inv differs from the workspace entry point"
    assert not torch.equal(outs[0][1], outs[1][1])    # the second call did not reuse the first scale


def test_noalloc_zero_length_and_errors(dev):
    L = _lib.load()
    si = torch.full((1,), -1.0, dtype=torch.float32, device=dev)
    x = torch.zeros(1, dtype=torch.float32, device=dev)
    _lib.check(L.dsa_fp8_tensorwise_quantize_noalloc(x.data_ptr(), 0, _lib.DTYPE_F32, None, si.data_ptr(),
                                                     _lib.stream_ptr(0)), "noalloc n=0")
    torch.cuda.synchronize()
    assert float(si) == 1.0                              # amax of nothing: scale 1
    rc = L.dsa_fp8_tensorwise_quantize_noalloc(x.data_ptr(), 1, 7, None, si.data_ptr(), _lib.stream_ptr(0))
    assert rc == _lib.DSA_ERR_INVALID_ARG
