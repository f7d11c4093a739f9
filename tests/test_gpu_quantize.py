"""Parity of the fp8-e4m3fn per-row quantisation kernel (dsa_quantize_fp8_rows) with the
oracle (scale = max(amax|row| / 448, 1e-12) and q = x / scale, correctly rounded fp32
divisions, then torch's float8_e4m3fn cast on the host).  Byte-exact (q bytes and scale
bits), including rows with exact rounding ties in the normal and subnormal e4m3 ranges."""

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _check(x):
    q, s = _ops().quantize_fp8_per_row(x)
    rq, rs = O.quantize_e4m3_per_row(x.cpu())
    assert q.dtype == torch.float8_e4m3fn and q.shape == x.shape and s.shape == x.shape[:-1]
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu().view(torch.int32), rs.view(torch.int32))


@pytest.mark.parametrize("shape,dtype", [((2, 33, 64, 128), torch.bfloat16), ((5, 128), torch.float32),
                                         ((7, 72), torch.bfloat16), ((9, 100), torch.bfloat16),
                                         ((3, 2048), torch.float32), ((11, 8), torch.bfloat16), ((1, 3), torch.float32)])
def test_quantize_random(shape, dtype):
    g = torch.Generator(device=DEV).manual_seed(sum(shape))
    x = (torch.randn(shape, device=DEV, generator=g) * 3).to(dtype)
    _check(x)


def test_quantize_unaligned_rows():
    # a view starting one element into its storage: rows are not 16-byte aligned (scalar path)
    g = torch.Generator(device=DEV).manual_seed(5)
    buf = torch.randn(17 * 128 + 1, device=DEV, generator=g).bfloat16()
    x = buf[1:].view(17, 128)
    _check(x)


def test_quantize_rounding_ties_zero_and_tiny_rows():
    # amax = 448 gives scale 1 exactly, so x / scale = x: put x on the midpoints between
    # adjacent e4m3fn values (ties go to the even code), subnormal ones included
    codes = torch.arange(0, 0x7F, dtype=torch.uint8, device=DEV)
    vals = codes.view(torch.float8_e4m3fn).float()  # every finite non-negative e4m3fn value
    mids = (vals[:-1].double() + vals[1:].double()) / 2
    row = torch.cat([torch.tensor([448.0], device=DEV, dtype=torch.float64), mids, -mids]).float()
    d = 8 * ((row.numel() + 7) // 8)
    x = torch.zeros(4, d, device=DEV)
    x[0, : row.numel()] = row
    x[1, : row.numel()] = row * 1.0000001  # just above the midpoints: rounds up
    x[2] = 0.0  # all-zero row: scale 1e-12, q = 0
    x[3, 0] = 1e-30  # tiny amax: the clamp decides the scale
    _check(x)


def test_quantize_nan_row_propagates():
    x = torch.randn(3, 128, device=DEV)
    x[1, 17] = float("nan")
    q, s = _ops().quantize_fp8_per_row(x)
    assert torch.isnan(s[1]) and torch.isnan(q[1].float()).all()
    rq, rs = O.quantize_e4m3_per_row(x.cpu())
    assert torch.isnan(rs[1])
    assert torch.equal(q[[0, 2]].cpu().view(torch.uint8), rq[[0, 2]].view(torch.uint8))
