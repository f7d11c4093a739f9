"""The MLA absorb kernels (dsa_mla_absorb) and their autograd wrappers against the oracle:
forward outputs at bf16 2e-2 relative (fp32 accumulation, one bf16 rounding), the q_pe
columns copied bit for bit, and the gradients to q_nope, q_pe, the attention output and
both weights against fp64 autograd of the oracle's einsums at 2e-2."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


@pytest.mark.parametrize("B,S,H", [(1, 300, 16), (2, 64, 128), (1, 1, 4)])
def test_absorb_q_forward_backward(B, S, H):
    ops = _ops()
    g = torch.Generator().manual_seed(B * S + H)
    q_nope = (torch.randn(B, S, H, 128, generator=g) * 0.5).bfloat16()
    q_pe = torch.randn(B, S, H, 64, generator=g).bfloat16()
    w_uk = (torch.randn(H, 128, 512, generator=g) * 128 ** -0.5).bfloat16()
    dq = torch.randn(B, S, H, 576, generator=g).bfloat16()
    a, p, w = (t.to(DEV).requires_grad_(True) for t in (q_nope, q_pe, w_uk))
    q = ops.mla_absorb_q(a, p, w)
    q.backward(dq.to(DEV))
    torch.cuda.synchronize()
    assert q.shape == (B, S, H, 576) and q.dtype == torch.bfloat16 and q.is_contiguous()
    rn, rp, rw = (t.double().requires_grad_(True) for t in (q_nope, q_pe, w_uk))
    ref = O.mla_absorb_q(rn, rp, rw)
    ref.backward(dq.double())
    assert rel_err(q[..., :512], ref[..., :512].detach()) <= 2e-2
    assert torch.equal(q[..., 512:].cpu(), q_pe)
    assert rel_err(a.grad, rn.grad) <= 2e-2 and rel_err(p.grad, rp.grad) <= 2e-2
    assert rel_err(w.grad, rw.grad) <= 2e-2


@pytest.mark.parametrize("B,S,H", [(1, 300, 16), (2, 64, 128)])
def test_absorb_out_forward_backward(B, S, H):
    ops = _ops()
    g = torch.Generator().manual_seed(B * S + H + 1)
    out = torch.randn(B, S, H, 512, generator=g).bfloat16()
    w_uv_t = (torch.randn(H, 512, 128, generator=g) * 512 ** -0.5).bfloat16()
    dy = torch.randn(B, S, H, 128, generator=g).bfloat16()
    o, w = (t.to(DEV).requires_grad_(True) for t in (out, w_uv_t))
    y = ops.mla_absorb_out(o, w)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (B, S, H, 128) and y.is_contiguous()
    ro, rw = (t.double().requires_grad_(True) for t in (out, w_uv_t))
    ref = O.mla_absorb_out(ro, rw)
    ref.backward(dy.double())
    assert rel_err(y, ref.detach()) <= 2e-2
    assert rel_err(o.grad, ro.grad) <= 2e-2 and rel_err(w.grad, rw.grad) <= 2e-2


def test_absorb_strided_rows():
    """Rows read from a strided view (the first 512 columns of a 576-wide tensor) and an
    appended block taken from a view, as the backward and the forward use them."""
    ops = _ops()
    g = torch.Generator().manual_seed(5)
    big = torch.randn(3, 40, 8, 576, generator=g).bfloat16().to(DEV)
    wt = (torch.randn(8, 128, 512, generator=g) * 512 ** -0.5).bfloat16().to(DEV)
    got = ops.mla_absorb(big[..., :512], wt, append=big[..., 512:])
    ref = torch.einsum("bshr,hvr->bshv", big[..., :512].double(), wt.double())
    assert rel_err(got[..., :128], ref) <= 2e-2
    assert torch.equal(got[..., 128:], big[..., 512:])
