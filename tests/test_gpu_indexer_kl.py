"""Parity of dsa_indexer_kl_grad (HIP) against the CPU oracle's autograd of DSAIndexerLoss.

Gradients are accumulated in fp32 from bf16 q/k and a bf16-rounded E = g w [S > 0], so
the tolerance is 1e-2 relative; the summed loss (fp32 statistics) 1e-4 relative.
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rand_indices, rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(S, H, D, K, seed, q_offset=0, holes=0.0):
    g = torch.Generator().manual_seed(seed)
    s_k = S + q_offset
    qi = torch.randn(1, S, H, D, generator=g).bfloat16()
    ki = torch.randn(1, s_k, D, generator=g).bfloat16()
    w = torch.rand(1, S, H, generator=g) * H ** -0.5 * D ** -0.5
    idx = rand_indices(S, K, q_offset=q_offset, seed=seed, holes=holes)
    # a positive target mass per row (as the head-summed attention mass would be)
    mass = torch.rand(1, S, K, generator=g) * 4.0
    return qi, ki, w, idx, mass


def _gpu(qi, ki, w, idx, mass, q_offset=0, loss_scale=1.0, grad_scale=1.0):
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    out = ops.indexer_kl_grad_from_mass(qi.to(DEV), ki.to(DEV), w.to(DEV), idx.to(DEV), mass.to(DEV),
                                        q_offset=q_offset, loss_scale=loss_scale, grad_scale=grad_scale)
    torch.cuda.synchronize()
    return [t.cpu() for t in out]


@pytest.mark.parametrize("S,H,D,K,q_offset,holes", [(160, 64, 128, 96, 0, 0.0), (100, 64, 128, 64, 28, 0.1),
                                                    (90, 64, 128, 72, 0, 0.05),
                                                    (40, 4, 32, 16, 0, 0.0)])
def test_indexer_kl_parity(S, H, D, K, q_offset, holes):
    qi, ki, w, idx, mass = _case(S, H, D, K, seed=S + K, q_offset=q_offset, holes=holes)
    dq, dk, dw, loss_rows = _gpu(qi, ki, w, idx, mass, q_offset=q_offset, loss_scale=0.5, grad_scale=2.0)
    rdq, rdk, rdw, rloss = O.indexer_kl_from_mass(qi, ki, w, idx, mass, q_offset=q_offset, loss_scale=0.5)
    assert abs(float(loss_rows.double().sum()) - float(rloss)) <= 1e-4 * abs(float(rloss))
    assert rel_err(dq, 2.0 * rdq) <= 1e-2, rel_err(dq, 2.0 * rdq)
    assert rel_err(dk, 2.0 * rdk) <= 1e-2, rel_err(dk, 2.0 * rdk)
    assert rel_err(dw, 2.0 * rdw) <= 1e-2, rel_err(dw, 2.0 * rdw)


def test_indexer_kl_dk_is_bitwise_reproducible():
    """dk_idx sums each key's contributions in a fixed order: two runs give the same bits
    (key lists of ~250-500 pairs straddle the 256-pair reduction segments)."""
    qi, ki, w, idx, mass = _case(768, 64, 128, 384, seed=5, holes=0.02)
    a = _gpu(qi, ki, w, idx, mass)
    b = _gpu(qi, ki, w, idx, mass)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_indexer_kl_zero_when_distributions_match():
    """If softmax(I) over the selected keys equals the target, loss and gradients vanish."""
    S, H, D, K = 64, 64, 128, 32
    qi, ki, w, idx, _ = _case(S, H, D, K, seed=3)
    I = O.indexer_scores(qi, ki, w, dtype=torch.float64)  # [1,S,S]
    sel = torch.gather(I, -1, idx.clamp_min(0).long()).masked_fill(idx < 0, float("-inf"))
    mass = torch.softmax(sel, dim=-1).float() * 3.0  # target proportional to softmax(I)
    dq, dk, dw, loss_rows = _gpu(qi, ki, w, idx, mass)
    assert float(loss_rows.abs().max()) <= 1e-4
    assert float(dq.abs().max()) <= 1e-4 and float(dw.abs().max()) <= 1e-4 and float(dk.abs().max()) <= 1e-4
