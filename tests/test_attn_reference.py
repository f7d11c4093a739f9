"""The full-output fp32 reference used by the full-size GPU tests (tests/attn_reference.py)
against the CPU oracle on small inputs: out, LSE, mass, dQ and dKV with and without a
per-head sink, 576-column (latent + rope, v = the first 512 columns) and 512-column rows,
causal offsets and -1 holes."""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.attn_reference import attention_reference
from tests.dsa_cases import rand_indices


@pytest.mark.parametrize("D,q_offset,sink,rows", [(576, 0, False, 7), (576, 5, False, 64), (512, 0, True, 5)])
def test_reference_matches_oracle(D, q_offset, sink, rows):
    S, H, K = 23, 3, 9
    g = torch.Generator().manual_seed(D + q_offset)
    q = torch.randn(1, S, H, D, generator=g, dtype=torch.float64)
    kv = torch.randn(1, S + q_offset, D, generator=g, dtype=torch.float64)
    dout = torch.randn(1, S, H, 512, generator=g, dtype=torch.float64)
    idx = rand_indices(S, K, q_offset=q_offset, seed=3, holes=0.2)
    scale = 0.06
    sinks = torch.randn(H, generator=g, dtype=torch.float64) if sink else None
    ref = attention_reference(q, kv, idx, dout, scale, q_offset=q_offset, sinks=sinks, rows=rows)
    if sink:
        oq = q.clone().requires_grad_(True)
        okv = kv.clone().requires_grad_(True)
        osk = sinks.clone().requires_grad_(True)
        out, lse = O.sparse_attn_sink(oq, okv, osk, idx, scale)
        out.backward(dout)
        torch.testing.assert_close(ref["out"].double(), out[0].detach(), rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["lse"].double(), lse[0].detach(), rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["dq"].double(), oq.grad[0], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["dkv"].double(), okv.grad[0], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["dsink"].double(), osk.grad, rtol=1e-4, atol=1e-5)
    else:
        out, lse = O.sparse_mla_fwd(q, kv, idx, scale, q_offset=q_offset)
        dq, dkv, mass = O.sparse_mla_bwd_closed_form(q, kv, idx, out, lse, dout, scale, q_offset=q_offset)
        torch.testing.assert_close(ref["out"].double(), out[0], rtol=1e-4, atol=1e-5)
        fin = torch.isfinite(lse[0])
        torch.testing.assert_close(ref["lse"].double()[fin], lse[0][fin], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["mass"].double(), mass[0], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["dq"].double(), dq[0], rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(ref["dkv"].double(), dkv[0], rtol=1e-4, atol=1e-5)
