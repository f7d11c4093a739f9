"""The attention sink folded into the gathered-attention kernels (dsa_sparse_mla_fwd_sink /
dsa_sparse_mla_bwd_sink) on the GPU.

Checked three ways: against the oracle's ``sparse_attn_sink`` (fp64, the reference's
SparseAttention.forward math; bf16 within 2e-2, fp32 within 1e-5 relative), against the
unfused sequence (sparse_mla_fwd, then dsa_attn_sink_fold; the backward's d sink against
dsa_attn_sink_grad on the same out / dout / statistics), and on the rows the epilogue
treats apart: rows with no valid slot (out = 0, statistics (sink, 1)) and rows whose
logits outgrow the online-softmax headroom (recomputed by the exact fixup pass, which
must fold the sink the same way).
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import attn_inputs, rand_indices, rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _sinks(H, seed, spread=3.0):
    g = torch.Generator().manual_seed(1000 + seed)
    return torch.randn(H, generator=g) * spread


@pytest.mark.parametrize("S,H,K,seed,holes", [(256, 64, 128, 0, 0.0), (160, 40, 96, 1, 0.25)])
def test_fused_sink_fwd_bwd_matches_oracle_512(S, H, K, seed, holes):
    """d_qk = d_v = 512 rows (k = v = the row, the DeepSeek-V4 layout) against fp64 autograd."""
    ops = _ops()
    q, kv, _, scale = attn_inputs(S, H, seed=seed, d_qk=512)
    idx = rand_indices(S, K, seed=seed, shuffle=True, holes=holes)
    sink = _sinks(H, seed)
    out, m2, s2 = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), scale, sinks=sink.to(DEV))
    oq, okv, osk = (t.double().requires_grad_(True) for t in (q, kv, sink))
    ref, ref_lse = O.sparse_attn_sink(oq, okv, osk, idx, scale)
    assert rel_err(out.cpu(), ref.detach()) <= 2e-2
    lse = m2.double().cpu() + torch.log(s2.double().cpu())
    assert (lse - ref_lse.detach()).abs().max() <= 0.2

    g = torch.Generator().manual_seed(77 + seed)
    dout = torch.randn(out.shape, generator=g).to(torch.bfloat16)
    dq, dkv, dsink = ops.sparse_mla_bwd(q.to(DEV), kv.to(DEV), idx.to(DEV), out, dout.to(DEV), m2, s2, scale,
                                        sinks=sink.to(DEV))
    ref.backward(dout.double())
    assert rel_err(dq.cpu(), oq.grad) <= 2e-2, rel_err(dq.cpu(), oq.grad)
    assert rel_err(dkv.cpu(), okv.grad) <= 2e-2, rel_err(dkv.cpu(), okv.grad)
    assert rel_err(dsink.cpu(), osk.grad) <= 2e-2, rel_err(dsink.cpu(), osk.grad)


@pytest.mark.parametrize("d_qk", [576, 512])
def test_fused_sink_fwd_matches_fold(d_qk):
    """Same inputs through sparse_mla_fwd + attn_sink_fold_ and through the fused forward:
    one bf16 rounding of out apart (the fused epilogue rounds once, the fold twice)."""
    ops = _ops()
    S, H, K = 192, 128, 128
    q, kv, _, scale = attn_inputs(S, H, seed=3, d_qk=d_qk, logit_std=2.0)
    idx = rand_indices(S, K, seed=3, shuffle=True, holes=0.1)
    sink = _sinks(H, 3, spread=5.0)
    qd, kvd, idd, skd = q.to(DEV), kv.to(DEV), idx.to(DEV), sink.to(DEV)
    o1, m1, l1 = ops.sparse_mla_fwd(qd, kvd, idd, scale)
    o1, m1, l1 = ops.attn_sink_fold_(o1, m1, l1, skd)
    o2, m2, l2 = ops.sparse_mla_fwd(qd, kvd, idd, scale, sinks=skd)
    assert rel_err(o2.cpu(), o1.cpu()) <= 8e-3
    assert torch.allclose(m2.cpu(), m1.cpu(), rtol=1e-6, atol=1e-6)
    assert torch.allclose(l2.cpu(), l1.cpu(), rtol=1e-4)


def test_fused_sink_rows_without_keys_and_fixup_rows():
    """Rows with no valid slot: out = 0, (softmax_max, softmax_sum) = (sink, 1), d sink part 0.
    Rows whose later keys dominate by ~e^100 go through the exact fixup pass with the sink."""
    ops = _ops()
    S, H, K = 96, 32, 64
    q, kv, _, scale = attn_inputs(S, H, seed=9, d_qk=512)
    kv = kv.float()
    kv[0, 40:] *= 40.0
    kv = kv.to(torch.bfloat16)
    idx = rand_indices(S, K, seed=9)
    idx[0, ::5] = -1  # every fifth row has no usable key
    sink = _sinks(H, 9)
    out, m2, s2 = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), scale, sinks=sink.to(DEV))
    out, m2, s2 = out.cpu(), m2.cpu(), s2.cpu()
    assert torch.all(out[0, ::5] == 0)
    assert torch.equal(m2[0, ::5], sink.view(1, H).expand(m2[0, ::5].shape))
    assert torch.all(s2[0, ::5] == 1.0)
    assert torch.all(s2 > 0)  # no row left marked for the fixup
    oq, okv, osk = (t.double().requires_grad_(True) for t in (q, kv, sink))
    ref, ref_lse = O.sparse_attn_sink(oq, okv, osk, idx, scale)
    assert rel_err(out, ref.detach()) <= 2e-2
    lse = m2.double() + torch.log(s2.double())
    assert (lse - ref_lse.detach()).abs().max() <= 0.2

    g = torch.Generator().manual_seed(99)
    dout = torch.randn(out.shape, generator=g).to(torch.bfloat16)
    dq, dkv, dsink = ops.sparse_mla_bwd(q.to(DEV), kv.to(DEV), idx.to(DEV), out.to(DEV), dout.to(DEV), m2.to(DEV),
                                        s2.to(DEV), scale, sinks=sink.to(DEV))
    ref.backward(dout.double())
    assert rel_err(dsink.cpu(), osk.grad) <= 2e-2
    assert rel_err(dq.cpu(), oq.grad) <= 2e-2


@pytest.mark.parametrize("chunk_bytes", [None, 6 << 20])
def test_fused_sink_grad_matches_sink_grad_kernel(chunk_bytes):
    """d sink from the backward's delta pass equals dsa_attn_sink_grad on the same out / dout /
    statistics (fp32 sums of the same bf16 products); a small workspace splits the rows into
    chunks whose parts must all land in d sink.  dq / dkv equal the plain backward's."""
    ops = _ops()
    S, H, K = 256, 64, 128
    q, kv, _, scale = attn_inputs(S, H, seed=12, d_qk=512)
    idx = rand_indices(S, K, seed=12, shuffle=True)
    sink = _sinks(H, 12).to(DEV)
    qd, kvd, idd = q.to(DEV), kv.to(DEV), idx.to(DEV)
    out, m2, s2 = ops.sparse_mla_fwd(qd, kvd, idd, scale, sinks=sink)
    g = torch.Generator().manual_seed(5)
    dout = torch.randn(out.shape, generator=g).to(torch.bfloat16).to(DEV)
    dq1, dkv1 = ops.sparse_mla_bwd(qd, kvd, idd, out, dout, m2, s2, scale, workspace_bytes=chunk_bytes)
    dq2, dkv2, dsink = ops.sparse_mla_bwd(qd, kvd, idd, out, dout, m2, s2, scale, workspace_bytes=chunk_bytes,
                                          sinks=sink)
    ref = ops.attn_sink_grad(out, dout, m2, s2, sink)
    assert rel_err(dsink.cpu(), ref.cpu()) <= 1e-5, rel_err(dsink.cpu(), ref.cpu())
    assert torch.equal(dq1.cpu(), dq2.cpu())
    assert rel_err(dkv2.cpu(), dkv1.cpu()) <= 1e-6


def test_fused_sink_fp32_exact_path():
    """fp32 inputs take the exact kernels; the sink is folded there the same way (1e-5)."""
    ops = _ops()
    S, H, K, D = 48, 8, 32, 64
    q, kv, _, scale = attn_inputs(S, H, seed=4, d_qk=D, dtype=torch.float32)
    idx = rand_indices(S, K, seed=4, holes=0.2)
    idx[0, 7] = -1
    sink = _sinks(H, 4)
    out, m2, s2 = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), scale, d_v=D, sinks=sink.to(DEV))
    oq, okv, osk = (t.double().requires_grad_(True) for t in (q, kv, sink))
    ref, ref_lse = O.sparse_attn_sink(oq, okv, osk, idx, scale)
    assert rel_err(out.cpu(), ref.detach()) <= 1e-5
    lse = m2.double().cpu() + torch.log(s2.double().cpu())
    assert (lse - ref_lse.detach()).abs().max() <= 1e-4
    g = torch.Generator().manual_seed(8)
    dout = torch.randn(out.shape, generator=g)
    dq, dkv, dsink = ops.sparse_mla_bwd(q.to(DEV), kv.to(DEV), idx.to(DEV), out, dout.to(DEV), m2, s2, scale,
                                        sinks=sink.to(DEV))
    ref.backward(dout.double())
    assert rel_err(dq.cpu(), oq.grad) <= 1e-5
    assert rel_err(dkv.cpu(), okv.grad) <= 1e-5
    assert rel_err(dsink.cpu(), osk.grad) <= 1e-5
