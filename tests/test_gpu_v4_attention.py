"""DeepSeek-V4 shared-KV sparse attention on the GPU (npu_sparse_attn_shared_kv).

Forward and the gradients to query, ori_kv, cmp_kv and the sinks against the oracle's
``sparse_attn_sink`` (fp64 autograd on the same bf16 / fp32 inputs): bf16 within 2e-2,
fp32 within 1e-5 relative.  Cases: ratio 4 with a given top-k, ratio 128 (every causal
compressed block), no compressed KV (ratio 1).
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(S, H, D, ratio, K, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, S, H, D, generator=g).to(dtype)
    ori = torch.randn(1, S, D, generator=g).to(dtype)
    n_cmp = S // ratio if ratio > 1 else 0
    cmp = torch.randn(1, n_cmp, D, generator=g).to(dtype) if n_cmp else None
    sink = torch.randn(H, generator=g)
    idx = None
    if ratio == 4:
        idx = torch.full((1, S, K), -1, dtype=torch.int32)
        for s in range(S):
            nv = min(n_cmp, (s + 1) // ratio)
            c = min(K, nv)
            if c:
                idx[0, s, :c] = torch.sort(torch.randperm(nv, generator=g)[:c]).values.int() + S
    dout = torch.randn(1, S, H, D, generator=g).to(dtype)
    return q, ori, cmp, sink, idx, dout


def _run(S, H, D, ratio, K, dtype, seed, tol, window=128):
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    q, ori, cmp, sink, idx, dout = _case(S, H, D, ratio, K, dtype, seed)
    scale = D ** -0.5
    leaves = [t.to(DEV).requires_grad_(True) if t is not None else None for t in (q, ori, cmp)]
    sk = sink.to(DEV).requires_grad_(True)
    out = ops.npu_sparse_attn_shared_kv(leaves[0], leaves[1], leaves[2], None if idx is None else idx.to(DEV), sk,
                                        scale, ratio, ori_win_left=window - 1)
    out.backward(dout.to(DEV))
    # oracle on the same rounded inputs
    kv_all = ori if cmp is None else torch.cat([ori, cmp], dim=1)
    full_idx = O.v4_attn_indices(1, S, window, ratio, S, cmp_idxs=idx)
    oq = q.double().requires_grad_(True)
    okv = kv_all.double().requires_grad_(True)
    osk = sink.double().requires_grad_(True)
    ref, _ = O.sparse_attn_sink(oq, okv, osk, full_idx, scale)
    ref.backward(dout.double())
    assert rel_err(out.detach(), ref.detach()) <= tol, rel_err(out.detach(), ref.detach())
    assert rel_err(leaves[0].grad, oq.grad) <= tol
    got_dkv = leaves[1].grad if cmp is None else torch.cat([leaves[1].grad, leaves[2].grad], dim=1)
    assert rel_err(got_dkv, okv.grad) <= tol
    assert rel_err(sk.grad, osk.grad) <= tol, (sk.grad, osk.grad)


@pytest.mark.parametrize("S,H,ratio,K", [(256, 16, 4, 32), (384, 32, 128, 0), (200, 16, 1, 0)])
def test_v4_sink_attention_bf16(S, H, ratio, K):
    _run(S, H, 512, ratio, K, torch.bfloat16, seed=S + ratio, tol=2e-2)


def test_v4_sink_attention_fp32_small_head_dim():
    _run(96, 4, 64, 4, 8, torch.float32, seed=5, tol=1e-5, window=16)


def test_v4_sink_dominates_empty_rows():
    """A very large sink takes almost all the mass: output -> 0 and the sink gradient stays finite."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    q, ori, _, _, _, dout = _case(64, 16, 512, 1, 0, torch.bfloat16, seed=9)
    sink = torch.full((16,), 60.0, device=DEV, requires_grad=True)
    out = ops.npu_sparse_attn_shared_kv(q.to(DEV), ori.to(DEV), None, None, sink, 512 ** -0.5, 1)
    out.backward(dout.to(DEV))
    assert out.abs().max().item() < 1e-6
    assert torch.isfinite(sink.grad).all()


def test_v4_li_loss_gradients():
    """NpuLiLoss (loss deferred to backward) against the oracle's LiLoss: target = the
    combined-softmax probability at the selected compressed rows averaged over heads,
    loss = DSAIndexerLoss(eps 1e-10, loss_scale = softmax_scale), mean over tokens."""
    from types import SimpleNamespace

    from torchtitan_npu_simulator_amd.converters import npu_smla as smla_mod

    S, H, D, r, K, HI, DI, window = 256, 16, 512, 4, 32, 64, 128, 128
    q, ori, cmp, sink, idx_off, _ = _case(S, H, D, r, K, torch.bfloat16, seed=41)
    g = torch.Generator().manual_seed(42)
    qi = torch.randn(1, S, HI, DI, generator=g).bfloat16()
    ki = torch.randn(1, S // r, DI, generator=g).bfloat16()
    w = torch.rand(1, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5
    scale = D ** -0.5
    parent = SimpleNamespace(softmax_scale=scale, window_size=window, layer_id=None, n_layers=0)
    mod = smla_mod.NpuLiLoss(torch.nn.Module())
    mod.__dict__.update(parent.__dict__)
    leaves = [t.to(DEV).requires_grad_(True) for t in (qi, ki, w)]
    loss = mod(q.to(DEV), ori.to(DEV), cmp.to(DEV), sink.to(DEV), *leaves, idx_off.to(DEV), None, None, S)
    assert float(loss) == 0.0  # deferred to backward
    loss.backward()
    local = torch.where(idx_off < 0, idx_off, idx_off - S)
    dist = O.v4_selected_attn_dist(q, ori, cmp, sink, local, scale, window)
    rdq, rdk, rdw, _ = O.indexer_kl_from_mass(qi, ki, w, local, dist, q_offset=1 << 40, loss_scale=scale, eps=1e-10)
    n = S  # B * S tokens
    assert rel_err(leaves[0].grad, rdq / n) <= 2e-2, rel_err(leaves[0].grad, rdq / n)
    assert rel_err(leaves[1].grad, rdk / n) <= 2e-2
    assert rel_err(leaves[2].grad, rdw / n) <= 2e-2


@pytest.mark.parametrize("dtype,dv", [(torch.bfloat16, 512), (torch.float32, 512), (torch.bfloat16, 100)])
def test_sink_fold_and_grad_kernels(dtype, dv):
    """dsa_attn_sink_fold / dsa_attn_sink_grad against the same formulas in fp64: rows with
    no key (max -inf, sum 0), sinks above and below the row max."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    g = torch.Generator().manual_seed(31)
    B, S, H = 2, 37, 24
    out = torch.randn(B, S, H, dv, generator=g).to(dtype)
    dout = torch.randn(B, S, H, dv, generator=g).to(dtype)
    smax = torch.randn(B, S, H, generator=g) * 3
    ssum = torch.rand(B, S, H, generator=g) * 5 + 1
    smax[0, 0] = float("-inf")
    ssum[0, 0] = 0.0
    sinks = torch.randn(H, generator=g) * 4
    o, m2, s2 = ops.attn_sink_fold_(out.to(DEV), smax.to(DEV), ssum.to(DEV), sinks.to(DEV))
    sk = sinks.double().view(1, 1, -1)
    rm2 = torch.maximum(smax.double(), sk)
    a = torch.where(ssum > 0, ssum.double() * torch.exp(smax.double() - rm2), torch.zeros_like(rm2))
    rs2 = a + torch.exp(sk - rm2)
    ro = out.double() * (a / rs2).unsqueeze(-1)
    assert torch.allclose(m2.cpu().double(), rm2, rtol=1e-6)
    assert torch.allclose(s2.cpu().double(), rs2, rtol=1e-5)
    tol = 8e-3 if dtype == torch.bfloat16 else 1e-5
    assert rel_err(o.cpu(), ro) <= tol
    dsink = ops.attn_sink_grad(o, dout.to(DEV), m2, s2, sinks.to(DEV)).cpu()
    delta = (dout.double() * o.cpu().double()).sum(-1)
    ref = -(torch.exp(sk - rm2) / rs2 * delta).sum(dim=(0, 1))
    assert rel_err(dsink, ref) <= 1e-5
