"""The npu_dsa drop-in end to end on the GPU: a DSV32_SDPA stand-in converted by the
registered converter, run forward + backward, checked against the CPU oracle.

Selection: the GPU top-k runs on bf16-MFMA scores, so the indices are checked to be a
valid top-k of the oracle's fp32 scores (every chosen score >= the K-th largest minus
the score tolerance); attention, its gradients and the indexer gradients are then
compared with the oracle on the GPU's indices (2e-2 relative, bf16; 1e-2 for the KL
gradients whose E term is rounded to bf16).
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


class DSV32_SDPA(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.config = SimpleNamespace(kv_lora_rank=512, qk_rope_head_dim=64)


class _Attn(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.inner_attention = DSV32_SDPA()


class _Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.attention = _Attn()


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.layers = torch.nn.ModuleDict({"0": _Block()})


@pytest.mark.parametrize("S,H,K,views", [(256, 16, 64, False), (192, 128, 128, False), (160, 128, 96, True)])
def test_npu_dsa_end_to_end(S, H, K, views):
    """views: q and k arrive as the reference model builds them, transposed views of
    [B, S, H, D] tensors (models/deepseek_v32/model.py:526-535), with the gradients landing
    in those tensors; otherwise as BHSD-contiguous tensors."""
    from torchtitan_npu_simulator_amd import converters as conv
    from torchtitan_npu_simulator_amd.converters.dsa_indexer_loss import DSAIndexerLossAutoScaler

    model = _Model()
    conv.registry().converter_class("npu_dsa")(model_spec=SimpleNamespace(name="deepseek_v32")).convert(model)
    sdpa = model.layers["0"].attention.inner_attention

    HI, DI = 64, 128
    g = torch.Generator().manual_seed(S + H)
    q = (torch.randn(1, H, S, 576, generator=g) / 24).bfloat16()
    kv = torch.randn(1, 1, S, 576, generator=g).bfloat16()
    qi = torch.randn(1, S, HI, DI, generator=g).bfloat16()
    ki = torch.randn(1, S, 1, DI, generator=g).bfloat16()
    w = (torch.rand(1, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5)
    dout = torch.randn(1, H, S, 512, generator=g)
    scale = 576 ** -0.5

    if views:
        q_leaf = q.transpose(1, 2).contiguous().to(DEV).requires_grad_(True)
        kv_leaf = kv.transpose(1, 2).contiguous().to(DEV).requires_grad_(True)
        qd, kvd = q_leaf.transpose(1, 2), kv_leaf.transpose(1, 2)
    else:
        qd = q.to(DEV).requires_grad_(True)
        kvd = kv.to(DEV).requires_grad_(True)
        q_leaf, kv_leaf = qd, kvd
    qid = qi.to(DEV).requires_grad_(True)
    kid = ki.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    loss, out = sdpa(qd, kvd, kvd[..., :512], None, scale, qid, kid, wd, None, K)
    y = DSAIndexerLossAutoScaler.apply(out, loss)
    (y.float() * dout.to(DEV)).sum().backward()
    torch.cuda.synchronize()

    # recover the GPU's selection from a second indexer call (same op, same inputs)
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    idx = ops.npu_lightning_indexer(qi.to(DEV), ki.to(DEV), w.to(DEV), sparse_count=K)[0][:, :, 0].cpu()
    scores = O.indexer_scores(qi, ki, w)
    kth = torch.sort(scores, dim=-1, descending=True).values[..., K - 1 : K].clamp_min(-1e30)
    chosen = torch.gather(scores, -1, idx.clamp_min(0).long()).masked_fill(idx < 0, float("inf"))
    assert bool((chosen >= kth - 1e-4 * scores.abs().amax()).all())
    for s in range(S):
        assert int((idx[0, s] >= 0).sum()) == min(K, s + 1)

    q_b = q.transpose(1, 2)
    kv_b = kv[:, 0]
    ref_out, ref_lse = O.sparse_mla_fwd(q_b, kv_b, idx, scale)
    assert rel_err(out.detach().cpu().transpose(1, 2), ref_out) <= 2e-2
    dq, dkv = O.sparse_mla_bwd(q_b, kv_b, idx, dout.transpose(1, 2), scale)
    gq = q_leaf.grad.cpu() if views else q_leaf.grad.cpu().transpose(1, 2)
    gkv = kv_leaf.grad.cpu()[:, :, 0] if views else kv_leaf.grad.cpu()[:, 0]
    assert rel_err(gq, dq) <= 2e-2
    assert rel_err(gkv, dkv) <= 2e-2
    rdq, rdk, rdw, rloss = O.indexer_kl_loss_grad(q_b, kv_b, qi, ki, w, idx, ref_lse, scale)
    n = S  # B*S
    assert rel_err(qid.grad.cpu(), rdq / n) <= 1e-2
    assert rel_err(kid.grad.cpu()[:, :, 0], rdk / n) <= 1e-2
    assert rel_err(wd.grad.cpu(), rdw / n) <= 1e-2


def test_npu_dsa_under_activation_checkpointing():
    """The converted layer inside torch.utils.checkpoint (non-reentrant, as torchtitan's
    activation checkpointing wraps each block): the same gradients as the plain run, bit for
    bit, and the mass link holds no tensor between forward and backward (the attention node
    owns its inputs through save_for_backward, so the checkpoint's hooks see them)."""
    from unittest.mock import patch

    from torch.utils.checkpoint import checkpoint

    from torchtitan_npu_simulator_amd import converters as conv
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops
    from torchtitan_npu_simulator_amd.converters import dsa as dsa_mod
    from torchtitan_npu_simulator_amd.converters.dsa_indexer_loss import DSAIndexerLossAutoScaler

    model = _Model()
    conv.registry().converter_class("npu_dsa")(model_spec=SimpleNamespace(name="deepseek_v32")).convert(model)
    sdpa = model.layers["0"].attention.inner_attention
    S, H, K, HI, DI = 256, 32, 64, 64, 128
    g = torch.Generator().manual_seed(11)
    q = (torch.randn(1, H, S, 576, generator=g) / 24).bfloat16().to(DEV)
    kv = torch.randn(1, 1, S, 576, generator=g).bfloat16().to(DEV)
    qi = torch.randn(1, S, HI, DI, generator=g).bfloat16().to(DEV)
    ki = torch.randn(1, S, 1, DI, generator=g).bfloat16().to(DEV)
    w = (torch.rand(1, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5).to(DEV)
    dout = torch.randn(1, H, S, 512, generator=g).to(DEV)
    links = []

    class _Recorded(ops.MassLink):
        __slots__ = ()

        def __init__(self):
            super().__init__()
            links.append(self)

    def run(ckpt):
        leaves = [t.clone().requires_grad_(True) for t in (q, kv, qi, ki, w)]

        def layer(qq, kk, qii, kii, ww):
            loss, out = sdpa(qq, kk, kk[..., :512], None, 576 ** -0.5, qii, kii, ww, None, K)
            return DSAIndexerLossAutoScaler.apply(out, loss)

        y = checkpoint(layer, *leaves, use_reentrant=False) if ckpt else layer(*leaves)
        link = links[-1]
        assert not any(isinstance(getattr(link, a), torch.Tensor) for a in ops.MassLink.__slots__)
        (y.float() * dout).sum().backward()
        torch.cuda.synchronize()
        return [t.grad for t in leaves]

    with patch.object(dsa_mod.npu, "MassLink", _Recorded):
        plain = run(False)
        ckpt = run(True)
    for a, b in zip(plain, ckpt):
        assert torch.equal(a, b)
    assert all(float(t.abs().sum()) > 0 for t in plain)
