"""Converter / host-plumbing tests with the fused ops mocked (CPU).

Mirrors the reference's hardware-free converter tests
(tests/unit_tests/converters/test_npu_li.py:36-72, test_npu_smla.py:35-68 and
tests/unit_tests/models/test_dsa_indexer_loss.py:135-167): argument plumbing, dtypes,
shapes, -1 preservation, +offset, loss deferral and scaling, the registry.
"""

from __future__ import annotations

import weakref
from types import SimpleNamespace
from unittest.mock import patch

import pytest
import torch

from torchtitan_npu_simulator_amd import converters as conv
from torchtitan_npu_simulator_amd.converters import dsa as dsa_mod
from torchtitan_npu_simulator_amd.converters import npu_smla as smla_mod
from torchtitan_npu_simulator_amd.converters.dsa_indexer_loss import (
    DSAIndexerLossAutoScaler,
    DSAIndexerLossLoggingHelper,
)


# ---------------------------------------------------------------- registry
def test_registry_configs_and_lookup():
    for name in ("npu_dsa", "npu_smla"):
        cfg = conv.get_model_converter_config(name)
        assert cfg is not None and cfg.to_dict() == {"name": name}
        assert conv.has_npu_converter([cfg], name)
        assert not conv.has_npu_converter([cfg], "other")
    assert conv.get_model_converter_config("missing") is None


def test_converter_errors_are_wrapped():
    class Boom(conv.ModelCustomConverter):
        def convert(self, model):
            raise ValueError("bad model")

    @conv.register_model_converter("test_boom")
    class BoomConfig(conv.ModelCustomConfig):
        model_converter = Boom

    cls = conv.registry().converter_class("test_boom")
    with pytest.raises(RuntimeError, match="Failed to apply custom model config 'test_boom'"):
        cls(cls.Config(), model_spec=SimpleNamespace(name="x")).convert(torch.nn.Module())


# ---------------------------------------------------------------- npu_smla LiCompute
class LiCompute(torch.nn.Module):  # stand-in with the reference's attributes
    def __init__(self, ratio, index_topk):
        super().__init__()
        self.ratio = ratio
        self.index_topk = index_topk


def test_npu_li_compute_plumbing():
    B, S, D, K, r = 2, 16, 8, 6, 4
    calls = {}

    def fake(q, k, w, *args, **kw):
        calls.update(q=q, k=k, w=w, args=args, kw=kw)
        idx = torch.full((B, S, 1, K), 10, dtype=torch.int32)
        idx[0, 0, 0, 0] = -1
        idx[..., 1] += kw["index_offset"]  # the HIP top-k adds the offset to valid entries
        idx[0, 0, 0, 0] = -1
        return idx, torch.randn(B, S, 1, K)

    mod = smla_mod.NpuLiCompute(LiCompute(r, K))
    with patch.object(smla_mod.npu, "npu_lightning_indexer", side_effect=fake):
        ind, sc = mod(torch.randn(B, S, 4, D), torch.randn(B, S // r, D), torch.randn(B, S, 4), seqlen=S, offset=100)
    assert calls["q"].dtype == torch.bfloat16 and calls["k"].dtype == torch.bfloat16
    assert calls["w"].dtype == torch.bfloat16
    assert calls["k"].ndim == 4
    assert calls["args"][9] == r  # cmp_ratio
    assert calls["args"][5] == K and calls["args"][6] == 3  # sparse_count, sparse_mode
    assert ind.shape == (B, S, K) and sc.shape == (B, S, K)
    assert ind[0, 0, 0].item() == -1
    assert ind[0, 0, 1].item() == 110


def test_npu_smla_converter_swaps_li_compute():
    model = torch.nn.Sequential(torch.nn.Linear(2, 2), LiCompute(4, 8))
    conv.registry().converter_class("npu_smla")(model_spec=SimpleNamespace(name="deepseek_v4")).convert(model)
    assert isinstance(model[1], smla_mod.NpuLiCompute)
    assert model[1].ratio == 4 and model[1].index_topk == 8


# ---------------------------------------------------------------- npu_dsa
class DSV32_SDPA(torch.nn.Module):  # stand-in of the reference class name
    def __init__(self):
        super().__init__()
        self.config = SimpleNamespace(kv_lora_rank=512, qk_rope_head_dim=64)

    def forward(self, *a, **k):
        raise AssertionError("torch-native forward should have been replaced")


class _Attn(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.inner_attention = DSV32_SDPA()


class _Block(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.attention = _Attn()


class _Model(torch.nn.Module):
    def __init__(self, n):
        super().__init__()
        self.layers = torch.nn.ModuleDict({str(i): _Block() for i in range(n)})


def test_npu_dsa_converter_installs_forward_and_loss():
    model = _Model(3)
    conv.registry().converter_class("npu_dsa")(model_spec=SimpleNamespace(name="deepseek_v32")).convert(model)
    assert DSV32_SDPA.forward is dsa_mod.dsa_forward
    for i, blk in model.layers.items():
        inner = blk.attention.inner_attention
        assert isinstance(inner.compute_dsa_indexer_loss, dsa_mod.SparseLightningIndexerKLLoss)
        assert inner.layer_number == int(i) and inner.num_layers == 3


def test_npu_dsa_converter_skips_other_models():
    model = _Model(1)
    conv.registry().converter_class("npu_dsa")(model_spec=SimpleNamespace(name="qwen3")).convert(model)
    assert not hasattr(model.layers["0"].attention.inner_attention, "layer_number")


def _dsa_case(B=1, H=4, S=8, HI=2, DI=16):
    self_ = SimpleNamespace(config=SimpleNamespace(kv_lora_rank=512, qk_rope_head_dim=64), layer_number=0,
                            num_layers=1, compute_dsa_indexer_loss=dsa_mod.SparseLightningIndexerKLLoss())
    q = torch.randn(B, H, S, 576)
    kv = torch.randn(B, 1, S, 576)
    qi, ki, w = torch.randn(B, S, HI, DI, requires_grad=True), torch.randn(B, S, 1, DI), torch.rand(B, S, HI)
    return self_, q, kv, qi, ki, w


class _FakeLinkedAttention(torch.autograd.Function):
    """Stands in for the linked attention op: it saves its forward statistics on its own node
    (as the real op does), leaves only a weak reference to that node in the link, and its
    backward hands a mass to the link."""

    @staticmethod
    def forward(ctx, q_nope, after, link, mass):
        B, S, H, _ = q_nope.shape
        K = mass.shape[-1] if mass is not None else 4
        idx = torch.zeros(B, S, K, dtype=torch.int32)
        ctx.save_for_backward(q_nope, q_nope, idx, q_nope, torch.zeros(B, S, H), torch.ones(B, S, H))
        ctx.link, ctx.mass = link, mass
        link.attn = weakref.ref(ctx)
        link.scale, link.q_offset = 0.1, 0
        return q_nope.new_zeros(q_nope.shape)

    @staticmethod
    def backward(ctx, dout):
        ctx.link.mass = ctx.mass
        return dout, torch.zeros(()), None, None


def test_dsa_forward_plumbing_and_loss_deferral():
    B, H, S, K, HI, DI = 1, 4, 8, 4, 2, 16
    self_, q, kv, qi, ki, w = _dsa_case(B, H, S, HI, DI)
    seen = {}

    def fake_li(q_, k_, w_, **kw):
        seen["li"] = kw
        return torch.zeros(B, S, 1, K, dtype=torch.int32), None

    def fake_sfa(q_, k_, idx, scale, after, link, d_v=512):
        seen["sfa"] = dict(q=q_, k=k_, idx=idx, scale=scale, d_v=d_v)
        out = _FakeLinkedAttention.apply(torch.zeros(B, S, H, d_v, requires_grad=True), after, link, None)
        seen["link"] = link
        return out, torch.zeros(B, S, H), torch.ones(B, S, H)

    with patch.object(dsa_mod.npu, "npu_lightning_indexer", side_effect=fake_li), \
            patch.object(dsa_mod.npu, "sparse_flash_attention_linked", side_effect=fake_sfa):
        loss, out = dsa_mod.dsa_forward(self_, q, kv, kv[..., :512], None, 0.1, qi, ki, w, None, K)
    assert seen["li"]["sparse_count"] == K and seen["li"]["sparse_mode"] == 3
    s = seen["sfa"]
    assert s["q"].shape == (B, S, H, 576) and s["k"].shape == (B, S, 1, 576) and s["d_v"] == 512
    assert s["idx"].shape == (B, S, 1, K) and s["scale"] == 0.1
    assert out.shape == (B, H, S, 512)
    assert float(loss.detach()) == 0.0  # deferred to backward
    # the link holds no tensor between forward and backward (the attention node owns them)
    link = seen["link"]
    assert not any(isinstance(getattr(link, a), torch.Tensor) for a in type(link).__slots__)

    # backward of the loss alone: the attention node is not on the path, so the loss
    # recomputes the mass from the attention node's saved forward statistics; the upstream
    # grad scales the KL gradients as a tensor (no host round trip) and loss/(B*S) is logged
    def fake_mass(q_, kv_, idx_, smax_, ssum_, scale_, *, q_offset=0):
        seen["mass_args"] = (q_, kv_, idx_, smax_, ssum_, scale_, q_offset)
        return torch.rand(B, S, K)

    def fake_kl(qi_, ki_, w_, idx_, mass_, *, q_offset=0, loss_scale=1.0, eps=1e-8, grad_scale=1.0):
        seen["grad_scale"] = grad_scale
        g = grad_scale
        return (torch.ones(B, S, HI, DI) * g, torch.ones(B, S, DI) * g, torch.ones(B, S, HI) * g,
                torch.full((B, S), 1.0))

    DSAIndexerLossLoggingHelper.tracker.clear()
    with patch.object(dsa_mod.npu, "attn_mass", side_effect=fake_mass), \
            patch.object(dsa_mod.npu, "indexer_kl_grad_from_mass", side_effect=fake_kl):
        (loss * 3.0).backward()
    assert seen["mass_args"][0].shape == (B, S, H, 512) and seen["mass_args"][5] == 0.1
    assert torch.equal(seen["mass_args"][4], torch.ones(B, S, H))
    # d(loss/(B*S))/d(z) = 1/(B*S), times 3
    torch.testing.assert_close(qi.grad, torch.full_like(qi, 3.0 / (B * S)))
    assert isinstance(seen["grad_scale"], torch.Tensor)
    assert DSAIndexerLossLoggingHelper.tracker["values"][0].item() == pytest.approx(S / (B * S))


def test_dsa_loss_backward_waits_for_the_attention_mass():
    """The loss's output is an input of the attention op, so in a backward through both the
    attention backward runs first and its mass reaches the loss (no recompute)."""
    B, H, S, K, HI, DI = 1, 4, 8, 4, 2, 16
    self_, q, kv, qi, ki, w = _dsa_case(B, H, S, HI, DI)
    mass = torch.rand(B, S, K)
    seen = {}

    def fake_li(q_, k_, w_, **kw):
        return torch.zeros(B, S, 1, K, dtype=torch.int32), None

    def fake_sfa(q_, k_, idx, scale, after, link, d_v=512):
        out = _FakeLinkedAttention.apply(q_[..., :d_v].detach().requires_grad_(True), after, link, mass)
        return out, None, None

    def fake_kl(qi_, ki_, w_, idx_, mass_, **kw):
        seen["mass"] = mass_
        return torch.zeros(B, S, HI, DI), torch.zeros(B, S, DI), torch.zeros(B, S, HI), torch.zeros(B, S)

    with patch.object(dsa_mod.npu, "npu_lightning_indexer", side_effect=fake_li), \
            patch.object(dsa_mod.npu, "sparse_flash_attention_linked", side_effect=fake_sfa):
        loss, out = dsa_mod.dsa_forward(self_, q, kv, kv[..., :512], None, 0.1, qi, ki, w, None, K)
    with patch.object(dsa_mod.npu, "attn_mass", side_effect=AssertionError("mass recomputed")), \
            patch.object(dsa_mod.npu, "indexer_kl_grad_from_mass", side_effect=fake_kl):
        (out.sum() + loss).backward()
    assert seen["mass"] is mass


def test_dsa_linked_loss_second_backward_with_retain_graph():
    """A graph kept with retain_graph=True backpropagates twice: the attention backward hands
    the mass over again and the loss backward finds the link intact."""
    B, H, S, K, HI, DI = 1, 4, 8, 4, 2, 16
    self_, q, kv, qi, ki, w = _dsa_case(B, H, S, HI, DI)
    mass = torch.rand(B, S, K)
    calls = []

    def fake_li(q_, k_, w_, **kw):
        return torch.zeros(B, S, 1, K, dtype=torch.int32), None

    def fake_sfa(q_, k_, idx, scale, after, link, d_v=512):
        return _FakeLinkedAttention.apply(q_[..., :d_v].detach().requires_grad_(True), after, link, mass), None, None

    def fake_kl(qi_, ki_, w_, idx_, mass_, **kw):
        calls.append(mass_)
        assert idx_.shape == (B, S, K) and idx_.dtype == torch.int32
        return torch.ones(B, S, HI, DI), torch.zeros(B, S, DI), torch.zeros(B, S, HI), torch.zeros(B, S)

    with patch.object(dsa_mod.npu, "npu_lightning_indexer", side_effect=fake_li), \
            patch.object(dsa_mod.npu, "sparse_flash_attention_linked", side_effect=fake_sfa):
        loss, out = dsa_mod.dsa_forward(self_, q, kv, kv[..., :512], None, 0.1, qi, ki, w, None, K)
    with patch.object(dsa_mod.npu, "attn_mass", side_effect=AssertionError("mass recomputed")), \
            patch.object(dsa_mod.npu, "indexer_kl_grad_from_mass", side_effect=fake_kl):
        (out.sum() + loss).backward(retain_graph=True)
        g1 = qi.grad.clone()
        (out.sum() + loss).backward()
    assert len(calls) == 2 and all(m is mass for m in calls)
    torch.testing.assert_close(qi.grad, 2 * g1)


def test_dsa_linked_loss_alone_without_attention_node_raises():
    """With the attention output (and so its node) gone, a backward of the loss alone has no
    forward statistics to recompute the target from: a clear error, not a silent zero."""
    B, H, S, K, HI, DI = 1, 4, 8, 4, 2, 16
    self_, q, kv, qi, ki, w = _dsa_case(B, H, S, HI, DI)

    def fake_li(q_, k_, w_, **kw):
        return torch.zeros(B, S, 1, K, dtype=torch.int32), None

    def fake_sfa(q_, k_, idx, scale, after, link, d_v=512):
        return _FakeLinkedAttention.apply(torch.zeros(B, S, H, d_v, requires_grad=True), after, link, None), None, None

    with patch.object(dsa_mod.npu, "npu_lightning_indexer", side_effect=fake_li), \
            patch.object(dsa_mod.npu, "sparse_flash_attention_linked", side_effect=fake_sfa):
        loss, out = dsa_mod.dsa_forward(self_, q, kv, kv[..., :512], None, 0.1, qi, ki, w, None, K)
    del out
    with pytest.raises(RuntimeError, match="backpropagate through the attention output"):
        loss.backward()


def test_dsa_forward_rejects_multi_kv_heads():
    self_ = SimpleNamespace(config=SimpleNamespace(kv_lora_rank=512, qk_rope_head_dim=64))
    with pytest.raises(NotImplementedError):
        dsa_mod.dsa_forward(self_, torch.zeros(1, 2, 4, 576), torch.zeros(1, 2, 4, 576), torch.zeros(1, 2, 4, 512))


# ---------------------------------------------------------------- loss plumbing
def test_auto_scaler_injects_loss_scale():
    from torchtitan_npu_simulator_amd.converters import dsa_indexer_loss as m

    DSAIndexerLossAutoScaler.set_loss_scale(torch.tensor(0.5))
    assert m.LOSS_SCALE.item() == 0.5
    out = torch.randn(3, requires_grad=True)
    aux = torch.tensor(2.0, requires_grad=True)
    y = DSAIndexerLossAutoScaler.apply(out, aux)
    y.sum().backward()
    assert aux.grad.item() == 0.5
    torch.testing.assert_close(out.grad, torch.ones(3))
    DSAIndexerLossAutoScaler.set_loss_scale(torch.tensor(1.0))


def test_logging_helper_save_clean_and_track():
    DSAIndexerLossLoggingHelper.tracker.clear()
    DSAIndexerLossLoggingHelper.save_loss_to_tracker(torch.tensor(0.123), layer_number=0, num_layers=4)
    assert DSAIndexerLossLoggingHelper.tracker["values"][0].item() == pytest.approx(0.123)
    DSAIndexerLossLoggingHelper.save_loss_to_tracker(torch.tensor(0.2), layer_number=2, num_layers=4)
    assert DSAIndexerLossLoggingHelper.track_dsa_indexer_metrics(2) == pytest.approx((0.123 + 0.2) / 2 / 2)
    assert DSAIndexerLossLoggingHelper.tracker["values"].abs().sum().item() == 0.0
    with pytest.raises(ValueError):
        DSAIndexerLossLoggingHelper.save_loss_to_tracker(torch.tensor(1.0), layer_number=7, num_layers=4)


def test_logging_helper_skips_none_layer_number():
    DSAIndexerLossLoggingHelper.tracker.clear()
    DSAIndexerLossLoggingHelper.save_loss_to_tracker(torch.tensor(0.1), layer_number=None, num_layers=4)
    assert "values" not in DSAIndexerLossLoggingHelper.tracker


def test_sparse_mode_offsets():
    from torchtitan_npu_simulator_amd.torch_npu_ops import _resolve_q_offset

    assert _resolve_q_offset(3, 128, 512, None) == 384  # bottom-right causal (one CP shard)
    assert _resolve_q_offset(3, 128, 128, None) == 0
    assert _resolve_q_offset(3, 128, 512, 7) == 7
    assert _resolve_q_offset(0, 128, 512, None) >= 1 << 40  # no mask
    with pytest.raises(ValueError):
        _resolve_q_offset(1, 4, 4, None)
