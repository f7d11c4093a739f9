"""DeepSeek-V4 shared-KV sparse attention (window + compressed KV + per-head sink), CPU part.

The oracle's ``sparse_attn_sink`` restates SparseAttention.forward
(models/deepseek_v4/model.py:573-623) and is pinned here by a sink of -inf (it must equal
the plain gathered attention with v = the whole row), brute-force loops over (s, h), and an
fp64 gradcheck; the op layer's index builder must select the same key sets as the
reference's GetWindowTopkIdxs / GetCompressTopkIdxs (:467-488).
"""

from __future__ import annotations

import math
from types import SimpleNamespace
from unittest.mock import patch

import pytest
import torch

from oracle import dsa_oracle as O
from torchtitan_npu_simulator_amd import torch_npu_ops as ops
from torchtitan_npu_simulator_amd.converters import npu_smla as smla_mod


def _inputs(B, S, H, D, T, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, D, generator=g, dtype=dtype)
    kv = torch.randn(B, T, D, generator=g, dtype=dtype)
    sink = torch.randn(H, generator=g, dtype=dtype)
    return q, kv, sink


def test_sink_minus_inf_is_plain_sparse_attention():
    B, S, H, D, r = 1, 24, 3, 8, 4
    q, kv, _ = _inputs(B, S, H, D, S + S // r)
    idx = O.v4_attn_indices(B, S, 6, r, S)
    out, lse = O.sparse_attn_sink(q, kv, torch.full((H,), float("-inf"), dtype=torch.float64), idx, 0.3)
    ref_out, ref_lse = O.sparse_mla_fwd(q, kv, idx, 0.3, d_v=D, q_offset=1 << 40)
    torch.testing.assert_close(out, ref_out, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, ref_lse, rtol=1e-12, atol=1e-12)


def test_sink_attention_brute_force():
    B, S, H, D, r, W = 2, 9, 2, 5, 4, 3
    q, kv, sink = _inputs(B, S, H, D, S + S // r, seed=1)
    idx = O.v4_attn_indices(B, S, W, r, S)
    out, lse = O.sparse_attn_sink(q, kv, sink, idx, 0.7)
    for b in range(B):
        for s in range(S):
            keys = [int(j) for j in idx[b, s] if j >= 0]
            for h in range(H):
                logits = [0.7 * float(q[b, s, h] @ kv[b, j]) for j in keys] + [float(sink[h])]
                m = max(logits)
                z = sum(math.exp(x - m) for x in logits)
                o = sum(math.exp(x - m) / z * kv[b, j] for x, j in zip(logits[:-1], keys))
                torch.testing.assert_close(out[b, s, h], o, rtol=1e-12, atol=1e-12)
                assert abs(float(lse[b, s, h]) - (m + math.log(z))) < 1e-12


def test_sink_attention_gradcheck():
    B, S, H, D, r = 1, 8, 2, 4, 4
    q, kv, sink = _inputs(B, S, H, D, S + S // r, seed=2)
    idx = O.v4_attn_indices(B, S, 3, r, S)
    q.requires_grad_(True)
    kv.requires_grad_(True)
    sink.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b, c: O.sparse_attn_sink(a, b, c, idx, 0.5)[0], (q, kv, sink))


@pytest.mark.parametrize("ratio,given", [(4, True), (128, False), (4, False), (1, False)])
def test_index_builder_matches_reference_sets(ratio, given):
    B, S, W = 2, 300, 128
    n_cmp = S // ratio if ratio > 1 else 0
    cmp = None
    if given:  # a top-k like LiCompute's: valid causal blocks + S, -1 padded
        g = torch.Generator().manual_seed(3)
        K = 16
        cmp = torch.full((B, S, K), -1, dtype=torch.int32)
        for b in range(B):
            for s in range(S):
                nv = min(n_cmp, (s + 1) // ratio)
                c = min(K, nv)
                if c:
                    cmp[b, s, :c] = torch.randperm(nv, generator=g)[:c].int() + S
    got = ops.v4_attention_indices(B, S, "cpu", win_left=W - 1, cmp_ratio=ratio, n_cmp=n_cmp, cmp_indices=cmp)
    ref = O.v4_attn_indices(B, S, W, ratio, S, cmp_idxs=cmp)
    for b in range(B):
        for s in range(S):
            assert sorted(v for v in got[b, s].tolist() if v >= 0) == sorted(v for v in ref[b, s].tolist() if v >= 0)


def test_npu_sparse_attention_plumbing():
    calls = {}

    def fake(*args, **kw):
        calls.update(args=args, kw=kw)
        return torch.zeros(2, 16, 4, 8)

    parent = SimpleNamespace(softmax_scale=0.125, compress_ratio=4, window_size=128)
    mod = smla_mod.NpuSparseAttention(torch.nn.Module())
    mod.__dict__.update(parent.__dict__)
    idx = torch.zeros(2, 16, 6, dtype=torch.int64)
    with patch.object(smla_mod.npu, "npu_sparse_attn_shared_kv", side_effect=fake):
        mod(torch.randn(2, 16, 4, 8), torch.randn(2, 16, 8), torch.randn(4), torch.randn(2, 4, 8), idx)
    a = calls["args"]
    assert a[3].dtype == torch.int32 and a[4].dtype == torch.float32
    assert a[5] == 0.125 and a[6] == 4 and calls["kw"]["ori_win_left"] == 127
    parent.compress_ratio = 128
    mod.__dict__.update(parent.__dict__)
    with patch.object(smla_mod.npu, "npu_sparse_attn_shared_kv", side_effect=fake):
        mod(torch.randn(2, 16, 4, 8), torch.randn(2, 16, 8), torch.randn(4), torch.randn(2, 1, 8), None)
    assert calls["args"][3] is None and calls["args"][6] == 128


def test_npu_smla_converter_swaps_sparse_attention():
    from torchtitan_npu_simulator_amd import converters as conv

    class SparseAttention(torch.nn.Module):  # stand-in with the reference's attributes
        def __init__(self):
            super().__init__()
            self.softmax_scale, self.compress_ratio, self.window_size = 0.1, 4, 128

    model = torch.nn.Sequential(torch.nn.Linear(2, 2), SparseAttention())
    conv.registry().converter_class("npu_smla")(model_spec=SimpleNamespace(name="deepseek_v4")).convert(model)
    assert isinstance(model[1], smla_mod.NpuSparseAttention) and model[1].window_size == 128


def test_selected_attn_dist_is_sink_attention_mass():
    """The LiLoss target equals the compressed-slot probabilities of sparse_attn_sink,
    summed over heads / H (recomputed from its lse), and rows sum to at most one."""
    B, S, H, D, r, W = 1, 20, 3, 6, 4, 5
    q, kv_all, sink = _inputs(B, S, H, D, S + S // r, seed=7)
    kv, kvc = kv_all[:, :S], kv_all[:, S:]
    g = torch.Generator().manual_seed(8)
    K = 3
    cmp = torch.full((B, S, K), -1, dtype=torch.int32)
    for s in range(S):
        nv = (s + 1) // r
        c = min(K, nv)
        if c:
            cmp[0, s, :c] = torch.randperm(nv, generator=g)[:c].int()
    dist = O.v4_selected_attn_dist(q, kv, kvc, sink, cmp, 0.4, W)
    idx = O.v4_attn_indices(B, S, W, r, S, cmp_idxs=torch.where(cmp < 0, cmp, cmp + S))
    _, lse = O.sparse_attn_sink(q, kv_all, sink, idx, 0.4)
    for s in range(S):
        for k in range(K):
            j = int(cmp[0, s, k])
            if j < 0:
                assert dist[0, s, k] == 0
                continue
            p = torch.exp(0.4 * (q[0, s] @ kv_all[0, S + j]) - lse[0, s]).sum() / H
            assert abs(float(dist[0, s, k] - p)) < 1e-12
    assert float(dist.sum(-1).max()) <= 1.0 + 1e-12


def test_npu_smla_converter_swaps_li_loss():
    from torchtitan_npu_simulator_amd import converters as conv

    class LiLoss(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.softmax_scale, self.window_size, self.layer_id, self.n_layers = 0.1, 128, 0, 2

    model = torch.nn.Sequential(LiLoss())
    conv.registry().converter_class("npu_smla")(model_spec=SimpleNamespace(name="deepseek_v4")).convert(model)
    assert isinstance(model[0], smla_mod.NpuLiLoss) and model[0].softmax_scale == 0.1
