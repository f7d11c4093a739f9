"""Host logic of the packed-sequence (global TND) DeepSeek-V4 branch, on the CPU.

* ``sharedkv_tnd_indices`` (the slot indices a packed batch runs with) against
  ``v4_attention_indices`` applied to each sequence on its own (the BSND rule the GPU tests
  pin against the oracle), for ratio 4 (given top-k, with entries the causal rule must
  drop), ratio 128 (every causal block, padded to the longest sequence) and ratio 1;
* the converter's packed branch: which modules it swaps, the shared metadata cache, the
  compressors switched to TND metadata, and the error paths of the reference's wrappers
  (converters/kernels/npu_smla.py:59-80, :842-917, :1274-1316).
"""

from types import SimpleNamespace

import pytest
import torch

from torchtitan_npu_simulator_amd import torch_npu_ops as ops
from torchtitan_npu_simulator_amd.converters import npu_smla as smla


def _packed(lengths, ratio, K, seed):
    g = torch.Generator().manual_seed(seed)
    cu_q = [0]
    for n in lengths:
        cu_q.append(cu_q[-1] + n)
    n_cmp = [n // ratio for n in lengths] if ratio > 1 else [0] * len(lengths)
    cu_c = [0]
    for n in n_cmp:
        cu_c.append(cu_c[-1] + n)
    local = []
    for n, nc in zip(lengths, n_cmp):
        rows = torch.full((n, K), -1, dtype=torch.int32)
        for p in range(n):
            vis = min(nc, (p + 1) // ratio) if ratio > 1 else 0
            c = min(K, vis)
            if c:
                rows[p, :c] = torch.randperm(vis, generator=g)[:c].int()
        local.append(rows)
    return cu_q, cu_c, n_cmp, local


@pytest.mark.parametrize("ratio,K", [(4, 8), (128, 0), (1, 0)])
def test_tnd_indices_match_per_sequence_rule(ratio, K):
    lengths = [37, 300, 5, 129]
    cu_q, cu_c, n_cmp, local = _packed(lengths, ratio, max(K, 1), seed=ratio)
    T = cu_q[-1]
    win = 16
    cmp_idx = torch.cat(local) if ratio == 4 else None
    max_cmp = max(n_cmp)
    got = ops.sharedkv_tnd_indices(torch.tensor(cu_q), torch.tensor(cu_q), T, T, torch.device("cpu"),
                                   win_left=win - 1, cmp_ratio=ratio, cu_seqlens_cmp_kv=torch.tensor(cu_c),
                                   cmp_indices=cmp_idx, max_cmp=max_cmp)
    W = win
    assert got.shape == (T, W + (K if ratio == 4 else (max_cmp if ratio > 1 else 0)))
    for i, n in enumerate(lengths):
        q0, c0 = cu_q[i], cu_c[i]
        ci = None if ratio != 4 else torch.where(local[i] < 0, local[i], local[i] + n).unsqueeze(0)
        ref = ops.v4_attention_indices(1, n, torch.device("cpu"), win_left=win - 1, cmp_ratio=ratio,
                                       n_cmp=n_cmp[i], cmp_indices=ci)[0].long()
        # BSND numbering (window rows 0..n-1, compressed rows n + c) -> packed rows
        exp = torch.where(ref < 0, ref, torch.where(ref < n, ref + q0, ref - n + T + c0))
        rows = got[q0:q0 + n].long()
        assert torch.equal(rows[:, :W], exp[:, :W])
        if ratio > 1:
            k = exp.shape[1] - W
            assert torch.equal(rows[:, W:W + k], exp[:, W:])
            assert torch.all(rows[:, W + k:] == -1)


def test_tnd_indices_drop_entries_the_causal_rule_hides():
    cu_q, cu_c = [0, 40], [0, 10]
    idx = torch.full((40, 3), -1, dtype=torch.int32)
    idx[:, 0] = 9  # visible from position 39 only ((39 + 1) // 4 = 10)
    idx[:, 1] = 10  # past the sequence's compressed rows
    idx[7, 2] = 1  # (7 + 1) // 4 = 2 rows visible at position 7: kept
    got = ops.sharedkv_tnd_indices(torch.tensor(cu_q), None, 40, 40, torch.device("cpu"), win_left=3, cmp_ratio=4,
                                   cu_seqlens_cmp_kv=torch.tensor(cu_c), cmp_indices=idx)
    cmp = got[:, 4:]
    assert cmp[39, 0] == 40 + 9 and torch.all(cmp[:39, 0] == -1)
    assert torch.all(cmp[:, 1] == -1)
    assert cmp[7, 2] == 40 + 1


def test_tnd_indices_without_window_columns():
    cu_q, cu_c = [0, 8, 20], [0, 2, 5]
    idx = torch.zeros(20, 1, dtype=torch.int32)
    got = ops.sharedkv_tnd_indices(torch.tensor(cu_q), None, 20, 0, torch.device("cpu"), cmp_ratio=4,
                                   cu_seqlens_cmp_kv=torch.tensor(cu_c), cmp_indices=idx, window=False)
    assert got.shape == (20, 1)
    # row 0 of each sequence becomes visible at position 3; packed numbering from 0
    assert got[:3, 0].tolist() == [-1, -1, -1] and got[3, 0] == 0
    assert got[8:11, 0].tolist() == [-1, -1, -1] and got[11, 0] == 2


class LiCompute(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.ratio, self.index_topk = 4, 8


class SparseAttention(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.softmax_scale, self.compress_ratio = 0.1, 4


class Compressor(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.use_tnd_metadata = False


class InnerAttention(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.compress_ratio = 4
        self.attn_sink = torch.nn.Parameter(torch.zeros(4))
        self.sparse_attn = SparseAttention()
        self.li_compute = LiCompute()


class _Layer(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.compressor = Compressor()
        self.inner_attention = InnerAttention()


class _Model(torch.nn.Module):
    def __init__(self, use_global_tnd):
        super().__init__()
        self.model_args = SimpleNamespace(use_global_tnd=use_global_tnd, head_dim=64, index_topk=8, index_n_heads=4,
                                          index_head_dim=32)
        self.layers = torch.nn.ModuleList([_Layer(), _Layer()])


def test_converter_packed_branch_swaps_modules():
    model = _Model(use_global_tnd=True)
    smla.NpuSMLAConverter(None).convert(model)
    caches = set()
    for layer in model.layers:
        inner = layer.inner_attention
        assert isinstance(inner, smla.NpuInnerAttentionSMLA)
        assert isinstance(inner.li_compute, smla.NpuLiComputeSMLA)
        assert isinstance(inner.sparse_attn, SparseAttention)  # kept: the packed op replaces it inside
        assert layer.compressor.use_tnd_metadata
        caches.add(id(inner._smla_metadata_cache))
        caches.add(id(inner.li_compute._smla_metadata_cache))
    assert len(caches) == 1  # one cache per model
    assert model.layers[0].inner_attention.attn_sink is not None


def test_converter_per_batch_branch_without_global_tnd():
    model = _Model(use_global_tnd=False)
    smla.NpuSMLAConverter(None).convert(model)
    layer = model.layers[0]
    assert isinstance(layer.inner_attention.li_compute, smla.NpuLiCompute)
    assert isinstance(layer.inner_attention.sparse_attn, smla.NpuSparseAttention)
    assert not isinstance(layer.inner_attention, smla.NpuInnerAttentionSMLA)
    with pytest.raises(RuntimeError, match="use_global_tnd"):
        smla.NpuSMLAConverter.convert_smla_kernel(model)


def test_metadata_cache_rebuilds_per_mask_batch():
    calls = []

    def builder(masks, model_args, ratio, *args):
        calls.append((masks.cache_id, ratio, args))
        return torch.tensor([len(calls)])

    cache = smla.SMLAMetadataCache(SimpleNamespace())
    m1, m2 = SimpleNamespace(cache_id=1), SimpleNamespace(cache_id=2)
    a = cache.get_or_create(m1, 4, "sparse_attn", builder, 16)
    assert cache.get_or_create(m1, 4, "sparse_attn", builder, 16) is a
    cache.get_or_create(m1, 128, "sparse_attn", builder, 16)
    assert len(calls) == 2
    cache.get_or_create(m2, 4, "sparse_attn", builder, 16)  # new batch: everything rebuilt
    cache.get_or_create(m1, 4, "sparse_attn", builder, 16)
    assert len(calls) == 4
    # masks without an id are keyed by the object
    m3 = SimpleNamespace(cache_id=-1)
    cache.get_or_create(m3, 4, "x", builder)
    cache.get_or_create(m3, 4, "x", builder)
    assert len(calls) == 5
    with pytest.raises(RuntimeError, match="metadata 'y' is missing"):
        smla._require_op_metadata(cache, m3, 4, "y", lambda *a: None)


def test_packed_wrappers_refuse_bad_shapes():
    cache = smla.SMLAMetadataCache(SimpleNamespace())
    masks = SimpleNamespace(cache_id=0)
    q = torch.zeros(4, 2, 8)
    with pytest.raises(RuntimeError, match="query must be TND"):
        smla.npu_sparse_flash_mla(q.unsqueeze(0), torch.zeros(4, 8), None, None, torch.zeros(2), 1.0, 1,
                                  attention_masks=masks, metadata_cache=cache)
    with pytest.raises(RuntimeError, match="ori_kv must be TND"):
        smla.npu_sparse_flash_mla(q, torch.zeros(4, 1, 8), None, None, torch.zeros(2), 1.0, 1,
                                  attention_masks=masks, metadata_cache=cache)
    with pytest.raises(RuntimeError, match="attention masks"):
        smla.npu_sparse_flash_mla(q, torch.zeros(4, 8), None, None, torch.zeros(2), 1.0, 1)
    with pytest.raises(RuntimeError, match="metadata cache"):
        smla.npu_sparse_flash_mla(q, torch.zeros(4, 8), None, None, torch.zeros(2), 1.0, 1, attention_masks=masks)
    with pytest.raises(RuntimeError, match="cmp_sparse_indices must be TND"):
        smla.npu_sparse_flash_mla(q, torch.zeros(4, 8), torch.zeros(1, 8), torch.zeros(4, 2, 3, dtype=torch.int32),
                                  torch.zeros(2), 1.0, 4, attention_masks=masks, metadata_cache=cache)
    li = SimpleNamespace(index_topk=4, ratio=4)
    with pytest.raises(RuntimeError, match="q_indexer must be TND"):
        smla.sdpa_to_li_adapter_smla(li, torch.zeros(1, 4, 2, 8), torch.zeros(1, 8), torch.zeros(4, 2), 4, 0, masks,
                                     cache)


def test_sharedkv_ops_accept_tnd_layout_arguments():
    """Layout checks of the binding-level ops: TND needs cu_seqlens_q; BSND takes none."""
    assert ops._check_sharedkv_args("TND", "TND", None, (), (torch.tensor([0, 4]), None, None), 4, 3) is True
    assert ops._check_sharedkv_args("BSND", "BSND", None, (), (None, None, None), 4, 3) is False
    with pytest.raises(ValueError, match="cu_seqlens_q"):
        ops._check_sharedkv_args("TND", "TND", None, (), (None, None, None), 4, 3)
    with pytest.raises(NotImplementedError, match="need layout TND"):
        ops._check_sharedkv_args("BSND", "BSND", None, (), (torch.tensor([0, 4]), None, None), 4, 3)
    with pytest.raises(NotImplementedError, match="layouts"):
        ops._check_sharedkv_args("TND", "BSND", None, (), (None,), 4, 3)


def test_grad_metadata_record_kind_matches_on_host_and_device():
    """The backward record says kind 2 in the host tuple and in the int32 record alike."""
    from torchtitan_npu_simulator_amd import smla_ops

    cu = torch.tensor([0, 5, 9], dtype=torch.int32)
    kw = dict(cu_seqlens_q=cu, cu_seqlens_ori_kv=cu, batch_size=2, max_seqlen_q=5, max_seqlen_ori_kv=5,
              num_heads_q=8, head_dim=512)
    fwd = smla_ops.sparse_flash_mla_metadata(**kw)
    bwd = smla_ops.sparse_flash_mla_grad_metadata(**kw)
    assert fwd._dsa_record[1] == 1 and int(fwd[1]) == 1
    assert bwd._dsa_record[1] == 2 and int(bwd[1]) == 2
    assert bwd._dsa_record[2:] == fwd._dsa_record[2:]
    assert torch.equal(bwd[2:], fwd[2:])
