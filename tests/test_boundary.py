"""Op-boundary plumbing on the CPU (no GPU): the V4 shared-KV wrapper and its autograd
function, the metadata record, the dtype / cmp_ratio / deterministic conventions of the
indexer and KL ops, and the torch.library custom ops' fake implementations.

The first test mirrors the reference's hardware-free converter test
(tests/unit_tests/converters/test_npu_smla.py:35-68): SparseAttnSharedKV.apply mocked, the
arguments NpuSparseAttention hands it checked.
"""

from __future__ import annotations

import warnings
from types import SimpleNamespace
from unittest.mock import MagicMock, patch

import pytest
import torch

from torchtitan_npu_simulator_amd import torch_npu_ops as ops
from torchtitan_npu_simulator_amd.converters import npu_smla as smla_mod


def test_npu_sparse_attention_forward_flow():
    B, S, H, D, r, K = 2, 64, 16, 128, 4, 16
    query = torch.randn(B, S, H, D)
    kv_states = torch.randn(S, B, D)
    kv_compress = torch.randn(S // r, B, D)
    indices = torch.randint(0, S, (B, S, K)).to(torch.int64)
    sinks = torch.randn(1, 128)
    fused = MagicMock(return_value=torch.randn(B, S, H, D))
    parent = SimpleNamespace(softmax_scale=0.125, compress_ratio=r, window_size=128)
    with patch.object(ops.SparseAttnSharedKV, "apply", fused):
        out = smla_mod.NpuSparseAttention(parent).forward(query, kv_states, sinks, kv_compress, indices)
    args, _ = fused.call_args
    assert args[7].dtype == torch.int32 and args[7].shape == (B, S, 1, K)  # cmp_sparse_indices
    assert args[1].shape == (S, B, 1, D)  # ori_kv with its KV-head axis
    assert args[6] is None  # ori_sparse_indices: band mode
    assert args[9] == 0.125 and args[10] == r and args[11:15] == (4, 3, 127, 0)
    assert args[15:22] == (H, 1, D, B, S, B, K)  # heads q / kv, head_dim, batch, max lens, top-k
    assert args[22:] == ("BSND", "BSND")
    assert out.is_contiguous()


def test_shared_kv_ratio_128_passes_no_indices():
    fused = MagicMock(return_value=torch.randn(1, 8, 2, 16))
    with patch.object(ops.SparseAttnSharedKV, "apply", fused):
        ops.npu_sparse_attn_shared_kv(torch.randn(1, 8, 2, 16), torch.randn(1, 8, 16), torch.randn(1, 0, 16),
                                      torch.zeros(1, 8, 4, dtype=torch.int64), torch.zeros(2), 0.25, 128)
    args, _ = fused.call_args
    assert args[7] is None and args[21] == 0  # every causal block: no index tensor, topk 0


def test_sharedkv_metadata_record_and_check():
    meta = ops.npu_sparse_attn_sharedkv_metadata(None, None, None, None, None, 16, 1, 512, 2, 64, 64, 0, 32, 4, 4, 3,
                                                 127, 0, "BSND", "BSND", True, True, device="meta")
    assert meta.shape == (1024,) and meta.dtype == torch.int32
    rec = meta._dsa_record
    assert rec[0] == 0x44534B56 and rec[2:6] == (16, 1, 512, 2) and rec[9:11] == (32, 4) and rec[18] == 1
    q = torch.empty(2, 64, 16, 512, device="meta")
    ops._check_sharedkv_metadata(meta, q, torch.empty(2, 16, 1, 512, device="meta"), 4, 127, 0)
    with pytest.raises(ValueError, match="num_heads_q"):
        ops._check_sharedkv_metadata(meta, torch.empty(2, 64, 8, 512, device="meta"), q, 4, 127, 0)
    with pytest.raises(NotImplementedError):
        ops.npu_sparse_attn_sharedkv_metadata(num_heads_kv=2, device="meta")


def test_sharedkv_rejects_what_it_does_not_support():
    q = torch.randn(1, 8, 2, 16)
    kv = torch.randn(1, 8, 1, 16)
    with pytest.raises(NotImplementedError, match="layouts"):
        ops.npu_sparse_attn_sharedkv(q, kv, layout_q="TND", layout_kv="BSND")
    with pytest.raises(ValueError, match="cu_seqlens_q"):
        ops.npu_sparse_attn_sharedkv(q, kv, layout_q="TND", layout_kv="TND")
    with pytest.raises(NotImplementedError, match="band"):
        ops.npu_sparse_attn_sharedkv(q, kv, ori_sparse_indices=torch.zeros(1, 8, 1, 4, dtype=torch.int32))
    with pytest.raises(NotImplementedError, match="mask modes"):
        ops.npu_sparse_attn_sharedkv(q, kv, ori_mask_mode=3)


def _fake_indexer_call():
    def fake_indexer(q, k, w, kk, return_value=False, **kw):
        B, S = q.shape[:2]
        return torch.zeros(B, S, kk, dtype=torch.int32), (torch.randn(B, S, kk) if return_value else None)

    return patch.object(ops, "lightning_indexer", side_effect=fake_indexer)


@pytest.mark.parametrize("qdt,vdt", [(torch.bfloat16, torch.bfloat16), (torch.float8_e4m3fn, torch.bfloat16),
                                     (torch.float32, torch.float32)])
def test_indexer_values_in_query_dtype(qdt, vdt):
    B, S, H, D, K = 1, 12, 4, 8, 5
    with _fake_indexer_call():
        idx, vals = ops.npu_lightning_indexer(torch.zeros(B, S, H, D).to(qdt), torch.zeros(B, S, 1, D).to(qdt),
                                              torch.zeros(B, S, H), sparse_count=K, return_value=True)
    assert idx.shape == (B, S, 1, K) and idx.dtype == torch.int32
    assert vals.shape == (B, S, 1, K) and vals.dtype == vdt


def test_kl_op_cmp_ratio_dtypes_and_deterministic_warning():
    B, S, H, K, HI, DI, r = 1, 16, 4, 6, 8, 16, 4
    seen = {}

    def fake_mass(q, kv, idx, smax, ssum, scale, *, q_offset=0):
        seen["mass_q_offset"] = q_offset
        return torch.rand(B, S, K)

    def fake_kl(qi, ki, w, idx, mass, *, q_offset=0, loss_scale=1.0, eps=1e-8, grad_scale=1.0):
        seen["kl_q_offset"] = q_offset
        return (torch.randn(*qi.shape), torch.randn(ki.shape[0], ki.shape[1], ki.shape[-1]), torch.randn(*w.shape),
                torch.rand(B, S))

    qi = torch.randn(B, S, HI, DI).bfloat16()
    ki = torch.randn(B, S // r, 1, DI).bfloat16()
    w = torch.rand(B, S, HI).bfloat16()
    args = (torch.randn(B, S, H, 32), torch.randn(B, S // r, 1, 32), qi, ki, w, torch.zeros(B, S, 1, K,
            dtype=torch.int32), torch.zeros(B, S, H), torch.ones(B, S, H))
    ops._warned_nondeterministic = False
    with patch.object(ops, "attn_mass", side_effect=fake_mass), \
            patch.object(ops, "indexer_kl_grad_from_mass", side_effect=fake_kl), warnings.catch_warnings(record=True) as ws:
        warnings.simplefilter("always")
        dq, dk, dw, loss = ops.npu_sparse_lightning_indexer_grad_kl_loss(*args, 0.1, cmp_ratio=r, deterministic=True)
    assert seen["mass_q_offset"] == ops._NO_MASK_OFFSET == seen["kl_q_offset"]  # validity is in the indices
    assert dq.dtype == qi.dtype and dk.dtype == ki.dtype and dw.dtype == w.dtype and loss.dtype == torch.float32
    assert dk.shape == ki.shape and loss.shape == (1,)
    assert any("deterministic" in str(x.message) for x in ws)


def test_kl_deterministic_flag_is_met_on_the_mfma_shapes():
    """H_I = 64, D_I = 128 runs the KL MFMA kernel, whose d_key_index is bitwise reproducible:
    deterministic=True gives no warning there."""
    assert ops._kl_mfma_shape(torch.empty(1, 4, 64, 128), torch.empty(1, 4, 1, 128))
    assert not ops._kl_mfma_shape(torch.empty(1, 4, 8, 16), torch.empty(1, 4, 1, 16))


def test_custom_ops_fake_shapes_and_autograd_on_meta():
    from torchtitan_npu_simulator_amd import library  # noqa: F401  (registers dsa_mi355x::*)

    dev = "meta"
    B, S, H = 1, 16, 4
    lib = torch.ops.dsa_mi355x
    q = torch.empty(B, S, H, 512, dtype=torch.bfloat16, device=dev, requires_grad=True)
    qp = torch.empty(B, S, H, 64, dtype=torch.bfloat16, device=dev, requires_grad=True)
    k = torch.empty(B, S, 1, 512, dtype=torch.bfloat16, device=dev, requires_grad=True)
    kp = torch.empty(B, S, 1, 64, dtype=torch.bfloat16, device=dev, requires_grad=True)
    idx = torch.empty(B, S, 1, 8, dtype=torch.int32, device=dev)
    out, smax, ssum = lib.npu_sparse_flash_attention(q, k, k, idx, qp, kp, 0.1, 3)
    assert out.shape == (B, S, H, 512) and smax.shape == ssum.shape == (B, S, H) and smax.dtype == torch.float32
    out.sum().backward()
    assert q.grad.shape == q.shape and k.grad.shape == k.shape and kp.grad.shape == kp.shape
    qi = torch.empty(B, S, 64, 128, dtype=torch.float8_e4m3fn, device=dev)
    ki = torch.empty(B, S, 1, 128, dtype=torch.float8_e4m3fn, device=dev)
    w = torch.empty(B, S, 64, device=dev)
    i, v = lib.npu_lightning_indexer(qi, ki, w, sparse_count=8, return_value=True)
    assert i.shape == (B, S, 1, 8) and i.dtype == torch.int32 and v.dtype == torch.bfloat16
    i, v = lib.npu_lightning_indexer(qi, ki, w, sparse_count=8)
    assert v.numel() == 0
    g = lib.npu_sparse_lightning_indexer_grad_kl_loss(q, k, qi, ki, w, idx, smax, ssum)
    assert [t.shape for t in g] == [qi.shape, ki.shape, w.shape, (1,)]
    meta = lib.npu_sparse_attn_sharedkv_metadata(None, None, None, None, None, H, 1, 512, B, S, S, 0, 8, 4, 4, 3,
                                                 127, 0, "BSND", "BSND", True, True, torch.device(dev))
    assert meta.shape == (1024,) and meta.dtype == torch.int32
    Q = torch.empty(B, S, H, 512, dtype=torch.bfloat16, device=dev, requires_grad=True)
    ori = torch.empty(B, S, 1, 512, dtype=torch.bfloat16, device=dev, requires_grad=True)
    cmp = torch.empty(B, S // 4, 1, 512, dtype=torch.bfloat16, device=dev, requires_grad=True)
    sk = torch.empty(H, device=dev, requires_grad=True)
    o, lse = lib.npu_sparse_attn_sharedkv(Q, ori, cmp, idx, sk, meta, 0.1, 4)
    assert o.shape == Q.shape and lse.shape == (B, S, H, 1)
    o.sum().backward()
    assert Q.grad.shape == Q.shape and ori.grad.shape == ori.shape and cmp.grad.shape == cmp.shape
    assert sk.grad.shape == sk.shape


def test_host_tensors_are_refused_before_any_launch():
    """A host tensor handed to a kernel argument raises (the kernel would read a CPU address)."""
    from torchtitan_npu_simulator_amd import DSAError
    from torchtitan_npu_simulator_amd import _lib

    assert _lib.ptr(None) is None
    with pytest.raises(DSAError, match="passed to a GPU kernel"):
        _lib.ptr(torch.zeros(4))
    with pytest.raises(DSAError):
        ops._rope_args(torch.polar(torch.ones(4, 32), torch.zeros(4, 32)), 64, torch.device("cpu"))[0].data_ptr() \
            and _lib.ptr(ops._rope_args(torch.polar(torch.ones(4, 32), torch.zeros(4, 32)), 64,
                                        torch.device("cpu"))[0])


def test_host_ints_reads_a_device_tensor_once_per_version():
    """The cu_seqlens read-back cache: a hit needs the same tensor object and version, and
    the entry goes when the tensor is freed.  (A CPU tensor that reports is_cuda stands in
    for a device tensor.)"""
    import gc

    from torchtitan_npu_simulator_amd import _lib

    class Dev(torch.Tensor):
        @property
        def is_cuda(self):
            return True

    cu = torch.tensor([0, 100, 250], dtype=torch.int32).as_subclass(Dev)
    twin = torch.tensor([0, 100, 250], dtype=torch.int32).as_subclass(Dev)  # equal values, other object
    first = _lib.host_ints(cu)
    assert first == [0, 100, 250] and _lib.host_ints(cu) is first
    assert _lib.host_ints(twin) == first and _lib.host_ints(twin) is not first
    cu[2] = 260
    assert _lib.host_ints(cu) == [0, 100, 260]
    n = len(_lib._host_cache)
    del cu, twin
    gc.collect()
    assert len(_lib._host_cache) == n - 2


def test_band_rule_cuts_and_masks():
    """pre_tokens / next_tokens: whether a band removes keys the mode admits, and the index
    masking the KL op applies (band of row s: [a(s) - pre, a(s) + next], a(s) = s in
    sparse_mode 0 and s + q_offset in sparse_mode 3)."""
    from torchtitan_npu_simulator_amd.torch_npu_ops import _band_cuts, _band_mask_indices

    # the reference's defaults never cut at the configs' lengths
    assert not _band_cuts(3, 8192, 8192, 0, 65536, 65536)
    assert not _band_cuts(3, 4096, 8192, 4096, (1 << 63) - 1, (1 << 63) - 1)
    assert _band_cuts(3, 131072, 131072, 0, 65536, 65536)
    assert _band_cuts(3, 16, 16, 0, 4, 0) and _band_cuts(3, 16, 16, 0, 100, -1)
    assert not _band_cuts(0, 16, 16, 0, 15, 15) and _band_cuts(0, 16, 16, 0, 15, 14)
    idx = torch.tensor([[[0, 3, 5, -1], [1, 2, 6, 7]]], dtype=torch.int32)  # rows 0, 1
    m3 = _band_mask_indices(idx, 3, 6, 2, 0)  # a(s) = s + 6: rows see [4, 6] and [5, 7]
    assert m3.tolist() == [[[-1, -1, 5, -1], [-1, -1, 6, 7]]]
    m0 = _band_mask_indices(idx, 0, 0, 1, 1)  # a(s) = s: [-1, 1] and [0, 2]
    assert m0.tolist() == [[[0, -1, -1, -1], [1, 2, -1, -1]]]
