"""The packed-sequence (global TND) DeepSeek-V4 branch on the GPU.

A packed batch of sequences of different lengths runs through ``npu_sparse_flash_mla``
(the reference's A5 wrapper, converters/kernels/npu_smla.py:842-917, here on the gathered-
attention kernels) and is checked against the oracle's ``sparse_attn_sink`` applied to each
sequence on its own in fp64 (bf16 within 2e-2, fp32 within 1e-5): the output, the LSE, the
gradients to query, ori_kv, cmp_kv and the sinks, and for ratio 4 the indexer loss's
gradients to q_indexer, k_indexer and weights (oracle: ``v4_selected_attn_dist`` target and
``indexer_kl_from_mass``, scaled by LOSS_SCALE * softmax_scale / T as the reference's
backward does, :600-608).  The binding-level ops in layout TND and the packed indexer are
checked against the same oracle / against the per-sequence indexer.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _masks(lengths, ratio):
    from torchtitan_npu_simulator_amd import tnd

    cu_q = [0]
    for n in lengths:
        cu_q.append(cu_q[-1] + n)
    n_cmp = [n // ratio for n in lengths] if ratio > 1 else [0] * len(lengths)
    cu_c = [0]
    for n in n_cmp:
        cu_c.append(cu_c[-1] + n)
    t = lambda v: torch.tensor(v, dtype=torch.int32, device=DEV)  # noqa: E731
    res = [n - ratio * c for n, c in zip(lengths, n_cmp)]
    return tnd.DeepSeekV4SMLAAttentionMasks(
        cu_seqlens_q=t(cu_q), cu_seqlens_ori_kv=t(cu_q), cu_seqlens_cmp_kv={ratio: t(cu_c)},
        cmp_residual_k={ratio: t(res)}, block_starts_by_ratio={}, max_seqlen_q=max(lengths),
        max_seqlen_cmp_kv={ratio: max(n_cmp)}, batch_size=len(lengths), seq_len=sum(lengths), cache_id=7), cu_q, cu_c, n_cmp


def _case(lengths, ratio, H, D, K, dtype, seed, HI=64, DI=128):
    g = torch.Generator().manual_seed(seed)
    T = sum(lengths)
    n_cmp = [n // ratio for n in lengths] if ratio > 1 else [0] * len(lengths)
    q = torch.randn(T, H, D, generator=g).to(dtype)
    ori = torch.randn(T, D, generator=g).to(dtype)
    cmp = torch.randn(sum(n_cmp), D, generator=g).to(dtype) if ratio > 1 else None
    sink = torch.randn(H, generator=g)
    dout = torch.randn(T, H, D, generator=g).to(dtype)
    local = None
    if ratio == 4:
        rows = []
        for n, nc in zip(lengths, n_cmp):
            r = torch.full((n, K), -1, dtype=torch.int32)
            for p in range(n):
                vis = min(nc, (p + 1) // ratio)
                c = min(K, vis)
                if c:
                    r[p, :c] = torch.sort(torch.randperm(vis, generator=g)[:c]).values.int()
            rows.append(r)
        local = torch.cat(rows)
    qi = torch.randn(T, HI, DI, generator=g).bfloat16()
    ki = torch.randn(sum(n_cmp), DI, generator=g).bfloat16() if ratio > 1 else None
    w = torch.rand(T, HI, generator=g) * HI ** -0.5 * DI ** -0.5
    return q, ori, cmp, sink, dout, local, qi, ki, w


def _oracle(lengths, ratio, q, ori, cmp, sink, dout, local, scale, window):
    """Per-sequence fp64 sink attention; returns out, lse and the gradients (packed)."""
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    n_cmp = [n // ratio for n in lengths] if ratio > 1 else [0] * len(lengths)
    cu_c = [0]
    for n in n_cmp:
        cu_c.append(cu_c[-1] + n)
    oq = q.double().requires_grad_(True)
    oori = ori.double().requires_grad_(True)
    ocmp = cmp.double().requires_grad_(True) if cmp is not None else None
    osk = sink.double().requires_grad_(True)
    outs, lses = [], []
    for i, n in enumerate(lengths):
        qs = oq[cu[i]:cu[i + 1]].unsqueeze(0)
        kv = oori[cu[i]:cu[i + 1]]
        ci = None
        if ratio > 1:
            kv = torch.cat([kv, ocmp[cu_c[i]:cu_c[i + 1]]], dim=0)
            if ratio == 4:
                li = local[cu[i]:cu[i + 1]]
                ci = torch.where(li < 0, li, li + n).unsqueeze(0)
        idx = O.v4_attn_indices(1, n, window, ratio, n, cmp_idxs=ci)
        o, lse = O.sparse_attn_sink(qs, kv.unsqueeze(0), osk, idx, scale)
        outs.append(o[0])
        lses.append(lse[0])
    out = torch.cat(outs)
    out.backward(dout.double())
    return out.detach(), torch.cat(lses).detach(), oq.grad, oori.grad, (ocmp.grad if ocmp is not None else None), \
        osk.grad


@pytest.mark.parametrize("ratio,dtype,D,H,window,tol", [
    (4, torch.bfloat16, 512, 16, 128, 2e-2),
    (128, torch.bfloat16, 512, 16, 128, 2e-2),
    (1, torch.bfloat16, 512, 16, 128, 2e-2),
    (4, torch.float32, 64, 4, 128, 1e-5),
])
def test_packed_sparse_flash_mla_matches_oracle(ratio, dtype, D, H, window, tol):
    from torchtitan_npu_simulator_amd.converters import dsa_indexer_loss
    from torchtitan_npu_simulator_amd.converters import npu_smla as smla

    lengths = [96, 300, 7, 161] if ratio != 128 else [300, 520, 129]
    K = 16
    masks, cu_q, cu_c, n_cmp = _masks(lengths, ratio)
    q, ori, cmp, sink, dout, local, qi, ki, w = _case(lengths, ratio, H, D, K, dtype, seed=ratio + D)
    scale = D ** -0.5
    args = SimpleNamespace(head_dim=D, index_topk=K, index_n_heads=64, index_head_dim=128)
    cache = smla.SMLAMetadataCache(args)
    leaves = [t.to(DEV).requires_grad_(True) for t in (q, ori)]
    lc = cmp.to(DEV).requires_grad_(True) if cmp is not None else None
    sk = sink.to(DEV).requires_grad_(True)
    li = [t.to(DEV).requires_grad_(True) for t in (qi, ki, w)] if ratio == 4 else [None, None, None]
    out = smla.npu_sparse_flash_mla(leaves[0], leaves[1], lc, None if local is None else local.to(DEV), sk, scale,
                                    ratio, ori_win_left=window - 1, indexer_q=li[0], indexer_k=li[1], weights=li[2],
                                    attention_masks=masks, metadata_cache=cache)
    out.backward(dout.to(DEV))
    ref, ref_lse, rdq, rdori, rdcmp, rdsk = _oracle(lengths, ratio, q, ori, cmp, sink, dout, local, scale, window)
    assert out.shape == q.shape
    assert rel_err(out.detach(), ref) <= tol, rel_err(out.detach(), ref)
    assert rel_err(leaves[0].grad, rdq) <= tol, rel_err(leaves[0].grad, rdq)
    assert rel_err(leaves[1].grad, rdori) <= tol, rel_err(leaves[1].grad, rdori)
    if ratio > 1:
        assert rel_err(lc.grad, rdcmp) <= tol, rel_err(lc.grad, rdcmp)
    assert rel_err(sk.grad, rdsk) <= tol, (sk.grad, rdsk)
    # the LSE the forward saves for backward
    meta = smla.SparseFlashMLA.sparse_attn_metadata(cache, masks, ratio, H)
    from torchtitan_npu_simulator_amd import smla_ops

    _, lse = smla_ops.sparse_flash_mla(q.to(DEV), ori_kv=ori.to(DEV).unsqueeze(1),
                                       cmp_kv=None if cmp is None else cmp.to(DEV).unsqueeze(1),
                                       cmp_sparse_indices=None if local is None else local.to(DEV).unsqueeze(1),
                                       cu_seqlens_q=masks.cu_seqlens_q, cu_seqlens_ori_kv=masks.cu_seqlens_ori_kv,
                                       cu_seqlens_cmp_kv=masks.cu_seqlens_cmp_kv[ratio],
                                       cmp_residual_kv=masks.cmp_residual_k[ratio], sinks=sink.to(DEV), metadata=meta,
                                       softmax_scale=scale, cmp_ratio=ratio, ori_win_left=window - 1)
    assert lse.shape == (q.shape[0], H, 1)
    assert (lse.squeeze(-1).double().cpu() - ref_lse).abs().max() <= 5 * tol

    if ratio == 4:
        # indexer loss gradients, per sequence against the oracle
        T = sum(lengths)
        gs = float(dsa_indexer_loss.LOSS_SCALE) * scale / T
        rq, rk, rw = [], [], []
        for i, n in enumerate(lengths):
            s0, s1, c0, c1 = cu_q[i], cu_q[i + 1], cu_c[i], cu_c[i + 1]
            lcl = local[s0:s1].unsqueeze(0)
            dist = O.v4_selected_attn_dist(q[s0:s1].unsqueeze(0), ori[s0:s1].unsqueeze(0),
                                           cmp[c0:c1].unsqueeze(0), sink, lcl, scale, window)
            dq_i, dk_i, dw_i, _ = O.indexer_kl_from_mass(qi[s0:s1].unsqueeze(0), ki[c0:c1].unsqueeze(0),
                                                         w[s0:s1].unsqueeze(0), lcl, dist, q_offset=1 << 40,
                                                         loss_scale=1.0, eps=1e-10)
            rq.append(dq_i[0])
            rk.append(dk_i[0])
            rw.append(dw_i[0])
        rq, rk, rw = torch.cat(rq) * gs, torch.cat(rk) * gs, torch.cat(rw) * gs
        assert rel_err(li[0].grad, rq) <= 2e-2, rel_err(li[0].grad, rq)
        assert rel_err(li[1].grad, rk) <= 2e-2, rel_err(li[1].grad, rk)
        assert rel_err(li[2].grad, rw) <= 2e-2, rel_err(li[2].grad, rw)


def test_packed_binding_ops_match_oracle():
    """npu_sparse_attn_sharedkv / _grad with layout TND (binding.cpp:30-88 argument lists)."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    lengths, ratio, H, D, K, window = [130, 64, 211], 4, 16, 512, 16, 128
    masks, cu_q, cu_c, _ = _masks(lengths, ratio)
    q, ori, cmp, sink, dout, local, *_ = _case(lengths, ratio, H, D, K, torch.bfloat16, seed=3)
    scale = D ** -0.5
    out, lse = ops.npu_sparse_attn_sharedkv(
        q.to(DEV), ori.to(DEV).unsqueeze(1), cmp.to(DEV).unsqueeze(1), None, local.to(DEV).unsqueeze(1),
        cu_seqlens_q=masks.cu_seqlens_q, cu_seqlens_ori_kv=masks.cu_seqlens_ori_kv,
        cu_seqlens_cmp_kv=masks.cu_seqlens_cmp_kv[ratio], sinks=sink.to(DEV), softmax_scale=scale, cmp_ratio=ratio,
        ori_win_left=window - 1, layout_q="TND", layout_kv="TND")
    dq, d_ori, d_cmp, d_sink = ops.npu_sparse_attn_sharedkv_grad(
        q.to(DEV), ori.to(DEV).unsqueeze(1), cmp.to(DEV).unsqueeze(1), dout.to(DEV), out, lse, None,
        local.to(DEV).unsqueeze(1), masks.cu_seqlens_q, masks.cu_seqlens_ori_kv, masks.cu_seqlens_cmp_kv[ratio],
        sink.to(DEV), scale, ratio, ori_win_left=window - 1, layout="TND")
    ref, ref_lse, rdq, rdori, rdcmp, rdsk = _oracle(lengths, ratio, q, ori, cmp, sink, dout, local, scale, window)
    assert out.shape == q.shape and lse.shape == (q.shape[0], H, 1)
    assert rel_err(out, ref) <= 2e-2
    assert (lse.squeeze(-1).double().cpu() - ref_lse).abs().max() <= 0.1
    assert d_ori.shape == (sum(lengths), 1, D) and d_cmp.shape == (cmp.shape[0], 1, D)
    assert rel_err(dq, rdq) <= 2e-2
    assert rel_err(d_ori.squeeze(1), rdori) <= 2e-2
    assert rel_err(d_cmp.squeeze(1), rdcmp) <= 2e-2
    assert rel_err(d_sink, rdsk) <= 2e-2


def test_packed_lightning_indexer_module():
    """NpuLiComputeSMLA: [T,1,K] sequence-local indices equal to the per-sequence indexer's."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops
    from torchtitan_npu_simulator_amd.converters import npu_smla as smla

    lengths, ratio, K = [200, 75, 333], 4, 32
    masks, cu_q, cu_c, _ = _masks(lengths, ratio)
    _, _, _, _, _, _, qi, ki, w = _case(lengths, ratio, 4, 64, K, torch.bfloat16, seed=11)
    args = SimpleNamespace(head_dim=512, index_topk=K, index_n_heads=64, index_head_dim=128)
    cache = smla.SMLAMetadataCache(args)
    mod = smla.NpuLiComputeSMLA(torch.nn.Module(), cache)
    mod.index_topk, mod.ratio = K, ratio
    idx, vals = mod(qi.to(DEV), ki.to(DEV), w.to(DEV), max(lengths), 0, masks)
    assert idx.shape == (sum(lengths), 1, K) and vals.shape == (sum(lengths), 1, K)
    ref_idx, _ = ops.lightning_indexer_varlen(qi.to(DEV), ki.to(DEV), w.to(DEV).bfloat16(), cu_q, cu_c, K,
                                              cmp_ratio=ratio, cmp_residual_k=masks.cmp_residual_k[ratio])
    assert torch.equal(idx.squeeze(1).cpu(), ref_idx.cpu())
    # every selected row is visible to its query
    for i, n in enumerate(lengths):
        rows = idx[cu_q[i]:cu_q[i + 1], 0].cpu().long()
        pos = torch.arange(n).view(n, 1)
        ok = (rows < 0) | (rows < (pos + 1) // ratio)
        assert bool(ok.all())


def test_packed_kl_loss_grad_returns_indexer_softmax():
    """softmax_out of ``sparse_lightning_indexer_kl_loss_grad`` (reference npu_smla.py:584-602):
    per row, the softmax of the indexer scores over the row's usable compressed slots (0 at
    the others), against the oracle's scores gathered at the same slots; the logged loss the
    converter builds from it (``_compute_li_loss``) equals the per-row losses the kernel
    returns, mean over rows."""
    from torchtitan_npu_simulator_amd import smla_ops
    from torchtitan_npu_simulator_amd.converters.npu_smla import _compute_li_loss

    ratio, K = 4, 16
    lengths = [96, 300, 7, 161]
    masks, cu_q, cu_c, n_cmp = _masks(lengths, ratio)
    _, _, _, _, _, local, qi, ki, w = _case(lengths, ratio, 16, 512, K, torch.bfloat16, seed=5)
    T = sum(lengths)
    g = torch.Generator().manual_seed(9)
    l1 = torch.rand(T, K, generator=g) * (local >= 0)
    l1[3] = 0.0  # a row with no teacher mass
    dq, dk, dw, sm, loss_rows = smla_ops.sparse_lightning_indexer_kl_loss_grad(
        q=qi.to(DEV), k=ki.to(DEV).unsqueeze(1), w=w.to(DEV), sparse_indices=local.to(DEV),
        attn_softmax_l1_norm=l1.to(DEV), cmp_residual_k=masks.cmp_residual_k[ratio], cu_seqlens_q=masks.cu_seqlens_q,
        cu_seqlens_k=masks.cu_seqlens_cmp_kv[ratio], cmp_ratio=ratio, eps=1e-10, return_loss_rows=True)
    sm = sm.cpu()
    assert sm.shape == (T, K)
    for i, n in enumerate(lengths):
        s0, s1, c0, c1 = cu_q[i], cu_q[i + 1], cu_c[i], cu_c[i + 1]
        if c1 == c0:
            assert float(sm[s0:s1].abs().max()) == 0.0
            continue
        sc = O.indexer_scores(qi[s0:s1].unsqueeze(0), ki[c0:c1].unsqueeze(0), w[s0:s1].unsqueeze(0),
                              cmp_ratio=ratio)[0].double()
        lcl = local[s0:s1].long()
        ok = lcl >= 0
        sel = torch.gather(sc, 1, lcl.clamp_min(0)).masked_fill(~ok, float("-inf"))
        ref = torch.softmax(sel, dim=-1).nan_to_num(0.0)  # rows with no usable slot: all 0
        assert (sm[s0:s1].double() - ref).abs().max() <= 1e-5
        assert float(sm[s0:s1][~ok].abs().max() if (~ok).any() else 0.0) == 0.0
    logged = _compute_li_loss(sm.to(DEV), l1.to(DEV), 1.0)
    assert abs(float(logged) - float(loss_rows.sum()) / T) <= 1e-4 * abs(float(loss_rows.sum()) / T) + 1e-7
