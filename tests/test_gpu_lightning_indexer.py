"""The fused lightning indexer (dsa_lightning_indexer) against its two halves.

dsa_lightning_indexer leaves the score spans past every causal frontier unwritten and its
top-k reads only each row's valid prefix; the selection must equal dsa_indexer_fwd_ws +
dsa_topk on the fully written score matrix bit for bit (indices and values), for fp8 with
the linear split (H_I = 64) and bf16 (H_I = 16), batches > 1, compressed keys, a causal
offset, rows with fewer valid keys than k, and workspaces small enough to force the
batch-by-batch row chunks.  The selection on those identical scores is itself pinned
against the oracle by the top-k tests.
"""

import pytest
import torch

from torchtitan_npu_simulator_amd import torch_npu_ops as ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(B, S, s_k, H, fp8, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, S, H, 128, generator=g)
    k = torch.randn(B, s_k, 128, generator=g)
    w = torch.randn(B, S, H, generator=g) * H ** -0.5
    if fp8:
        q8, qs = ops.quantize_fp8_per_row(q.bfloat16().to(DEV))
        k8, ks = ops.quantize_fp8_per_row(k.bfloat16().to(DEV))
        return q8, k8, w.to(DEV), qs, ks
    return q.bfloat16().to(DEV), k.bfloat16().to(DEV), w.to(DEV), None, None


CASES = [
    # B, S, s_k, H, fp8, K, q_offset, cmp_ratio, budget (bytes; None = default)
    (1, 1024, 1024, 64, True, 256, 0, 1, None),
    (2, 700, 700, 64, True, 128, 0, 1, None),
    (2, 700, 700, 64, True, 128, 0, 1, 300 * 700 * 4),   # batch by batch, 300-row chunks
    (2, 513, 777, 16, False, 64, 264, 1, 100 * 777 * 4),  # causal offset, bf16, 100-row chunks
    (1, 2048, 512, 64, True, 96, 0, 4, None),             # compressed keys (r = 4)
    (3, 300, 300, 16, False, 400, 0, 1, None),            # k > every row's valid count
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}-S{c[1]}-sk{c[2]}-H{c[3]}-{'fp8' if c[4] else 'bf16'}-r{c[7]}"
                                             f"{'-chunked' if c[8] else ''}" for c in CASES])
def test_fused_indexer_equals_scores_plus_topk(case, monkeypatch):
    B, S, s_k, H, fp8, K, q_off, r, budget = case
    q, k, w, qs, ks = _inputs(B, S, s_k, H, fp8, seed=S + s_k)
    if budget is not None:
        monkeypatch.setattr(ops, "_SCORE_BUDGET_BYTES", budget)
    idx, vals = ops.lightning_indexer(q, k, w, K, query_scale=qs, key_scale=ks, q_offset=q_off, cmp_ratio=r,
                                      index_offset=7, return_value=True)
    sc = ops.indexer_scores(q, k, w, q_scale=qs, k_scale=ks, q_offset=q_off, cmp_ratio=r)
    ref_i, ref_v = ops.topk_select(sc, K, q_offset=q_off, cmp_ratio=r, index_offset=7, return_values=True)
    torch.cuda.synchronize()
    assert torch.equal(idx.cpu(), ref_i.cpu())
    assert torch.equal(vals.cpu(), ref_v.cpu())
    # every row holds min(k, n_valid) indices
    nv = torch.clamp((torch.arange(S) + q_off + 1) // r, max=s_k)
    cnt = (idx.cpu() >= 0).sum(-1)
    assert torch.equal(cnt, torch.minimum(nv, torch.tensor(K)).expand(B, S))


def test_npu_lightning_indexer_op_uses_the_fused_call():
    q, k, w, qs, ks = _inputs(2, 256, 256, 64, True, seed=3)
    idx, vals = ops.npu_lightning_indexer(q, k.unsqueeze(2), w, sparse_count=64, sparse_mode=3, return_value=True,
                                          query_scale=qs, key_scale=ks)
    sc = ops.indexer_scores(q, k, w, q_scale=qs, k_scale=ks, q_offset=0)
    ref_i, ref_v = ops.topk_select(sc, 64, q_offset=0, return_values=True)
    torch.cuda.synchronize()
    assert torch.equal(idx[:, :, 0].cpu(), ref_i.cpu())
    assert vals.dtype == torch.bfloat16 and torch.equal(vals[:, :, 0].cpu(), ref_v.bfloat16().cpu())
