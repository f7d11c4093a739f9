"""Parity of the lightning indexer (dsa_indexer_fwd) and top-k (dsa_topk) HIP kernels.

Top-k is bit-exact: identical fp32 scores must give identical index sets (ties broken by
lower index, -0.0 == +0.0, NaN excluded).  Indexer scores are fp32 sums of exact
products (bf16 x bf16 or e4m3 x e4m3), so only the summation order differs from the
oracle: relative tolerance 1e-5 of the row's magnitude (5e-5 for fp8, whose per-token
scales are folded into the weights and the final sum with extra fp32 roundings).
"""

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _oracle_topk(scores, k, q_offset=0, cmp_ratio=1, index_offset=0):
    S, n = scores.shape[1], scores.shape[2]
    nv = np.array([O.valid_key_count(s, q_offset, cmp_ratio, n) for s in range(S)])
    ref = O.topk_select_numpy(scores[0].numpy(), k, nv)
    ref = np.where(ref >= 0, ref + index_offset, -1)
    return torch.from_numpy(ref).unsqueeze(0)


@pytest.mark.parametrize("S,n,k,q_offset,cmp_ratio", [(64, 64, 16, 0, 1), (300, 300, 64, 0, 1), (128, 512, 100, 384, 1),
                                                     (256, 64, 32, 0, 4), (40, 20000, 2048, 19960, 1)])
def test_topk_bit_exact_random(S, n, k, q_offset, cmp_ratio):
    g = torch.Generator().manual_seed(S + n + k)
    scores = torch.randn(1, S, n, generator=g)
    idx, vals = _ops().topk_select(scores.to(DEV), k, q_offset=q_offset, cmp_ratio=cmp_ratio, return_values=True)
    ref = _oracle_topk(scores, k, q_offset, cmp_ratio)
    assert torch.equal(idx.cpu(), ref)
    ref_vals = torch.where(ref >= 0, torch.gather(scores, -1, ref.clamp_min(0).long()), torch.tensor(float("-inf")))
    assert torch.equal(vals.cpu(), ref_vals)


def test_topk_ties_signed_zero_nan_inf():
    S, n, k = 96, 256, 40
    g = torch.Generator().manual_seed(3)
    scores = torch.randint(-3, 4, (1, S, n), generator=g).float()  # heavy ties
    scores[0, :, ::7] = -0.0
    scores[0, :, 3::11] = 0.0
    scores[0, 5:, 1::13] = float("nan")
    scores[0, 7:, 2::17] = float("inf")
    scores[0, 9:, 4::19] = float("-inf")
    idx, _ = _ops().topk_select(scores.to(DEV), k)
    assert torch.equal(idx.cpu(), _oracle_topk(scores, k))


def test_topk_all_equal_and_short_rows():
    S, n, k = 50, 50, 8
    scores = torch.zeros(1, S, n)
    idx, _ = _ops().topk_select(scores.to(DEV), k)
    ref = _oracle_topk(scores, k)
    assert torch.equal(idx.cpu(), ref)
    # rows s < k have s+1 candidates: all chosen, rest -1
    assert torch.all(idx.cpu()[0, 0, 1:] == -1) and idx.cpu()[0, 0, 0] == 0


def _topk_check(scores, k, **kw):
    idx, vals = _ops().topk_select(scores.to(DEV), k, return_values=True, **kw)
    ref = _oracle_topk(scores, k, kw.get("q_offset", 0), kw.get("cmp_ratio", 1), kw.get("index_offset", 0))
    assert torch.equal(idx.cpu(), ref)
    src = torch.where(ref >= 0, ref - kw.get("index_offset", 0), 0).long()
    ref_vals = torch.where(ref >= 0, torch.gather(scores, -1, src), torch.tensor(float("-inf")))
    assert torch.equal(vals.cpu().view(torch.int32), ref_vals.view(torch.int32))  # bit for bit, -0.0 kept


@pytest.mark.parametrize("n", [8191, 8192, 8193, 16383, 16384, 16385, 24577, 40003])
def test_topk_segment_boundaries(n):
    # rows of one register-resident segment (<= 8192 / 16384 scores) and rows re-read in
    # segments, with lengths that are not multiples of 4 (scalar tail chunk)
    S, k = 6, 2048
    g = torch.Generator().manual_seed(n)
    scores = torch.randn(1, S, n, generator=g)
    _topk_check(scores, k, q_offset=n - S)


def test_topk_unaligned_row_stride():
    # a column slice: rows start at 4-byte but not 16-byte aligned offsets (scalar loads)
    S, n, k = 40, 3001, 300
    g = torch.Generator().manual_seed(11)
    wide = torch.randn(1, S, n + 2, generator=g)  # row stride 3003 floats
    scores = wide[:, :, :n]
    idx, _ = _ops().topk_select(wide.to(DEV)[:, :, :n], k, q_offset=n - S)
    assert torch.equal(idx.cpu(), _oracle_topk(scores.contiguous(), k, q_offset=n - S))


def test_topk_clustered_keys_need_every_pass():
    # scores 1 + m * 2^-23 with m < 2^22 (one exponent, 22 significant key bits) and runs of
    # equal values: the threshold needs all refinement passes and then the tie rule
    S, n, k = 24, 6000, 1000
    g = torch.Generator().manual_seed(12)
    m = torch.randint(0, 1 << 22, (1, S, n), generator=g)
    m[:, :, ::5] = m[:, :, :1]  # many copies of each row's first value
    scores = 1.0 + m.double() * 2.0 ** -23
    _topk_check(scores.float(), k, q_offset=n - S)


def test_topk_outliers_and_infinities():
    S, n, k = 16, 9000, 2048
    g = torch.Generator().manual_seed(13)
    scores = torch.full((1, S, n), 0.5)
    scores[:, :, torch.randint(0, n, (50,), generator=g)] = torch.randn(50, generator=g) * 1e30
    scores[:, 3:, 7::97] = float("inf")
    scores[:, 5:, 9::89] = float("-inf")
    scores[:, 8:, 11::83] = float("nan")
    scores[:, 10:, 13::71] = -0.0
    _topk_check(scores, k, q_offset=n - S)


def test_topk_index_offset():
    S, n, k = 32, 32, 8
    scores = torch.randn(1, S, n, generator=torch.Generator().manual_seed(4))
    idx, _ = _ops().topk_select(scores.to(DEV), k, index_offset=100)
    assert torch.equal(idx.cpu(), _oracle_topk(scores, k, index_offset=100))


@pytest.mark.parametrize("S,H,D,q_offset,cmp_ratio", [(256, 64, 128, 0, 1), (200, 32, 128, 56, 1), (512, 4, 64, 0, 1),
                                                     (128, 16, 128, 0, 4)])
def test_indexer_bf16_parity(S, H, D, q_offset, cmp_ratio):
    g = torch.Generator().manual_seed(S + H)
    s_k = (S + q_offset) // cmp_ratio
    q = torch.randn(1, S, H, D, generator=g).bfloat16()
    k = torch.randn(1, s_k, D, generator=g).bfloat16()
    w = torch.rand(1, S, H, generator=g) * H ** -0.5 * D ** -0.5
    got = _ops().indexer_scores(q.to(DEV), k.to(DEV), w.to(DEV), q_offset=q_offset, cmp_ratio=cmp_ratio).cpu()
    ref = O.indexer_scores(q, k, w, q_offset=q_offset, cmp_ratio=cmp_ratio, dtype=torch.float64)
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    err = (got.double() - ref).abs().masked_fill(~fin, 0).amax(-1)
    mag = ref.abs().masked_fill(~fin, 0).amax(-1).clamp_min(1e-6)
    assert float((err / mag).max()) <= 1e-5


def test_indexer_fp8_quantise_dequantise_parity():
    S, H, D = 256, 64, 128
    g = torch.Generator().manual_seed(21)
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, S, D, generator=g)
    w = torch.rand(1, S, H, generator=g) * H ** -0.5 * D ** -0.5
    q8, qs = O.quantize_e4m3_per_row(q)
    k8, ks = O.quantize_e4m3_per_row(k)
    got = _ops().indexer_scores(q8.to(DEV), k8.to(DEV), w.to(DEV), q_scale=qs.to(DEV), k_scale=ks.to(DEV)).cpu()
    qd = q8.double() * qs.double().unsqueeze(-1)
    kd = k8.double() * ks.double().unsqueeze(-1)
    ref = O.indexer_scores(qd, kd, w.double(), dtype=torch.float64)
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    err = (got.double() - ref).abs().masked_fill(~fin, 0).amax(-1)
    mag = ref.abs().masked_fill(~fin, 0).amax(-1).clamp_min(1e-6)
    # the per-token scales are folded into w and the final sum in fp32: a few extra roundings
    assert float((err / mag).max()) <= 5e-5


@pytest.mark.parametrize("S,s_k,q_offset,cmp_ratio,signed_w,split", [
    (256, 256, 0, 1, False, True), (256, 256, 0, 1, False, False), (203, 1400, 1197, 1, True, True),
    (96, 600, 2300, 4, True, True), (1, 64, 63, 1, False, True), (1030, 1030, 0, 1, True, True)])
def test_indexer_fp8_linear_split_parity(S, s_k, q_offset, cmp_ratio, signed_w, split):
    """fp8 H_I=64 scores through the linear split sum_h c|x|/2 + u.k (u as four fp8 pieces from
    the pre-pass) and through the relu form, against the fp64 oracle of the dequantised
    operands: 5e-5 of the row magnitude; mixed-sign head weights make the |x| and u.k halves
    cancel, ragged S leaves a partial query pair, q_offset / cmp_ratio move the frontier."""
    H, D = 64, 128
    g = torch.Generator().manual_seed(S * 7 + s_k)
    n_k = s_k
    q = torch.randn(1, S, H, D, generator=g)
    k = torch.randn(1, n_k, D, generator=g) * 3.0
    w = (torch.randn(1, S, H, generator=g) if signed_w else torch.rand(1, S, H, generator=g)) * H ** -0.5 * D ** -0.5
    q8, qs = O.quantize_e4m3_per_row(q)
    k8, ks = O.quantize_e4m3_per_row(k)
    got = _ops().indexer_scores(q8.to(DEV), k8.to(DEV), w.to(DEV), q_scale=qs.to(DEV), k_scale=ks.to(DEV),
                                q_offset=q_offset, cmp_ratio=cmp_ratio, linear_split=split).cpu()
    qd = q8.double() * qs.double().unsqueeze(-1)
    kd = k8.double() * ks.double().unsqueeze(-1)
    ref = O.indexer_scores(qd, kd, w.double(), q_offset=q_offset, cmp_ratio=cmp_ratio, dtype=torch.float64)
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    err = (got.double() - ref).abs().masked_fill(~fin, 0).amax(-1)
    mag = ref.abs().masked_fill(~fin, 0).amax(-1).clamp_min(1e-6)
    assert float((err / mag).max()) <= 5e-5


def test_lightning_indexer_op_end_to_end():
    """npu_lightning_indexer == oracle top-k applied to the GPU's own fp32 scores (bit-exact)."""
    S, H, D, K = 300, 64, 128, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, S, H, D, generator=g).bfloat16()
    k = torch.randn(1, S, 1, D, generator=g).bfloat16()
    w = torch.rand(1, S, H, generator=g) * H ** -0.5 * D ** -0.5
    ops = _ops()
    idx, vals = ops.npu_lightning_indexer(q.to(DEV), k.to(DEV), w.to(DEV), sparse_count=K, sparse_mode=3,
                                          return_value=True)
    scores = ops.indexer_scores(q.to(DEV), k.to(DEV), w.to(DEV)).cpu()
    assert idx.shape == (1, S, 1, K)
    assert torch.equal(idx[:, :, 0].cpu(), _oracle_topk(scores, K))
    # sparse_values in the query's dtype, as the binding allocates them (binding.cpp:29)
    assert vals.shape == (1, S, 1, K) and vals.dtype == torch.bfloat16
    sel = idx[:, :, 0].cpu()
    ref_vals = torch.gather(scores, -1, sel.clamp_min(0).long()).masked_fill(sel < 0, float("-inf"))
    assert torch.equal(vals[:, :, 0].cpu(), ref_vals.to(torch.bfloat16))


def _long_rows_case(kind, S, n, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "normal":
        return torch.randn(1, S, n, generator=g)
    if kind == "rising":  # scores grow along the row: the sample must span it, not only its start
        return torch.randn(1, S, n, generator=g) + torch.linspace(0, 6, n)
    if kind == "clustered":  # one exponent, 22 significant key bits, runs of equal values
        m = torch.randint(0, 1 << 22, (1, S, n), generator=g)
        m[:, :, ::5] = m[:, :, :1]
        return (1.0 + m.double() * 2.0 ** -23).float()
    if kind == "plateau":  # a constant row with a few outliers: the list would overflow -> fallback
        x = torch.full((1, S, n), 0.5)
        x[:, :, torch.randint(0, n, (50,), generator=g)] = torch.randn(50, generator=g) * 1e30
        return x
    if kind == "special":  # ties, signed zeros, NaN, infinities
        x = torch.randint(-3, 4, (1, S, n), generator=g).float()
        x[0, :, ::7] = -0.0
        x[0, 1:, 1::13] = float("nan")
        x[0, 2:, 2::17] = float("inf")
        x[0, 3:, 4::19] = float("-inf")
        return x
    raise ValueError(kind)


@pytest.mark.parametrize("kind,n,k", [("normal", 40003, 2048), ("normal", 131072, 2048), ("rising", 65536, 2048),
                                      ("clustered", 50000, 1000), ("plateau", 30000, 2048), ("special", 20000, 2048),
                                      ("normal", 40000, 4096), ("normal", 17000, 64)])
@pytest.mark.parametrize("candidates", [True, False])
def test_topk_long_rows_candidate_lists(kind, n, k, candidates):
    """Rows longer than 16384 keys: the candidate-list path (one read of the row, selection
    over the keys at or above a sampled threshold, fallback to the multi-pass selection when
    the list would miss a key or overflow) and the multi-pass path, bit-exact against the
    oracle; causal rows of several lengths (the last rows the longest), values bit for bit."""
    S = 5
    scores = _long_rows_case(kind, S, n, seed=n + k)
    q_off = n - S - 2 * 4096  # rows of n - 8196 .. n - 8192 valid keys (more than the 4096-entry lists)
    idx, vals = _ops().topk_select(scores.to(DEV), k, q_offset=q_off, return_values=True, candidates=candidates)
    ref = _oracle_topk(scores, k, q_off)
    assert torch.equal(idx.cpu(), ref)
    ref_vals = torch.where(ref >= 0, torch.gather(scores, -1, ref.clamp_min(0).long()), torch.tensor(float("-inf")))
    assert torch.equal(vals.cpu().view(torch.int32), ref_vals.view(torch.int32))
