"""Packed varlen ("TND") entry points on the GPU.

A packed batch must give, for every sequence, exactly what the fixed-length entry points
give on that sequence alone (bit-exact: the same kernels run on the same slices with the
sequence's own causal offset; the key-gradient sums dKV / dk_idx only to 1e-6, since a
key whose contributions span several reduction segments adds them with fp32 atomics in
no fixed order), and the per-sequence oracle at the contract tolerance
(bf16 2e-2; top-k bit-exact on identical scores; compressor fp32 1e-5).  Batches mix an
empty sequence, a single-token one and lengths that are not multiples of any tile.
"""

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BF16_TOL = 2e-2


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _cu(lens):
    return [0] + list(np.cumsum(lens).tolist())


def _local_indices(lens_q, lens_k, K, seed, holes=0.1):
    """Sequence-local causal indices [T,K] (bottom-right aligned), ascending, -1 padded."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    for lq, lk in zip(lens_q, lens_k):
        off = max(0, lk - lq)
        for s in range(lq):
            lim = min(s + off + 1, lk)
            row = torch.full((K,), -1, dtype=torch.int32)
            c = min(K, lim)
            if c > 0:
                row[:c] = torch.sort(torch.randperm(lim, generator=g)[:c]).values.to(torch.int32)
                row[torch.rand(K, generator=g) < holes] = -1
            rows.append(row)
    return torch.stack(rows) if rows else torch.zeros(0, K, dtype=torch.int32)


def _attn_inputs(T, T_kv, H, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, H, 576, generator=g).to(torch.bfloat16)
    kv = torch.randn(T_kv, 576, generator=g).to(torch.bfloat16)
    dout = torch.randn(T, H, 512, generator=g).to(torch.bfloat16)
    return q, kv, dout, 576 ** -0.5


# ----- indexer + top-k -----
@pytest.mark.parametrize("fp8", [False, True])
def test_indexer_varlen_equals_per_sequence(fp8):
    ops = _ops()
    lens = [37, 0, 130, 1, 200]
    T, H, D, K = sum(lens), 64, 128, 48
    g = torch.Generator().manual_seed(5)
    qi = torch.randn(T, H, D, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(T, D, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(T, H, generator=g) * 0.01).to(DEV)
    qs = ks = None
    if fp8:
        qi, qs = ops.quantize_fp8_per_row(qi)
        ki, ks = ops.quantize_fp8_per_row(ki)
    cu = _cu(lens)
    idx, vals = ops.lightning_indexer_varlen(qi, ki, w, cu, cu, K, return_value=True, query_scale=qs, key_scale=ks)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        if a == b:
            continue
        ref_i, ref_v = ops.npu_lightning_indexer(qi[a:b].unsqueeze(0), ki[a:b].unsqueeze(0), w[a:b].unsqueeze(0),
                                                 sparse_count=K, sparse_mode=3, return_value=True,
                                                 query_scale=None if qs is None else qs[a:b].unsqueeze(0),
                                                 key_scale=None if ks is None else ks[a:b].unsqueeze(0))
        assert torch.equal(idx[a:b].cpu(), ref_i[0, :, 0].cpu()), f"sequence {i}"
        # the op returns sparse_values in the query's dtype (bf16 for fp8 queries)
        assert torch.equal(vals[a:b].to(ref_v.dtype).cpu(), ref_v[0, :, 0].cpu()), f"sequence {i}"
        # the oracle's selection on the same fp32 scores
        sc = ops.indexer_scores(qi[a:b].unsqueeze(0), ki[a:b].unsqueeze(0), w[a:b].unsqueeze(0),
                                q_scale=None if qs is None else qs[a:b].unsqueeze(0),
                                k_scale=None if ks is None else ks[a:b].unsqueeze(0)).cpu()
        nv = np.array([O.valid_key_count(s, 0, 1, b - a) for s in range(b - a)])
        ref = torch.from_numpy(O.topk_select_numpy(sc[0].numpy(), K, nv))
        assert torch.equal(idx[a:b].cpu().long(), ref.long()), f"sequence {i}"


def test_indexer_varlen_compressed_keys_with_residual():
    """V4 compressed keys: sequence i has len_q queries and len_q // 4 keys; the residual
    tokens past the last whole block keep the causal alignment at q_offset 0."""
    ops = _ops()
    lens_q = [37, 130, 3]
    r = 4
    lens_k = [n // r for n in lens_q]
    res = [n - r * k for n, k in zip(lens_q, lens_k)]
    H, D, K = 32, 128, 16
    g = torch.Generator().manual_seed(9)
    qi = torch.randn(sum(lens_q), H, D, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(sum(lens_k), D, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(sum(lens_q), H, generator=g) * 0.01).to(DEV)
    cq, ck = _cu(lens_q), _cu(lens_k)
    idx, _ = ops.npu_lightning_indexer(qi, ki.unsqueeze(1), w, layout_query="TND", layout_key="TND",
                                       actual_seq_lengths_query=cq[1:], actual_seq_lengths_key=ck[1:],
                                       sparse_count=K, cmp_ratio=r, cmp_residual_k=res)
    idx = idx[:, 0].cpu()
    for i in range(len(lens_q)):
        a, b, ka, kb = cq[i], cq[i + 1], ck[i], ck[i + 1]
        if kb > ka:
            sc = ops.indexer_scores(qi[a:b].unsqueeze(0), ki[ka:kb].unsqueeze(0), w[a:b].unsqueeze(0),
                                    cmp_ratio=r).cpu()
        else:
            sc = torch.zeros(1, b - a, 0)
        nv = np.array([O.valid_key_count(s, 0, r, kb - ka) for s in range(b - a)])
        ref = torch.from_numpy(O.topk_select_numpy(sc[0].numpy(), K, nv))
        assert torch.equal(idx[a:b].long(), ref.long()), f"sequence {i}"
    assert torch.all(idx[cq[2]:cq[3]] == -1)  # 3 tokens form no whole block: nothing to select


def test_indexer_bsnd_actual_seq_lengths():
    ops = _ops()
    B, S, H, D, K = 2, 64, 16, 128, 24
    g = torch.Generator().manual_seed(12)
    qi = torch.randn(B, S, H, D, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(B, S, 1, D, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(B, S, H, generator=g) * 0.01).to(DEV)
    idx, _ = ops.npu_lightning_indexer(qi, ki, w, actual_seq_lengths_query=[40, 64], actual_seq_lengths_key=[40, 64],
                                       sparse_count=K)
    idx = idx[:, :, 0].cpu()
    assert torch.all(idx[0, 40:] == -1)
    for b, n in ((0, 40), (1, 64)):
        ref, _ = ops.npu_lightning_indexer(qi[b : b + 1, :n], ki[b : b + 1, :n], w[b : b + 1, :n], sparse_count=K)
        assert torch.equal(idx[b, :n], ref[0, :, 0].cpu())


# ----- attention -----
LENS = [33, 0, 1, 150, 96]


@pytest.mark.parametrize("H", [64, 128])
def test_sparse_mla_fwd_bwd_varlen_equals_per_sequence(H):
    ops = _ops()
    K = 64
    T = sum(LENS)
    q, kv, dout, scale = _attn_inputs(T, T, H, seed=H)
    idx = _local_indices(LENS, LENS, K, seed=H)
    qd, kvd, idd, dod = q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV)
    cu = _cu(LENS)
    out, smax, ssum = ops.sparse_mla_fwd_varlen(qd, kvd, idd, scale, cu, cu)
    dq, dkv, mass = ops.sparse_mla_bwd_varlen(qd, kvd, idd, out, dod, smax, ssum, scale, cu, cu, return_mass=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_dq, ref_dkv = [], [], [], []
    for i, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        if a == b:
            continue
        sl = lambda t: t[a:b].unsqueeze(0)  # noqa: E731
        o1, m1, s1 = ops.sparse_mla_fwd(sl(qd), sl(kvd), sl(idd), scale)
        dq1, dkv1, mass1 = ops.sparse_mla_bwd(sl(qd), sl(kvd), sl(idd), o1, sl(dod), m1, s1, scale, return_mass=True)
        for got, ref, name in ((out, o1, "out"), (smax, m1, "smax"), (ssum, s1, "ssum"), (dq, dq1, "dq"),
                               (mass, mass1, "mass")):
            assert torch.equal(got[a:b].cpu(), ref[0].cpu()), f"{name} of sequence {i}"
        assert rel_err(dkv[a:b], dkv1[0]) <= 1e-6, f"dkv of sequence {i}"
        # per-sequence oracle, compared over the packed batch (a one-key row has dq = 0
        # exactly, so a sequence of such rows has no relative scale of its own)
        o_r, lse_r = O.sparse_mla_fwd(sl(q), sl(kv), sl(idx), scale)
        rdq, rdkv, _ = O.sparse_mla_bwd_closed_form(sl(q), sl(kv), sl(idx), o1.cpu(), lse_r, sl(dout), scale)
        ref_out.append(o_r[0])
        ref_lse.append(lse_r[0])
        ref_dq.append(rdq[0])
        ref_dkv.append(rdkv[0])
    assert rel_err(out.cpu(), torch.cat(ref_out)) <= BF16_TOL
    lse = smax.cpu().double() + torch.log(ssum.cpu().double())
    ref_lse = torch.cat(ref_lse)
    fin = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(lse), fin)
    assert torch.allclose(lse[fin], ref_lse[fin], atol=1e-3, rtol=1e-4)
    assert rel_err(dq.cpu(), torch.cat(ref_dq)) <= BF16_TOL
    assert rel_err(dkv.cpu(), torch.cat(ref_dkv)) <= BF16_TOL


def test_sparse_flash_attention_tnd_autograd_equals_bsnd():
    ops = _ops()
    H, K = 32, 40
    lens = [70, 5, 120]
    T = sum(lens)
    q, kv, dout, scale = _attn_inputs(T, T, H, seed=21)
    idx = _local_indices(lens, lens, K, seed=21)
    cu = _cu(lens)

    def leaves(qq, kk):
        qn = qq[..., :512].clone().to(DEV).requires_grad_(True)
        qp = qq[..., 512:].clone().to(DEV).requires_grad_(True)
        kn = kk[..., :512].clone().to(DEV).requires_grad_(True)
        kp = kk[..., 512:].clone().to(DEV).requires_grad_(True)
        return qn, qp, kn, kp

    qn, qp, kn, kp = leaves(q, kv.unsqueeze(1))
    out, _, _ = ops.npu_sparse_flash_attention(qn, kn, kn, idx.unsqueeze(1).to(DEV), query_rope=qp, key_rope=kp,
                                               scale_value=scale, layout_query="TND", layout_kv="TND",
                                               actual_seq_lengths_query=cu[1:], actual_seq_lengths_kv=cu[1:])
    out.backward(dout.to(DEV))
    for a, b in zip(cu[:-1], cu[1:]):
        rn, rp, rkn, rkp = leaves(q[a:b].unsqueeze(0), kv[a:b].unsqueeze(0).unsqueeze(2))
        o1, _, _ = ops.npu_sparse_flash_attention(rn, rkn, rkn, idx[a:b].view(1, b - a, 1, K).to(DEV), query_rope=rp,
                                                  key_rope=rkp, scale_value=scale)
        o1.backward(dout[a:b].unsqueeze(0).to(DEV))
        assert torch.equal(out[a:b].detach().cpu(), o1[0].detach().cpu())
        assert torch.equal(qn.grad[a:b].cpu(), rn.grad[0].cpu()) and torch.equal(qp.grad[a:b].cpu(), rp.grad[0].cpu())
        # key gradients are fp32 sums rounded to bf16: equal up to the rare rounding flip
        assert rel_err(kn.grad[a:b], rkn.grad[0]) <= 1e-3 and rel_err(kp.grad[a:b], rkp.grad[0]) <= 1e-3


# ----- indexer KL -----
def test_indexer_kl_tnd_equals_per_sequence():
    ops = _ops()
    H, K, HI, DI = 64, 48, 64, 128
    lens = [50, 1, 0, 140]
    T = sum(lens)
    q, kv, _, scale = _attn_inputs(T, T, H, seed=31)
    idx = _local_indices(lens, lens, K, seed=31, holes=0.05)
    g = torch.Generator().manual_seed(32)
    qi = torch.randn(T, HI, DI, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(T, 1, DI, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(T, HI, generator=g) * 0.01).to(DEV)
    qd, kvd, idd = q.to(DEV), kv.to(DEV), idx.to(DEV)
    cu = _cu(lens)
    _, smax, ssum = ops.sparse_mla_fwd_varlen(qd, kvd, idd, scale, cu, cu)
    # fp32 index operands (bf16 values): the op then returns fp32 gradients, compared below
    # bit for bit across the two layouts
    qi, ki = qi.float(), ki.float()
    dq_i, dk_i, dw, loss = ops.npu_sparse_lightning_indexer_grad_kl_loss(
        qd[..., :512], kvd[:, None, :512], qi, ki, w, idd.unsqueeze(1), smax, ssum, scale,
        query_rope=qd[..., 512:], key_rope=kvd[:, None, 512:], layout="TND", actual_seq_qlen=cu[1:],
        actual_seq_klen=cu[1:])
    torch.cuda.synchronize()
    total = 0.0
    for i, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        if a == b:
            continue
        sl = lambda t: t[a:b].unsqueeze(0)  # noqa: E731
        _, m1, s1 = ops.sparse_mla_fwd(sl(qd), sl(kvd), sl(idd), scale)
        r = ops.npu_sparse_lightning_indexer_grad_kl_loss(
            sl(qd)[..., :512], sl(kvd)[:, :, None, :512], sl(qi), sl(ki), sl(w), sl(idd).unsqueeze(2), m1, s1, scale,
            query_rope=sl(qd)[..., 512:], key_rope=sl(kvd)[:, :, None, 512:])
        assert torch.equal(dq_i[a:b].cpu(), r[0][0].cpu()), f"dq_idx of sequence {i}"
        assert rel_err(dk_i[a:b], r[1][0]) <= 1e-6, f"dk_idx of sequence {i}"
        assert torch.equal(dw[a:b].cpu(), r[2][0].cpu()), f"dw of sequence {i}"
        total += float(r[3])
    assert abs(float(loss) - total) <= 1e-5 * max(1.0, abs(total))


def test_attention_varlen_rejects_sequence_without_keys():
    from torchtitan_npu_simulator_amd import DSAError

    ops = _ops()
    q, kv, _, scale = _attn_inputs(8, 4, 16, seed=1)
    idx = torch.full((8, 4), -1, dtype=torch.int32)
    with pytest.raises(DSAError, match="no keys"):
        ops.sparse_mla_fwd_varlen(q.to(DEV), kv.to(DEV), idx.to(DEV), scale, [0, 4, 8], [0, 4, 4])


# ----- compressor -----
@pytest.mark.parametrize("D,r,overlap", [(512, 4, True), (128, 4, True), (128, 8, False)])
def test_compressor_tnd_parity(D, r, overlap):
    from torchtitan_npu_simulator_amd import tnd

    ops = _ops()
    # requests of lengths that are not multiples of r, the first starting mid-request
    pos = torch.cat([torch.arange(5, 5 + 23), torch.arange(0, 10), torch.arange(0, 3), torch.arange(0, 41)])
    T = pos.numel()
    g = torch.Generator().manual_seed(D + r)
    coff = 2 if overlap else 1
    kv = torch.randn(T, coff * D, generator=g)
    sc = torch.randn(T, coff * D, generator=g)
    ape = torch.randn(r, coff * D, generator=g) * 0.02
    bs = tnd.compressed_block_starts(pos, r)
    got = ops.compressor_pool_tnd(kv.to(DEV), sc.to(DEV), ape.to(DEV), r, bs.to(DEV), pos.to(DEV),
                                  overlap=overlap).cpu()
    ref = O.compressor_pool_tnd(kv.double(), sc.double(), ape.double(), r, bs, pos, overlap=overlap)
    assert got.shape == (bs.numel(), D)
    assert rel_err(got, ref) <= 1e-5
    w = torch.rand(D, generator=g) + 0.5
    got_n = ops.compressor_pool_tnd(kv.to(DEV), sc.to(DEV), ape.to(DEV), r, bs.to(DEV), pos.to(DEV), overlap=overlap,
                                    norm_weight=w.to(DEV)).cpu()
    ref_n = O.compressor_pool_tnd(kv, sc, ape, r, bs, pos, overlap=overlap, norm_weight=w, out_dtype=torch.bfloat16)
    assert rel_err(got_n.float(), ref_n) <= 2e-2
