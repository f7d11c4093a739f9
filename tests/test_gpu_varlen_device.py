"""Packed varlen ("TND") batches whose sequence bounds live on the GPU.

With device ``cu_seqlens`` the ops take their device paths: the indexer reads each row's key
window on the device (dsa_lightning_indexer_tnd, persistent score kernels over the
(query group, key span) pairs that hold work, top-k over each row's window), and the
attention, its mass and the indexer KL run the whole batch as one [1, T] problem on global
key rows (dsa_tnd_global_indices).  Nothing is copied back to the host, which these tests
check by making ``_lib.host_ints`` (the only read-back of the host schedule) raise.

The host schedule (``tests/test_gpu_varlen.py``, itself held to the per-sequence
fixed-length entry points and the oracle) is the reference here: indices, values, out,
softmax statistics, dQ, the mass, dq_I, dw and the row losses bit for bit (the same kernels
compute every row from the same keys in the same order); dKV and dk_I to 1e-6 relative (the
key-major reductions group the same fp32 contributions by other segments).  Batches mix an
empty sequence, a one-token sequence and lengths that are not multiples of any tile; the
indexer cases include compressed keys with device residuals and rows past 16384 keys (the
top-k candidate lists).
"""

import numpy as np
import pytest
import torch

from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _cu(lens):
    return [0] + list(np.cumsum(lens).tolist())


@pytest.fixture
def no_readback(monkeypatch):
    """Make any host read-back of a GPU tensor of sequence bounds fail inside the test (host
    lists, which the reference runs of the host schedule pass, still go through)."""
    from torchtitan_npu_simulator_amd import _lib

    real = _lib.host_ints

    def _refuse(values):
        if isinstance(values, torch.Tensor) and values.is_cuda:
            raise AssertionError("device path read sequence bounds back to the host")
        return real(values)

    monkeypatch.setattr(_lib, "host_ints", _refuse)


def _indexer_inputs(T, T_k, H, seed, fp8):
    ops = _ops()
    g = torch.Generator().manual_seed(seed)
    qi = torch.randn(T, H, 128, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(T_k, 128, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(T, H, generator=g) * 0.01).to(DEV)  # signed weights
    qs = ks = None
    if fp8:
        qi, qs = ops.quantize_fp8_per_row(qi)
        ki, ks = ops.quantize_fp8_per_row(ki)
    return qi, ki, w, qs, ks


@pytest.mark.parametrize("fp8,H", [(True, 64), (False, 64), (True, 32)])
def test_indexer_device_bounds_equals_host_schedule(fp8, H, no_readback):
    ops = _ops()
    lens = [37, 0, 130, 1, 200, 75]
    T, K = sum(lens), 48
    qi, ki, w, qs, ks = _indexer_inputs(T, T, H, 5 + H, fp8)
    cu = _cu(lens)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=DEV)
    idx, vals = ops.lightning_indexer_varlen(qi, ki, w, cu_d, cu_d, K, return_value=True, query_scale=qs,
                                             key_scale=ks)
    torch.cuda.synchronize()
    ref_i, ref_v = _host_indexer(qi, ki, w, cu, K, qs, ks)
    assert torch.equal(idx.cpu(), ref_i.cpu())
    assert torch.equal(vals.cpu(), ref_v.cpu())


def _host_indexer(qi, ki, w, cu, K, qs, ks, **kw):
    """The host schedule with host-list bounds (no read-back needed either)."""
    return _ops().lightning_indexer_varlen(qi, ki, w, cu, cu, K, return_value=True, query_scale=qs, key_scale=ks,
                                           **kw)


def test_indexer_device_bounds_compressed_keys(no_readback):
    ops = _ops()
    r = 4
    lens_q = [70, 1, 0, 129, 40]
    res = [1, 0, 0, 3, 2]
    lens_k = [(n - e) // r for n, e in zip(lens_q, res)]
    T, T_k, K = sum(lens_q), sum(lens_k), 16
    qi, ki, w, qs, ks = _indexer_inputs(T, T_k, 64, 21, True)
    cu_q, cu_k = _cu(lens_q), _cu(lens_k)
    dq = torch.tensor(cu_q, dtype=torch.int32, device=DEV)
    dk = torch.tensor(cu_k, dtype=torch.int32, device=DEV)
    dres = torch.tensor(res, dtype=torch.int32, device=DEV)
    for mode in (3, 0):
        idx, vals = ops.lightning_indexer_varlen(qi, ki, w, dq, dk, K, sparse_mode=mode, cmp_ratio=r,
                                                 cmp_residual_k=dres, return_value=True, query_scale=qs,
                                                 key_scale=ks, index_offset=7)
        ref_i, ref_v = ops.lightning_indexer_varlen(qi, ki, w, cu_q, cu_k, K, sparse_mode=mode, cmp_ratio=r,
                                                    cmp_residual_k=res, return_value=True, query_scale=qs,
                                                    key_scale=ks, index_offset=7)
        assert torch.equal(idx.cpu(), ref_i.cpu()), f"sparse_mode {mode}"
        assert torch.equal(vals.cpu(), ref_v.cpu()), f"sparse_mode {mode}"


def test_indexer_device_bounds_long_rows(no_readback):
    """A sequence past 16384 keys: the top-k of every row goes through candidate lists (the
    packed key count decides the path), also for the short sequences of the batch."""
    ops = _ops()
    lens = [300, 17000, 1]
    T, K = sum(lens), 2048
    qi, ki, w, qs, ks = _indexer_inputs(T, T, 64, 33, True)
    cu = _cu(lens)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=DEV)
    idx, vals = ops.lightning_indexer_varlen(qi, ki, w, cu_d, cu_d, K, return_value=True, query_scale=qs,
                                             key_scale=ks)
    ref_i, ref_v = _host_indexer(qi, ki, w, cu, K, qs, ks)
    assert torch.equal(idx.cpu(), ref_i.cpu())
    assert torch.equal(vals.cpu(), ref_v.cpu())


def test_indexer_device_bounds_small_workspace_chunks(no_readback, monkeypatch):
    """Row chunks of a few query groups (a score budget of 64 rows): chunk edges fall inside
    sequences and inside query groups."""
    ops = _ops()
    monkeypatch.setattr(ops, "_SCORE_BUDGET_BYTES", 64 * 4 * 400)
    lens = [37, 150, 1, 211]
    T, K = sum(lens), 32
    qi, ki, w, qs, ks = _indexer_inputs(T, T, 64, 41, True)
    cu = _cu(lens)
    idx, vals = ops.lightning_indexer_varlen(qi, ki, w, torch.tensor(cu, dtype=torch.int32, device=DEV),
                                             torch.tensor(cu, dtype=torch.int32, device=DEV), K, return_value=True,
                                             query_scale=qs, key_scale=ks)
    ref_i, ref_v = _host_indexer(qi, ki, w, cu, K, qs, ks)
    assert torch.equal(idx.cpu(), ref_i.cpu())
    assert torch.equal(vals.cpu(), ref_v.cpu())


# ----- global indices -----
def test_global_indices_rule():
    """Each slot against the per-sequence rule, computed here on the host: kept iff
    0 <= v < len_k and v <= s_local + max(0, len_k - len_q), then offset by the sequence's
    first key; everything else -1 (out of range, past the causal limit, negative)."""
    ops = _ops()
    lens_q, lens_k = [5, 0, 9, 1, 12], [7, 3, 9, 0, 4]
    T, T_k, K = sum(lens_q), sum(lens_k), 16
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(-3, 14, (T, K), generator=g, dtype=torch.int32)
    cq, ck = _cu(lens_q), _cu(lens_k)
    got = ops.tnd_global_indices(idx.to(DEV), torch.tensor(cq, dtype=torch.int32, device=DEV),
                                 torch.tensor(ck, dtype=torch.int32, device=DEV), T_k).cpu()
    want = torch.full_like(idx, -1)
    for i in range(len(lens_q)):
        off = max(0, lens_k[i] - lens_q[i])
        for sl in range(lens_q[i]):
            s = cq[i] + sl
            for j in range(K):
                v = int(idx[s, j])
                if 0 <= v < lens_k[i] and v <= sl + off:
                    want[s, j] = ck[i] + v
    assert torch.equal(got, want)


# ----- attention, mass, indexer KL -----
def _local_indices(lens_q, lens_k, K, seed, holes=0.1):
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
    return torch.stack(rows)


@pytest.mark.parametrize("H", [64, 128])
def test_attention_and_kl_device_bounds_equal_host_schedule(H, no_readback):
    ops = _ops()
    lens = [33, 0, 1, 150, 96, 260]
    T, K = sum(lens), 64
    g = torch.Generator().manual_seed(H)
    q = torch.randn(T, H, 576, generator=g).to(torch.bfloat16).to(DEV)
    kv = torch.randn(T, 576, generator=g).to(torch.bfloat16).to(DEV)
    dout = torch.randn(T, H, 512, generator=g).to(torch.bfloat16).to(DEV)
    qi = torch.randn(T, 64, 128, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(T, 128, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(T, 64, generator=g) * 0.01).to(DEV)
    idx = _local_indices(lens, lens, K, seed=H).to(DEV)
    scale = 576 ** -0.5
    cu = _cu(lens)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=DEV)
    runs = {}
    for name, b in (("host", cu), ("device", cu_d)):
        out, smax, ssum = ops.sparse_mla_fwd_varlen(q, kv, idx, scale, b, b)
        dq, dkv, mass = ops.sparse_mla_bwd_varlen(q, kv, idx, out, dout, smax, ssum, scale, b, b, return_mass=True)
        mass2 = ops.attn_mass_varlen(q, kv, idx, smax, ssum, scale, b, b)
        dq_i, dk_i, dw, loss = ops.indexer_kl_grad_from_mass_varlen(qi, ki, w, idx, mass, b, b)
        runs[name] = dict(out=out, smax=smax, ssum=ssum, dq=dq, dkv=dkv, mass=mass, mass2=mass2, dq_i=dq_i,
                          dk_i=dk_i, dw=dw, loss=loss)
    torch.cuda.synchronize()
    h, d = runs["host"], runs["device"]
    for k in ("out", "smax", "ssum", "dq", "mass", "mass2", "dq_i", "dw", "loss"):
        assert torch.equal(d[k].cpu(), h[k].cpu()), k
    # (the stand-alone mass kernel sums the heads in another grouping than the backward's
    # score kernel when H < 128)
    assert rel_err(d["mass2"].cpu(), d["mass"].cpu()) <= 1e-6
    for k in ("dkv", "dk_i"):
        assert rel_err(d[k].cpu(), h[k].cpu()) <= 1e-6, k


def test_op_surface_device_lengths(no_readback):
    """npu_sparse_flash_attention / npu_sparse_lightning_indexer_grad_kl_loss / npu_lightning_indexer
    in layout TND with device actual_seq_lengths (cumulative ends): forward, backward and the KL
    op with no host read, equal to the same calls with host lengths."""
    ops = _ops()
    lens = [50, 1, 130]
    T, H, K = sum(lens), 64, 32
    g = torch.Generator().manual_seed(8)
    ends = list(np.cumsum(lens).tolist())
    ends_d = torch.tensor(ends, dtype=torch.int64, device=DEV)
    qi = torch.randn(T, 64, 128, generator=g).to(torch.bfloat16).to(DEV)
    ki = torch.randn(T, 1, 128, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.rand(T, 64, generator=g) * 0.01).to(torch.bfloat16).to(DEV)
    q = torch.randn(T, H, 512, generator=g).to(torch.bfloat16).to(DEV)
    q_pe = torch.randn(T, H, 64, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(T, 1, 512, generator=g).to(torch.bfloat16).to(DEV)
    k_pe = torch.randn(T, 1, 64, generator=g).to(torch.bfloat16).to(DEV)
    dout = torch.randn(T, H, 512, generator=g).to(torch.bfloat16).to(DEV)
    res = {}
    for name, e in (("host", ends), ("device", ends_d)):
        idx, _ = ops.npu_lightning_indexer(qi, ki, w, actual_seq_lengths_query=e, actual_seq_lengths_key=e,
                                           layout_query="TND", layout_key="TND", sparse_count=K)
        qq, kk, qp, kp = (t.clone().requires_grad_(True) for t in (q, k, q_pe, k_pe))
        out, smax, ssum = ops.npu_sparse_flash_attention(qq, kk, kk, idx, query_rope=qp, key_rope=kp,
                                                         scale_value=576 ** -0.5, layout_query="TND",
                                                         layout_kv="TND", actual_seq_lengths_query=e,
                                                         actual_seq_lengths_kv=e)
        out.backward(dout)
        kl = ops.npu_sparse_lightning_indexer_grad_kl_loss(qq.detach(), kk.detach(), qi, ki, w, idx, smax, ssum,
                                                           scale_value=576 ** -0.5, query_rope=qp.detach(),
                                                           key_rope=kp.detach(), actual_seq_qlen=e,
                                                           actual_seq_klen=e, layout="TND")
        res[name] = dict(idx=idx, out=out.detach(), dq=qq.grad, dqp=qp.grad, dk=kk.grad, dkp=kp.grad, dqi=kl[0],
                         dki=kl[1], dw=kl[2], loss=kl[3])
    torch.cuda.synchronize()
    h, d = res["host"], res["device"]
    for k_ in ("idx", "out", "dq", "dqp", "dqi", "dw", "loss"):
        assert torch.equal(d[k_].cpu(), h[k_].cpu()), k_
    for k_ in ("dk", "dkp", "dki"):
        assert rel_err(d[k_].float().cpu(), h[k_].float().cpu()) <= 1e-2, k_  # bf16 outputs of fp32 sums
