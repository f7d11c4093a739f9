"""The binding-level DeepSeek-V4 ops and the torch.library custom ops on the GPU.

* npu_sparse_attn_sharedkv (out, softmax_lse) and npu_sparse_attn_sharedkv_grad (d_query,
  d_ori_kv, d_cmp_kv, d_sinks) against the oracle's ``sparse_attn_sink`` and its fp64
  autograd (bf16 2e-2; the LSE includes the sink), for ratio 4 with a given top-k and ratio
  128 (every causal compressed block);
* every dsa_mi355x custom op through ``torch.library.opcheck`` (schema, fake tensors,
  autograd registration) on small inputs;
* the absorb-mode attention custom op compiled with ``torch.compile(fullgraph=True)``
  (aot_eager) gives the eager results, forward and gradients.
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import attn_inputs, rand_indices, rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _v4_case(S, H, ratio, K, seed, D=512):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, S, H, D, generator=g).bfloat16()
    ori = torch.randn(1, S, D, generator=g).bfloat16()
    n_cmp = S // ratio
    cmp = torch.randn(1, n_cmp, D, generator=g).bfloat16()
    sink = torch.randn(H, generator=g)
    idx = None
    if ratio == 4:
        idx = torch.full((1, S, K), -1, dtype=torch.int32)
        for s in range(S):
            nv = min(n_cmp, (s + 1) // ratio)
            c = min(K, nv)
            if c:
                idx[0, s, :c] = torch.sort(torch.randperm(nv, generator=g)[:c]).values.int() + S
    dout = torch.randn(1, S, H, D, generator=g).bfloat16()
    return q, ori, cmp, sink, idx, dout


@pytest.mark.parametrize("S,H,ratio,K", [(256, 16, 4, 32), (384, 32, 128, 0)])
def test_sharedkv_binding_forward_and_grad(S, H, ratio, K):
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    q, ori, cmp, sink, idx, dout = _v4_case(S, H, ratio, K, seed=S + ratio)
    scale = 512 ** -0.5
    qd, od, cd, sd = q.to(DEV), ori.to(DEV).unsqueeze(2), cmp.to(DEV).unsqueeze(2), sink.to(DEV)
    cidx = None if idx is None else idx.to(DEV).unsqueeze(2)
    meta = ops.npu_sparse_attn_sharedkv_metadata(None, None, None, None, None, H, 1, 512, 1, S, S, 0, K, ratio, 4, 3,
                                                 127, 0, "BSND", "BSND", True, True, device=DEV)
    out, lse = ops.npu_sparse_attn_sharedkv(qd, od, cd, None, cidx, sinks=sd, metadata=meta, softmax_scale=scale,
                                            cmp_ratio=ratio)
    assert out.shape == q.shape and out.dtype == q.dtype and lse.shape == (1, S, H, 1) and lse.dtype == torch.float32
    dq, d_ori, d_cmp, d_sink = ops.npu_sparse_attn_sharedkv_grad(qd, od, cd, dout.to(DEV), out, lse, None, cidx,
                                                                 sinks=sd, scale_value=scale, cmp_ratio=ratio)
    torch.cuda.synchronize()
    assert d_ori.shape == od.shape and d_cmp.shape == cd.shape and d_sink.shape == sd.shape
    assert dq.dtype == q.dtype and d_ori.dtype == ori.dtype and d_sink.dtype == sink.dtype
    full_idx = O.v4_attn_indices(1, S, 128, ratio, S, cmp_idxs=idx)
    oq = q.double().requires_grad_(True)
    okv = torch.cat([ori, cmp], dim=1).double().requires_grad_(True)
    osk = sink.double().requires_grad_(True)
    ref, ref_lse = O.sparse_attn_sink(oq, okv, osk, full_idx, scale)
    ref.backward(dout.double())
    assert rel_err(out, ref.detach()) <= 2e-2
    assert float((lse[..., 0].double().cpu() - ref_lse.detach()).abs().max()) <= 2e-2
    assert rel_err(dq, oq.grad) <= 2e-2
    assert rel_err(torch.cat([d_ori[:, :, 0], d_cmp[:, :, 0]], dim=1), okv.grad) <= 2e-2
    assert rel_err(d_sink, osk.grad) <= 2e-2


def _opcheck(op, args, kwargs=None):
    torch.library.opcheck(op, args, kwargs or {},
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


def test_custom_ops_opcheck():
    from torchtitan_npu_simulator_amd import library  # noqa: F401
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    lib = torch.ops.dsa_mi355x
    S, H, K = 64, 16, 24
    q, kv, dout, scale = attn_inputs(S, H, seed=3)
    idx = rand_indices(S, K, seed=3).to(DEV).unsqueeze(2)
    qd, kvd = q.to(DEV), kv.to(DEV)
    qn = qd[..., :512].contiguous().requires_grad_(True)
    qp = qd[..., 512:].contiguous().requires_grad_(True)
    kn = kvd[:, :, None, :512].contiguous().requires_grad_(True)
    kp = kvd[:, :, None, 512:].contiguous().requires_grad_(True)
    _opcheck(lib.npu_sparse_flash_attention, (qn, kn, kn, idx, qp, kp, scale, 3))
    out, smax, ssum = lib.npu_sparse_flash_attention(qn, kn, kn, idx, qp, kp, scale, 3)
    _opcheck(lib.npu_sparse_flash_attention_grad,
             (qn.detach(), kn.detach(), qp.detach(), kp.detach(), idx, out.detach(), dout.to(DEV), smax, ssum, scale,
              3))
    g = torch.Generator().manual_seed(4)
    qi = torch.randn(1, S, 64, 128, generator=g).bfloat16().to(DEV)
    ki = torch.randn(1, S, 1, 128, generator=g).bfloat16().to(DEV)
    w = (torch.rand(1, S, 64, generator=g) * 0.01).to(DEV)
    _opcheck(lib.npu_lightning_indexer, (qi, ki, w), dict(sparse_count=K, return_value=True))
    # fp8 operands: opcheck's schema mode cannot handle float8 tensors, so the fake
    # implementation is compared with the real op directly
    q8, qs = ops.quantize_fp8_per_row(qi)
    k8, ks = ops.quantize_fp8_per_row(ki)
    i8, v8 = lib.npu_lightning_indexer(q8, k8, w, sparse_count=K, return_value=True, query_scale=qs, key_scale=ks)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode(allow_non_fake_inputs=True):
        fi, fv = lib.npu_lightning_indexer(q8, k8, w, sparse_count=K, return_value=True, query_scale=qs, key_scale=ks)
    assert (fi.shape, fi.dtype, fv.shape, fv.dtype) == (i8.shape, i8.dtype, v8.shape, v8.dtype)
    _opcheck(lib.npu_sparse_lightning_indexer_grad_kl_loss,
             (qn.detach(), kn.detach(), qi, ki, w, idx, smax, ssum),
             dict(query_rope=qp.detach(), key_rope=kp.detach(), scale_value=scale))
    qv, ori, cmp, sink, cidx, _ = _v4_case(64, 16, 4, 8, seed=5)
    args = (qv.to(DEV).requires_grad_(True), ori.to(DEV).unsqueeze(2).requires_grad_(True),
            cmp.to(DEV).unsqueeze(2).requires_grad_(True), cidx.to(DEV).unsqueeze(2), sink.to(DEV).requires_grad_(True),
            None, 512 ** -0.5, 4)
    _opcheck(lib.npu_sparse_attn_sharedkv, args)


def test_compiled_attention_matches_eager():
    from torchtitan_npu_simulator_amd import library  # noqa: F401

    S, H, K = 96, 16, 32
    q, kv, dout, scale = attn_inputs(S, H, seed=7)
    idx = rand_indices(S, K, seed=7).to(DEV).unsqueeze(2)
    dout = dout.to(DEV)

    def step(qn, qp, kn, kp):
        out, _, _ = torch.ops.dsa_mi355x.npu_sparse_flash_attention(qn, kn, kn, idx, qp, kp, scale, 3)
        return out

    def leaves():
        qd, kvd = q.to(DEV), kv.to(DEV)
        return [qd[..., :512].contiguous().requires_grad_(True), qd[..., 512:].contiguous().requires_grad_(True),
                kvd[:, :, None, :512].contiguous().requires_grad_(True),
                kvd[:, :, None, 512:].contiguous().requires_grad_(True)]

    eager_in = leaves()
    eager = step(*eager_in)
    eager.backward(dout)
    comp_in = leaves()
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)(*comp_in)
    compiled.backward(dout)
    torch.cuda.synchronize()
    assert torch.equal(compiled, eager)
    for a, b in zip(comp_in, eager_in):
        assert rel_err(a.grad, b.grad) <= 1e-6


def test_kernel_timing_records_each_launch():
    """dsa_kernel_timing: event pairs around the library's launches while enabled, summed per
    kernel name; nothing recorded once it is off."""
    from torchtitan_npu_simulator_amd import _lib
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    x = torch.randn(300, 128, device=DEV).bfloat16()
    with _lib.kernel_timing() as kt:
        for _ in range(3):
            ops.quantize_fp8_per_row(x)
        torch.cuda.synchronize()
    summary = kt.summary()
    assert list(summary) == ["quantize_fp8_kernel"]
    total_ms, launches = summary["quantize_fp8_kernel"]
    assert launches == 3 and total_ms > 0.0
    ops.quantize_fp8_per_row(x)  # timing is off: the last window's summary is unchanged
    torch.cuda.synchronize()
    lib = _lib.load_library()
    assert lib.dsa_kernel_timing_count() == 1
    with _lib.kernel_timing() as kt2:  # a new window starts empty
        pass
    assert kt2.summary() == {}


def test_device_cu_seqlens_read_back_once_per_version():
    """A device cu_seqlens tensor shared by the ops of a step is read back once; an in-place
    change (new version) is seen."""
    from torchtitan_npu_simulator_amd import _lib

    cu = torch.tensor([0, 100, 250], dtype=torch.int32, device=DEV)
    first = _lib.host_ints(cu)
    assert first == [0, 100, 250] and _lib.host_ints(cu) is first  # cached
    cu[2] = 260
    assert _lib.host_ints(cu) == [0, 100, 260]


@pytest.mark.parametrize("mode,pre,nxt,s_kv", [(3, 100, 0, 384), (3, 40, -3, 384), (0, 50, 70, 384), (3, 200, 5, 512)])
def test_lightning_indexer_band(mode, pre, nxt, s_kv):
    """npu_lightning_indexer with a pre_tokens / next_tokens band (binding.cpp:12-16): bit-exact
    against the oracle's top-k on the GPU's own scores with every key outside the row's band
    [a(s) - pre, a(s) + next] (a(s) = s, or s + q_offset in sparse_mode 3) excluded."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    S, K, HI, DI = 256, 48, 64, 128
    g = torch.Generator().manual_seed(pre + s_kv)
    qi = torch.randn(1, S, HI, DI, generator=g).bfloat16().to(DEV)
    ki = torch.randn(1, s_kv, DI, generator=g).bfloat16().to(DEV)
    w = (torch.rand(1, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5).to(DEV)
    q_off = s_kv - S if mode == 3 else 0
    idx, vals = ops.npu_lightning_indexer(qi, ki.unsqueeze(2), w, sparse_count=K, sparse_mode=mode, pre_tokens=pre,
                                          next_tokens=nxt, return_value=True)
    sc = ops.indexer_scores(qi, ki, w, q_offset=q_off if mode == 3 else ops._NO_MASK_OFFSET).cpu()[0].double()
    t = torch.arange(s_kv).view(1, -1)
    a = torch.arange(S).view(-1, 1) + q_off
    ok = (t >= a - pre) & (t <= a + nxt)
    if mode == 3:
        ok &= t <= a
    sc = sc.masked_fill(~ok, float("nan")).float().numpy()
    ref = O.topk_select_numpy(sc, K)
    assert torch.equal(idx[0, :, 0].cpu(), torch.from_numpy(ref).int())
    assert (idx >= 0).any()


def test_kl_loss_band_and_bsnd_lengths():
    """npu_sparse_lightning_indexer_grad_kl_loss: (1) a pre_tokens band drops the selected keys
    outside it from target and student alike - the same result as those slots set to -1;
    (2) BSND with actual_seq_qlen / actual_seq_klen equals each batch's valid prefix run on
    its own, with zero gradients on padded rows and keys."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops
    from torchtitan_npu_simulator_amd.torch_npu_ops import _band_mask_indices

    S, H, K, HI, DI = 192, 16, 32, 64, 128
    q, kv, _, _ = attn_inputs(S, H, seed=3)
    g = torch.Generator().manual_seed(4)
    qi = torch.randn(2, S, HI, DI, generator=g).bfloat16()
    ki = torch.randn(2, S, 1, DI, generator=g).bfloat16()
    w = torch.rand(2, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5
    q2 = torch.cat([q, torch.randn_like(q.float()).bfloat16() / 24]).to(DEV)
    kv2 = torch.cat([kv, torch.randn_like(kv.float()).bfloat16()]).to(DEV)
    idx2 = torch.cat([rand_indices(S, K, seed=1), rand_indices(S, K, seed=2)]).to(DEV)
    scale = 576 ** -0.5
    _, smax, ssum = ops.sparse_mla_fwd(q2, kv2, idx2, scale)
    common = dict(query_rope=q2[..., 512:], key_rope=kv2[..., 512:].unsqueeze(2))
    args = (q2[..., :512], kv2[..., :512].unsqueeze(2), qi.to(DEV), ki.to(DEV), w.to(DEV))
    # (1) the band
    banded = ops.npu_sparse_lightning_indexer_grad_kl_loss(*args, idx2, smax, ssum, scale, pre_tokens=60, **common)
    masked = _band_mask_indices(idx2, 3, 0, 60, 65536)
    assert bool((masked != idx2).any())
    ref = ops.npu_sparse_lightning_indexer_grad_kl_loss(*args, masked, smax, ssum, scale, **common)
    for a_, b_ in zip(banded, ref):
        assert torch.equal(a_, b_)
    # (2) per-batch lengths: batch 0 keeps 150 rows / keys, batch 1 all of them
    lq, lk = [150, S], [150, S]
    got = ops.npu_sparse_lightning_indexer_grad_kl_loss(*args, idx2, smax, ssum, scale, actual_seq_qlen=lq,
                                                        actual_seq_klen=lk, **common)
    loss = 0.0
    for b in range(2):
        n = lq[b]
        qb = q2[b:b + 1, :n].contiguous()
        kvb = kv2[b:b + 1, :n].contiguous()
        ib = idx2[b:b + 1, :n].contiguous()
        _, mb, sb = ops.sparse_mla_fwd(qb, kvb, ib, scale)
        one = ops.npu_sparse_lightning_indexer_grad_kl_loss(
            qb[..., :512], kvb[..., :512].unsqueeze(2), qi[b:b + 1, :n].to(DEV), ki[b:b + 1, :n].to(DEV),
            w[b:b + 1, :n].to(DEV), ib, mb, sb, scale, query_rope=qb[..., 512:], key_rope=kvb[..., 512:].unsqueeze(2))
        torch.testing.assert_close(got[0][b:b + 1, :n], one[0], rtol=1e-5, atol=1e-7)
        torch.testing.assert_close(got[1][b:b + 1, :n], one[1], rtol=1e-5, atol=1e-7)
        torch.testing.assert_close(got[2][b:b + 1, :n], one[2], rtol=1e-5, atol=1e-7)
        assert float(got[0][b, n:].abs().sum()) == 0.0 and float(got[1][b, n:].abs().sum()) == 0.0
        loss += float(one[3])
    assert abs(float(got[3]) - loss) <= 1e-5 * abs(loss)


def test_kl_op_takes_the_attention_backward_mass(monkeypatch):
    """The op-level route as the reference's dsa.py calls it (converters/kernels/dsa.py:238-253,
    then :159-177): npu_sparse_flash_attention on q_nope / q_pe and k_nope / k_pe split views,
    its backward, then npu_sparse_lightning_indexer_grad_kl_loss on the same (detached)
    pieces, indices and statistics.  The backward's mass reaches the KL op (dsa_attn_mass is
    not called), the results equal a recomputed target's bit for bit, the entry is used
    once, and an in-place change of the statistics makes the op recompute."""
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    S, H, K, HI, DI = 192, 16, 32, 64, 128
    q, kv, dout, scale = attn_inputs(S, H, seed=7)
    g = torch.Generator().manual_seed(8)
    qi = torch.randn(1, S, HI, DI, generator=g).bfloat16().to(DEV)
    ki = torch.randn(1, S, 1, DI, generator=g).bfloat16().to(DEV)
    w = (torch.rand(1, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5).to(DEV)
    q = q.to(DEV).requires_grad_()
    k = kv.to(DEV).unsqueeze(2).requires_grad_()  # [1,S,1,576]
    idx = rand_indices(S, K, seed=9).to(DEV).unsqueeze(2)  # [1,S,1,K]
    q_nope, q_pe = torch.split(q, [512, 64], dim=-1)
    k_nope, k_pe = torch.split(k, [512, 64], dim=-1)
    out, smax, ssum = ops.npu_sparse_flash_attention(q_nope, k_nope, k_nope, idx, query_rope=q_pe, key_rope=k_pe,
                                                     scale_value=scale)
    (out.float() * dout.to(DEV).float()).sum().backward()
    args = (q_nope.detach(), k_nope.detach(), qi, ki, w, idx, smax, ssum, scale)
    kw = dict(query_rope=q_pe.detach(), key_rope=k_pe.detach())
    assert ops._attn_mass_entry is not None

    def no_recompute(*a, **k_):
        raise AssertionError("the KL op recomputed a mass the backward had left for it")

    real_attn_mass = ops.attn_mass
    monkeypatch.setattr(ops, "attn_mass", no_recompute)
    taken = ops.npu_sparse_lightning_indexer_grad_kl_loss(*args, **kw)
    assert ops._attn_mass_entry is None
    monkeypatch.setattr(ops, "attn_mass", real_attn_mass)
    recomputed = ops.npu_sparse_lightning_indexer_grad_kl_loss(*args, **kw)
    for a_, b_ in zip(taken, recomputed):
        assert torch.equal(a_, b_)
    assert float(taken[3]) > 0.0

    # a statistics tensor changed in place after the backward: the kept mass is not used
    out2, smax2, ssum2 = ops.npu_sparse_flash_attention(q_nope, k_nope, k_nope, idx, query_rope=q_pe,
                                                        key_rope=k_pe, scale_value=scale)
    (out2.float() * dout.to(DEV).float()).sum().backward()
    assert ops._attn_mass_entry is not None
    ssum2.mul_(2.0)
    calls = []

    def counting(*a, **k_):
        calls.append(1)
        return real_attn_mass(*a, **k_)

    monkeypatch.setattr(ops, "attn_mass", counting)
    ops.npu_sparse_lightning_indexer_grad_kl_loss(q_nope.detach(), k_nope.detach(), qi, ki, w, idx, smax2, ssum2,
                                                  scale, **kw)
    assert calls == [1]
