"""Parity of dsa_sparse_mla_bwd (dQ, dKV) and dsa_attn_mass (HIP) against the CPU oracle.

Gradients: relative error ||gpu - oracle|| / ||oracle|| <= 2e-2 in bf16 (contract
tolerance), <= 1e-5 in fp32.  The oracle backward is the closed-form flash-attention
backward in fp64, itself pinned to torch.autograd (tests/test_oracle.py).
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import attn_inputs, rand_indices, rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BF16_TOL = 2e-2


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _gpu_fwd_bwd(q, kv, idx, dout, scale, q_offset=0, workspace_bytes=None):
    ops = _ops()
    qd, kvd, idd, dod = q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV)
    out, smax, ssum = ops.sparse_mla_fwd(qd, kvd, idd, scale, q_offset=q_offset)
    dq, dkv = ops.sparse_mla_bwd(qd, kvd, idd, out, dod, smax, ssum, scale, q_offset=q_offset,
                                 workspace_bytes=workspace_bytes)
    torch.cuda.synchronize()
    return out.cpu(), smax.cpu(), ssum.cpu(), dq.cpu(), dkv.cpu()


@pytest.mark.parametrize(
    "S,H,K,q_offset,seed,shuffle,holes",
    [
        (256, 128, 128, 0, 0, False, 0.0),
        (160, 128, 96, 32, 1, True, 0.2),  # arbitrary slot order, -1 holes, CP shard offset
        (128, 16, 64, 0, 2, False, 0.0),  # few heads (one partial head group)
        (96, 72, 40, 0, 3, True, 0.0),  # head count not a multiple of 16
    ],
)
def test_bwd_bf16_parity(S, H, K, q_offset, seed, shuffle, holes):
    q, kv, dout, scale = attn_inputs(S, H, q_offset=q_offset, seed=seed)
    idx = rand_indices(S, K, q_offset=q_offset, seed=seed, shuffle=shuffle, holes=holes)
    out, smax, ssum, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout, scale, q_offset)
    ref_out, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale, q_offset=q_offset)
    # backward of the bf16 forward output, as the GPU sees it
    rdq, rdkv, _ = O.sparse_mla_bwd_closed_form(q, kv, idx, out, ref_lse, dout, scale, q_offset=q_offset)
    assert rel_err(dq, rdq) <= BF16_TOL, rel_err(dq, rdq)
    assert rel_err(dkv, rdkv) <= BF16_TOL, rel_err(dkv, rdkv)
    # and against autograd of the exact forward
    adq, adkv = O.sparse_mla_bwd(q, kv, idx, dout, scale, q_offset=q_offset)
    assert rel_err(dq, adq) <= BF16_TOL and rel_err(dkv, adkv) <= BF16_TOL


@pytest.mark.parametrize(
    "S,H,K,q_offset,seed,holes,workspace",
    [
        (256, 128, 128, 0, 31, 0.0, None),
        (160, 128, 96, 32, 32, 0.2, None),  # -1 holes, CP shard offset
        (128, 16, 64, 0, 33, 0.0, None),  # one partial head group
        (96, 72, 40, 0, 34, 0.1, 40 * (256 * 2 + 512 * 2 + 4) * 24 + 3 * 97 * 4 + 8192),  # row chunks
    ],
)
def test_bwd_bf16_rows_of_512_columns(S, H, K, q_offset, seed, holes, workspace):
    """The rope-less variant (DeepSeek-V4 rows, d_qk = d_v = 512): dQ and dKV, with the
    contribution rows and the key-major reduction 512 wide."""
    q, kv, dout, scale = attn_inputs(S, H, q_offset=q_offset, seed=seed, d_qk=512)
    idx = rand_indices(S, K, q_offset=q_offset, seed=seed, shuffle=True, holes=holes)
    out, smax, ssum, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout, scale, q_offset, workspace_bytes=workspace)
    assert dq.shape == q.shape and dkv.shape == kv.shape
    _, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale, q_offset=q_offset)
    rdq, rdkv, _ = O.sparse_mla_bwd_closed_form(q, kv, idx, out, ref_lse, dout, scale, q_offset=q_offset)
    assert rel_err(dq, rdq) <= BF16_TOL, rel_err(dq, rdq)
    assert rel_err(dkv, rdkv) <= BF16_TOL, rel_err(dkv, rdkv)


@pytest.mark.parametrize("K", [96, 99])
def test_bwd_long_kv_spans_several_counting_ranges(K):
    """A KV prefix of 40000 rows: the key-major CSR behind dKV counts keys in 16384-key
    ranges, so the slots (boundary keys 16383/16384, 32767/32768 in every row) fall in
    three ranges; K = 99 takes the scalar index loads."""
    S, H = 24, 16
    s_kv = 40000
    q_offset = s_kv - S
    q, kv, dout, scale = attn_inputs(S, H, q_offset=q_offset, seed=21)
    g = torch.Generator().manual_seed(21)
    edge = torch.tensor([0, 16383, 16384, 32767, 32768, s_kv - S])
    idx = torch.empty(1, S, K, dtype=torch.int32)
    for s in range(S):
        pick = torch.randperm(s + q_offset + 1, generator=g)[: 2 * K]
        pick = pick[~torch.isin(pick, edge)][: K - len(edge)]
        row = torch.cat([edge, pick])
        idx[0, s] = row[torch.randperm(K, generator=g)].int()
    out, smax, ssum, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout, scale, q_offset)
    _, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale, q_offset=q_offset)
    rdq, rdkv, _ = O.sparse_mla_bwd_closed_form(q, kv, idx, out, ref_lse, dout, scale, q_offset=q_offset)
    assert rel_err(dq, rdq) <= BF16_TOL, rel_err(dq, rdq)
    assert rel_err(dkv, rdkv) <= BF16_TOL, rel_err(dkv, rdkv)
    touched = torch.zeros(s_kv, dtype=torch.bool)
    touched[idx.flatten().long()] = True
    assert float(dkv[0, ~touched].abs().sum()) == 0.0


@pytest.mark.parametrize("s_kv", [3584, 12000])
def test_bwd_staged_pair_fill_key_ranges(s_kv):
    """Key spaces of up to four 3584-key ranges take the staged CSR fill (pairs staged per
    key in LDS and written as 32-byte sectors of the key's list): one range exactly, and
    four with a partial last one; slots at the range edges in every row."""
    S, H, K = 160, 16, 256
    q_offset = s_kv - S
    q, kv, dout, scale = attn_inputs(S, H, q_offset=q_offset, seed=23)
    g = torch.Generator().manual_seed(23)
    edge = torch.tensor([e for e in (0, 3583, 3584, 7167, 7168, 10751, 10752, s_kv - S) if e < s_kv - S + 1])
    idx = torch.empty(1, S, K, dtype=torch.int32)
    for s in range(S):
        pick = torch.randperm(s + q_offset + 1, generator=g)[: 2 * K]
        pick = pick[~torch.isin(pick, edge)][: K - len(edge)]
        idx[0, s] = torch.sort(torch.cat([edge, pick])).values.int()
    out, smax, ssum, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout, scale, q_offset)
    _, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale, q_offset=q_offset)
    rdq, rdkv, _ = O.sparse_mla_bwd_closed_form(q, kv, idx, out, ref_lse, dout, scale, q_offset=q_offset)
    assert rel_err(dq, rdq) <= BF16_TOL, rel_err(dq, rdq)
    assert rel_err(dkv, rdkv) <= BF16_TOL, rel_err(dkv, rdkv)


def test_bwd_key_repeated_inside_a_row():
    """A key selected twice by one row (never the case for top-k output) counts twice, as the
    oracle's scatter-add does: the staged CSR fill detects the repeat and the unstaged fill
    redoes the pair list."""
    S, H, K = 128, 16, 64
    q, kv, dout, scale = attn_inputs(S, H, seed=24)
    idx = rand_indices(S, K, seed=24)
    for s in (40, 77, 127):  # rows with more than K causal keys: every slot valid
        idx[0, s, 1] = idx[0, s, 0]
        idx[0, s, 9] = idx[0, s, 5]
    out, smax, ssum, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout, scale)
    _, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale)
    rdq, rdkv, _ = O.sparse_mla_bwd_closed_form(q, kv, idx, out, ref_lse, dout, scale)
    assert rel_err(dq, rdq) <= BF16_TOL, rel_err(dq, rdq)
    assert rel_err(dkv, rdkv) <= BF16_TOL, rel_err(dkv, rdkv)


def test_bwd_bf16_chunked_workspace_matches_single_pass():
    """A workspace that only fits a few query rows gives the same gradients (row chunking)."""
    S, H, K = 128, 32, 64
    q, kv, dout, scale = attn_inputs(S, H, seed=4)
    idx = rand_indices(S, K, seed=4)
    *_, dq1, dkv1 = _gpu_fwd_bwd(q, kv, idx, dout, scale)
    small = (K * (256 * 2 + 576 * 2 + 4)) * 24 + 3 * (S + 1) * 4 + 4096
    *_, dq2, dkv2 = _gpu_fwd_bwd(q, kv, idx, dout, scale, workspace_bytes=small)
    assert torch.equal(dq1, dq2)
    assert rel_err(dkv2, dkv1) <= 1e-6


@pytest.mark.parametrize("d_qk,chunk_bytes", [(576, None), (512, None), (576, 40 << 20)])
def test_bwd_dkv_is_bitwise_reproducible(d_qk, chunk_bytes):
    """dKV sums every key's contributions in a fixed order (key lists placed row by row, the
    partial sums of keys that straddle reduction segments added in segment order): three runs
    of the same backward give the same bits.  The keys' lists here (~450 pairs) all straddle
    256-pair segments; the chunked case also adds over several row chunks."""
    S, H, K = 1024, 32, 512
    q, kv, dout, scale = attn_inputs(S, H, seed=12, d_qk=d_qk)
    idx = rand_indices(S, K, seed=12, shuffle=True, holes=0.05)
    ops = _ops()
    qd, kvd, idd, dod = q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV)
    out, smax, ssum = ops.sparse_mla_fwd(qd, kvd, idd, scale)
    runs = [ops.sparse_mla_bwd(qd, kvd, idd, out, dod, smax, ssum, scale, workspace_bytes=chunk_bytes)
            for _ in range(3)]
    for dq, dkv in runs[1:]:
        assert torch.equal(dq, runs[0][0])
        assert torch.equal(dkv, runs[0][1])


def test_bwd_dense_special_case_matches_sdpa_autograd():
    S, H = 96, 32
    q, kv, dout, scale = attn_inputs(S, H, seed=6)
    idx = rand_indices(S, S, seed=6)
    _, _, _, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout, scale)
    qd = q.double().requires_grad_(True)
    kvd = kv.double().requires_grad_(True)
    k = kvd.unsqueeze(1).expand(1, H, S, 576)
    o = torch.nn.functional.scaled_dot_product_attention(qd.permute(0, 2, 1, 3), k, k[..., :512], is_causal=True,
                                                         scale=scale)
    gq, gkv = torch.autograd.grad(o.permute(0, 2, 1, 3), (qd, kvd), dout.double())
    assert rel_err(dq, gq) <= BF16_TOL and rel_err(dkv, gkv) <= BF16_TOL


def test_bwd_fp32_parity():
    S, H, K = 48, 4, 24
    q, kv, dout, scale = attn_inputs(S, H, seed=8, dtype=torch.float32)
    idx = rand_indices(S, K, seed=8)
    out, smax, ssum, dq, dkv = _gpu_fwd_bwd(q, kv, idx, dout.float(), scale)
    adq, adkv = O.sparse_mla_bwd(q, kv, idx, dout, scale)
    assert rel_err(dq, adq) <= 1e-5 and rel_err(dkv, adkv) <= 1e-5


@pytest.mark.parametrize(
    "S,H,K,q_offset,d_qk",
    [
        (200, 128, 128, 0, 576),
        (64, 16, 32, 16, 576),  # one partial head group, CP shard offset
        (80, 128, 40, 0, 576),  # top-k not a multiple of the 32-slot block
        (64, 160, 96, 0, 576),  # two head groups adding into one row
        (96, 72, 40, 8, 512),  # rope-less 512-column rows (DeepSeek-V4)
        (48, 128, 2048, 2200, 576),  # 64 blocks per row, most slots usable
    ],
)
def test_attn_mass_parity(S, H, K, q_offset, d_qk):
    q, kv, _, scale = attn_inputs(S, H, q_offset=q_offset, seed=10, d_qk=d_qk)
    idx = rand_indices(S, K, q_offset=q_offset, seed=10, holes=0.1)
    ops = _ops()
    out, smax, ssum = ops.sparse_mla_fwd(q.to(DEV), kv.to(DEV), idx.to(DEV), scale, q_offset=q_offset)
    mass = ops.attn_mass(q.to(DEV), kv.to(DEV), idx.to(DEV), smax, ssum, scale, q_offset=q_offset).cpu()
    lse = smax.cpu().double() + torch.log(ssum.cpu().double())
    ref = O.attn_mass(q, kv, idx, lse, scale, q_offset=q_offset)
    assert rel_err(mass, ref) <= 1e-4
    # each head's softmax sums to one over the selected keys
    rows = torch.isfinite(lse).all(-1)
    assert torch.allclose(mass.sum(-1)[rows].double(), torch.full_like(mass.sum(-1)[rows].double(), H), rtol=1e-3)


@pytest.mark.parametrize("d_qk", [576, 512])
def test_attn_mass_batched(d_qk):
    """Two batch elements in one call (grid z) with their own keys and indices, each against
    the oracle."""
    S, H, K = 72, 128, 48
    parts = [attn_inputs(S, H, seed=20 + i, d_qk=d_qk) for i in range(2)]
    scale = parts[0][3]
    q = torch.cat([p[0] for p in parts])
    kv = torch.cat([p[1] for p in parts])
    idx = torch.cat([rand_indices(S, K, seed=20 + i, shuffle=True, holes=0.1) for i in range(2)])
    ops = _ops()
    qd, kvd, idxd = q.to(DEV), kv.to(DEV), idx.to(DEV)
    out, smax, ssum = ops.sparse_mla_fwd(qd, kvd, idxd, scale, d_v=512)
    mass = ops.attn_mass(qd, kvd, idxd, smax, ssum, scale).cpu()
    lse = smax.cpu().double() + torch.log(ssum.cpu().double())
    for b in range(2):
        ref = O.attn_mass(q[b:b + 1], kv[b:b + 1], idx[b:b + 1], lse[b:b + 1], scale)
        assert rel_err(mass[b:b + 1], ref) <= 1e-4


@pytest.mark.parametrize("S,H,K,q_offset", [(200, 128, 128, 0), (64, 16, 32, 16), (96, 72, 40, 0)])
def test_bwd_fused_mass_matches_attn_mass(S, H, K, q_offset):
    """The mass the backward returns (one or several head groups) equals dsa_attn_mass and the oracle."""
    q, kv, dout, scale = attn_inputs(S, H, q_offset=q_offset, seed=11)
    idx = rand_indices(S, K, q_offset=q_offset, seed=11, holes=0.1)
    ops = _ops()
    qd, kvd, idxd = q.to(DEV), kv.to(DEV), idx.to(DEV)
    out, smax, ssum = ops.sparse_mla_fwd(qd, kvd, idxd, scale, q_offset=q_offset)
    dq, dkv, mass = ops.sparse_mla_bwd(qd, kvd, idxd, out, dout.to(DEV), smax, ssum, scale, q_offset=q_offset,
                                       return_mass=True)
    dq2, dkv2 = ops.sparse_mla_bwd(qd, kvd, idxd, out, dout.to(DEV), smax, ssum, scale, q_offset=q_offset)
    standalone = ops.attn_mass(qd, kvd, idxd, smax, ssum, scale, q_offset=q_offset)
    torch.cuda.synchronize()
    assert torch.equal(dq.cpu(), dq2.cpu())
    lse = smax.cpu().double() + torch.log(ssum.cpu().double())
    ref = O.attn_mass(q, kv, idx, lse, scale, q_offset=q_offset)
    assert rel_err(mass.cpu(), ref) <= 1e-4
    assert rel_err(mass.cpu(), standalone.cpu()) <= 1e-4
    assert float(mass.cpu()[idx < 0].abs().sum()) == 0.0


@pytest.mark.parametrize("d_qk,s_kv_extra", [(576, 0), (512, 96)])
def test_shared_pair_csr_matches_per_op_builds(d_qk, s_kv_extra):
    """The attention backward and the indexer KL op reduce with one key-major pair CSR built
    once per index tensor (dsa_pair_csr_build): the KL op reuses the backward's (no second
    build) and both results are bit-identical to each op building its own CSR inside the
    library call (the same list order and segment sums)."""
    S, H, K, HI, DI = 768, 32, 256, 64, 128
    q, kv, dout, scale = attn_inputs(S, H, seed=21, d_qk=d_qk, q_offset=s_kv_extra)
    idx = rand_indices(S, K, q_offset=s_kv_extra, seed=21, holes=0.05)
    g = torch.Generator().manual_seed(22)
    s_k = S + s_kv_extra
    qi = torch.randn(1, S, HI, DI, generator=g).bfloat16().to(DEV)
    ki = torch.randn(1, s_k, DI, generator=g).bfloat16().to(DEV)
    w = (torch.rand(1, S, HI, generator=g) * HI ** -0.5 * DI ** -0.5).to(DEV)
    ops = _ops()
    qd, kvd, idd, dod = q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV)
    out, smax, ssum = ops.sparse_mla_fwd(qd, kvd, idd, scale, q_offset=s_kv_extra)

    def step():
        dq, dkv, mass = ops.sparse_mla_bwd(qd, kvd, idd, out, dod, smax, ssum, scale, q_offset=s_kv_extra,
                                           return_mass=True)
        built = ops._pair_csr_entry
        kl = ops.indexer_kl_grad_from_mass(qi, ki, w, idd, mass, q_offset=s_kv_extra)
        return (dq, dkv, mass) + tuple(kl), built

    ops._pair_csr_entry = None
    shared, built = step()
    assert built is not None and ops._pair_csr_entry is built  # the KL op found the backward's CSR
    try:
        ops._share_pair_csr = False
        ops._pair_csr_entry = None
        own, none = step()
        assert none is None and ops._pair_csr_entry is None
    finally:
        ops._share_pair_csr = True
    for a, b in zip(shared, own):
        assert torch.equal(a, b)


@pytest.mark.parametrize(
    "S,K,s_kv,windows",
    [
        # 512-row counting blocks, four 16384-key ranges: block b keeps to range b % 3
        (3000, 64, 50000, [(100, 2100), (16484, 18484), (32868, 34868)]),
        # 78-row blocks (34 of them: two column-scan chunks of 32), two ranges: even blocks in
        # range 0, odd blocks in range 1
        (2600, 1024, 20000, [(100, 8000), (16500, 19900)]),
    ],
)
def test_bwd_pair_fill_row_blocks_without_keys_in_a_range(S, K, s_kv, windows):
    """Key spaces past 14336 keys take the unstaged CSR fill, which skips the (row block,
    16384-key range) pairs that hold no pair.  Here every counting row block keeps its slots
    inside one range, so most pairs are skipped, including blocks next to a column-scan chunk
    edge: dQ and dKV equal the fp32 GPU reference (dKV per 256-key block), keys no row selects
    stay exactly zero, and a second run gives the same bits."""
    from tests.attn_reference import attention_reference, chunk_rel_errors

    H = 16
    q_offset = s_kv - S
    rows_per_block = max(16, min(512, 4 * s_kv // K))  # the counting workgroup's rows
    q, kv, dout, scale = attn_inputs(S, H, q_offset=q_offset, seed=45)
    g = torch.Generator().manual_seed(45)
    idx = torch.empty(1, S, K, dtype=torch.int32)
    for s in range(S):
        lo, hi = windows[(s // rows_per_block) % len(windows)]
        idx[0, s] = torch.sort(lo + torch.randperm(hi - lo, generator=g)[:K]).values.int()
    idx[0, ::7, ::5] = -1
    runs = [_gpu_fwd_bwd(q, kv, idx, dout, scale, q_offset) for _ in range(2)]
    out, _, _, dq, dkv = runs[0]
    assert torch.equal(runs[1][4], dkv) and torch.equal(runs[1][3], dq)
    ref = attention_reference(q.to(DEV), kv.to(DEV), idx.to(DEV), dout.to(DEV), scale, q_offset=q_offset)
    assert rel_err(dq, ref["dq"].cpu()) <= BF16_TOL, rel_err(dq, ref["dq"].cpu())
    e = chunk_rel_errors(dkv[0], ref["dkv"].cpu(), 256)
    assert float(e.max()) <= BF16_TOL, float(e.max())
    touched = torch.zeros(s_kv, dtype=torch.bool)
    sel = idx.flatten().long()
    touched[sel[sel >= 0]] = True
    assert float(dkv[0, ~touched].abs().sum()) == 0.0
