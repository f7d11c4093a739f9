"""Packed varlen ("TND") metadata, CP shard geometry and the oracle's TND compressor (CPU).

Known answers are the reference's own (tests/unit_tests/models/test_deepseek_v4_tnd.py
:65-79 for the block starts / max lengths, :140-165 for cu_seqlens_q of a packed pair of
requests); everything else is checked against brute-force loops over the tokens.
"""

from __future__ import annotations

import random
from types import SimpleNamespace

import pytest
import torch

from oracle import dsa_oracle as O
from torchtitan_npu_simulator_amd import tnd
from torchtitan_npu_simulator_amd.torch_npu_ops import to_cu_seqlens


def _args(ratios=(4, 128), mtp_ratio=1, n_mtp=0, use_global_tnd=True):
    return SimpleNamespace(compress_ratios=ratios, mtp_layer_compress_ratio=mtp_ratio, num_mtp_modules=n_mtp,
                           use_global_tnd=use_global_tnd)


def test_reference_known_answers_block_starts():
    m = tnd.build_smla_attention_masks(torch.tensor([0, 1, 2, 3, 0, 1, 2, 3]), _args())
    torch.testing.assert_close(m.block_starts_by_ratio[4], torch.tensor([0, 4]))
    assert m.block_starts_by_ratio[128].numel() == 0
    assert m.max_seqlen_q == 4
    assert m.max_seqlen_cmp_kv == {4: 1, 128: 0}


def test_reference_known_answer_cu_seqlens_q():
    # the packed positions of the reference's MTP test after dropping 2 MTP tokens
    m = tnd.build_smla_attention_masks(torch.tensor([0, 1, 2, 3, 0, 1], dtype=torch.int32), _args((1,)))
    torch.testing.assert_close(m.cu_seqlens_q, torch.tensor([0, 4, 6], dtype=torch.int32))
    torch.testing.assert_close(m.cu_seqlens_ori_kv, torch.tensor([0, 4, 6], dtype=torch.int32))
    assert m.batch_size == 2 and m.seq_len == 6
    assert m.cu_seqlens_cmp_kv == {} and m.block_starts_by_ratio == {}


def test_lengths_to_cu_seqlens_matches_oracle():
    for lengths in ([3, 0, 5], [1], [7, 7, 2, 9]):
        t = torch.tensor(lengths, dtype=torch.int32)
        torch.testing.assert_close(tnd.lengths_to_cu_seqlens(t), O.lengths_to_cu_seqlens(t))


def _random_positions(rng, n_req, max_len):
    pos = []
    for _ in range(n_req):
        pos.extend(range(rng.randint(1, max_len)))
    return torch.tensor(pos)


def _brute_block_starts(pos, r):
    p = pos.tolist()
    return [i for i in range(len(p)) if p[i] % r == 0 and i + r - 1 < len(p) and p[i + r - 1] == p[i] + r - 1]


@pytest.mark.parametrize("seed", range(6))
def test_block_starts_and_lengths_brute_force(seed):
    rng = random.Random(seed)
    pos = _random_positions(rng, rng.randint(1, 6), 40)
    m = tnd.build_smla_attention_masks(pos, _args((4, 8), mtp_ratio=16))
    p = pos.tolist()
    starts = [0] + [i for i in range(1, len(p)) if p[i] == 0]
    ends = starts[1:] + [len(p)]
    lengths = [e - s for s, e in zip(starts, ends)]
    assert m.cu_seqlens_q.tolist() == [0] + list(torch.tensor(lengths).cumsum(0).tolist())
    assert m.max_seqlen_q == max(lengths)
    for r in (4, 8, 16):
        bs = _brute_block_starts(pos, r)
        assert m.block_starts_by_ratio[r].tolist() == bs
        torch.testing.assert_close(m.block_starts_by_ratio[r], O.tnd_compressed_block_starts(pos, r))
        counts = [sum(1 for b in bs if s <= b < e) for s, e in zip(starts, ends)]
        assert m.cu_seqlens_cmp_kv[r].tolist() == [0] + list(torch.tensor(counts).cumsum(0).tolist())
        assert m.cmp_residual_k[r].tolist() == [l - r * c for l, c in zip(lengths, counts)]
        assert m.max_seqlen_cmp_kv[r] == max(counts)


def test_batched_positions_without_tnd_metadata():
    pos = torch.tensor([[0, 1, 2, 3, 4, 5, -1, -1, 9], [0, 1, 2, 3, 4, 5, 6, 7, 9]])
    m = tnd.build_smla_attention_masks(pos, _args((4,), n_mtp=1), use_tnd_metadata=False)
    assert m.cu_seqlens_q.tolist() == [0, 6, 14]
    assert m.cu_seqlens_cmp_kv[4].tolist() == [0, 1, 3]
    assert m.cmp_residual_k[4].tolist() == [2, 0]
    assert m.block_starts_by_ratio == {} and m.seq_len == 8


def test_padding_rules_and_errors():
    # padding after the valid tokens is dropped; the MTP column is not part of the sequence
    m = tnd.build_smla_attention_masks(torch.tensor([[0, 1, 2, 0, 1, -1, 7]]), _args((1,), n_mtp=1))
    assert m.cu_seqlens_q.tolist() == [0, 3, 5]
    with pytest.raises(ValueError, match="padding must come after"):
        tnd.build_smla_attention_masks(torch.tensor([[0, 1, -1, 3]]), _args((1,)))
    with pytest.raises(ValueError, match="no entry is a valid"):
        tnd.build_smla_attention_masks(torch.tensor([[-1, -1, 5]]), _args((1,), n_mtp=1))
    with pytest.raises(ValueError, match="rows for an input batch"):
        tnd.build_smla_attention_masks(torch.zeros(2, 4, dtype=torch.long), _args((1,)), batch_size=3)
    # a first request that does not start at position 0 still starts a sequence
    m = tnd.build_smla_attention_masks(torch.tensor([5, 6, 7, 0, 1]), _args((4,)))
    assert m.cu_seqlens_q.tolist() == [0, 3, 5]


def test_cp_shard_geometry():
    world, s_loc = 4, 96
    covered = []
    for r in range(world):
        sh = tnd.cp_shard(r, world, s_loc)
        covered.extend(range(*sh.q_rows))
        assert sh.kv_len == sh.q_rows[1]
        # bottom-right causal alignment of the shard == its first row's absolute position
        assert sh.q_offset == sh.kv_len - (sh.q_rows[1] - sh.q_rows[0]) == sh.q_rows[0]
    assert covered == list(range(world * s_loc))
    with pytest.raises(ValueError):
        tnd.cp_shard(4, 4, 8)


def test_to_cu_seqlens_conventions():
    assert to_cu_seqlens(actual_seq_lengths=[4, 6], total=6) == [0, 4, 6]
    assert to_cu_seqlens(cu_seqlens=torch.tensor([0, 4, 6]), total=6) == [0, 4, 6]
    with pytest.raises(ValueError):
        to_cu_seqlens(actual_seq_lengths=[4, 6], total=7)
    with pytest.raises(ValueError):
        to_cu_seqlens(cu_seqlens=[1, 4])
    with pytest.raises(ValueError):
        to_cu_seqlens(actual_seq_lengths=[4, 3])


# ----- oracle TND compressor pins -----
def _proj(T, D, r, overlap, seed):
    g = torch.Generator().manual_seed(seed)
    coff = 2 if overlap else 1
    return (torch.randn(T, coff * D, generator=g, dtype=torch.float64),
            torch.randn(T, coff * D, generator=g, dtype=torch.float64),
            torch.randn(r, coff * D, generator=g, dtype=torch.float64) * 0.1)


@pytest.mark.parametrize("r,overlap", [(4, True), (8, False)])
def test_oracle_tnd_compressor_single_request_is_bsnd(r, overlap):
    T, D = 6 * r, 16
    kv, sc, ape = _proj(T, D, r, overlap, seed=r)
    pos = torch.arange(T)
    bs = O.tnd_compressed_block_starts(pos, r)
    got = O.compressor_pool_tnd(kv, sc, ape, r, bs, pos, overlap=overlap)
    ref = O.compressor_pool(kv.unsqueeze(0), sc.unsqueeze(0), ape, r, overlap=overlap)[0]
    torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)


def test_oracle_tnd_compressor_requests_are_independent():
    r, D = 4, 8
    lens = [12, 8, 16]
    T = sum(lens)
    kv, sc, ape = _proj(T, D, r, True, seed=11)
    pos = torch.cat([torch.arange(n) for n in lens])
    bs = O.tnd_compressed_block_starts(pos, r)
    got = O.compressor_pool_tnd(kv, sc, ape, r, bs, pos)
    parts, t0 = [], 0
    for n in lens:
        parts.append(O.compressor_pool(kv[t0:t0 + n].unsqueeze(0), sc[t0:t0 + n].unsqueeze(0), ape, r)[0])
        t0 += n
    torch.testing.assert_close(got, torch.cat(parts), rtol=1e-12, atol=1e-12)
