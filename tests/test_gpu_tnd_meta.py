"""The device-side TND metadata builder (dsa_tnd_metadata) against the host builder
``tnd.build_smla_attention_masks`` (itself pinned by the reference's known answers in
tests/test_tnd.py): the same request boundaries, block starts, compressed lengths,
residuals and maxima, exactly, on packed and [B, S] positions with padding and MTP
columns; building it issues no device-to-host read (only ``host()`` reads back)."""

from types import SimpleNamespace

import pytest
import torch

from torchtitan_npu_simulator_amd import tnd

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _args(ratios=(4, 128), mtp_ratio=4, n_mtp=0):
    return SimpleNamespace(compress_ratios=list(ratios), mtp_layer_compress_ratio=mtp_ratio, num_mtp_modules=n_mtp,
                           use_global_tnd=True)


def _packed_positions(lengths, first_offset=0):
    parts = [torch.arange(first_offset, first_offset + lengths[0])] + [torch.arange(n) for n in lengths[1:]]
    return torch.cat(parts)


def _same(dev_masks, host_masks):
    assert torch.equal(dev_masks.cu_seqlens_q.cpu().long(), host_masks.cu_seqlens_q.cpu().long())
    assert torch.equal(dev_masks.cu_seqlens_ori_kv.cpu().long(), host_masks.cu_seqlens_ori_kv.cpu().long())
    assert dev_masks.max_seqlen_q == host_masks.max_seqlen_q and dev_masks.batch_size == host_masks.batch_size
    assert dev_masks.seq_len == host_masks.seq_len
    for r in host_masks.cu_seqlens_cmp_kv:
        assert torch.equal(dev_masks.cu_seqlens_cmp_kv[r].cpu().long(), host_masks.cu_seqlens_cmp_kv[r].cpu().long())
        assert torch.equal(dev_masks.cmp_residual_k[r].cpu().long(), host_masks.cmp_residual_k[r].cpu().long())
        assert torch.equal(dev_masks.block_starts_by_ratio[r].cpu(), host_masks.block_starts_by_ratio[r].cpu())
        assert dev_masks.max_seqlen_cmp_kv[r] == host_masks.max_seqlen_cmp_kv[r]


@pytest.mark.parametrize("lengths,first_offset", [([37, 130, 1, 256, 3], 0), ([5000, 12345, 8, 700], 13),
                                                  ([1], 0), ([2048] * 6, 0)])
def test_device_metadata_packed(lengths, first_offset):
    pos = _packed_positions(lengths, first_offset).to(DEV)
    args = _args()
    meta = tnd.build_smla_attention_masks_device(pos, args)
    _same(meta.host(), tnd.build_smla_attention_masks(pos, args))
    assert meta.host() is meta.host()  # read back once


def test_device_metadata_batch_rows_with_padding_and_mtp():
    args = _args(ratios=(4,), n_mtp=1)
    g = torch.Generator().manual_seed(3)
    rows = []
    for b in range(3):
        seg = _packed_positions([int(x) for x in torch.randint(1, 40, (3,), generator=g)])
        rows.append(seg)
    width = 1 + max(len(r) for r in rows) + 5
    pos = torch.full((3, width), -1, dtype=torch.long)
    for b, r in enumerate(rows):
        pos[b, : len(r)] = r
    pos[2, :] = torch.arange(width)  # a full last row: padding only ends rows 0-1 ... invalid order
    flat_ok = torch.full((3, width), -1, dtype=torch.long)
    flat_ok[0, :width - 1] = torch.arange(width - 1)
    flat_ok[1, :7] = torch.arange(7)  # padding only after the last valid token in row-major order
    for p in (flat_ok,):
        meta = tnd.build_smla_attention_masks_device(p.to(DEV), args)
        _same(meta.host(), tnd.build_smla_attention_masks(p.to(DEV), args))
    bad = tnd.build_smla_attention_masks_device(pos.to(DEV), args)
    with pytest.raises(ValueError, match="padding must come after"):
        bad.host()


def test_device_metadata_reference_known_answers():
    """The device builder on the reference's own known-answer inputs
    (tests/unit_tests/models/test_deepseek_v4_tnd.py:65-79 and :140-165), checked against
    those answers directly rather than through the host builder."""
    meta = tnd.build_smla_attention_masks_device(torch.tensor([0, 1, 2, 3, 0, 1, 2, 3], device=DEV),
                                                 _args(ratios=(4, 128), mtp_ratio=1)).host()
    torch.testing.assert_close(meta.block_starts_by_ratio[4].cpu().long(), torch.tensor([0, 4]))
    assert meta.block_starts_by_ratio[128].numel() == 0
    assert meta.max_seqlen_q == 4
    assert meta.max_seqlen_cmp_kv == {4: 1, 128: 0}

    meta = tnd.build_smla_attention_masks_device(torch.tensor([0, 1, 2, 3, 0, 1], dtype=torch.int32, device=DEV),
                                                 _args(ratios=(1,), mtp_ratio=1)).host()
    torch.testing.assert_close(meta.cu_seqlens_q.cpu().long(), torch.tensor([0, 4, 6]))
    torch.testing.assert_close(meta.cu_seqlens_ori_kv.cpu().long(), torch.tensor([0, 4, 6]))
    assert meta.batch_size == 2 and meta.seq_len == 6
