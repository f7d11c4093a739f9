"""Parity of dsa_sparse_mla_fwd (HIP) against the CPU oracle on seeded inputs.

Tolerances (from the task contract): relative error <= 2e-2 in bf16, <= 1e-5 in fp32,
measured as ||gpu - oracle|| / ||oracle|| over the whole output.
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import attn_inputs, rand_indices, rel_err

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
FP32_TOL = 1e-5


def _run(q, kv, idx, scale, q_offset=0):
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    dev = torch.device("cuda:0")
    out, smax, ssum = ops.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev), scale, q_offset=q_offset)
    torch.cuda.synchronize()
    return out.cpu(), smax.cpu(), ssum.cpu()


def _check(q, kv, idx, scale, q_offset, tol):
    out, smax, ssum = _run(q, kv, idx, scale, q_offset)
    ref_out, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale, q_offset=q_offset)
    assert rel_err(out, ref_out) <= tol, rel_err(out, ref_out)
    lse = smax.double() + torch.log(ssum.double())
    fin = torch.isfinite(ref_lse)
    assert torch.equal(fin, torch.isfinite(lse))
    assert (lse[fin] - ref_lse[fin]).abs().max() <= 10 * tol
    # softmax_max is the true max of the scaled logits
    assert torch.all(ssum[fin] >= 1.0 - 1e-3)


@pytest.mark.parametrize(
    "S,H,K,q_offset,seed",
    [
        (512, 16, 64, 0, 0),  # config-1 attention shape (16 heads, K=64), bf16
        (256, 128, 128, 0, 1),
        (192, 128, 256, 64, 2),  # one CP shard: rows start at 64 against a 256-key prefix
        (96, 40, 48, 0, 3),  # head count not a multiple of 32
    ],
)
def test_fwd_bf16_parity(S, H, K, q_offset, seed):
    q, kv, _, scale = attn_inputs(S, H, q_offset=q_offset, seed=seed)
    idx = rand_indices(S, K, q_offset=q_offset, seed=seed)
    _check(q, kv, idx, scale, q_offset, BF16_TOL)


@pytest.mark.parametrize(
    "S,H,K,q_offset,seed,holes",
    [
        (256, 128, 128, 0, 21, 0.0),
        (160, 64, 96, 32, 22, 0.2),  # -1 holes, CP shard offset
        (96, 40, 48, 0, 23, 0.0),  # head count not a multiple of 32
    ],
)
def test_fwd_bf16_rows_of_512_columns(S, H, K, q_offset, seed, holes):
    """The rope-less variant (DeepSeek-V4 rows): d_qk = d_v = 512, v = the whole key row."""
    q, kv, _, scale = attn_inputs(S, H, q_offset=q_offset, seed=seed, d_qk=512)
    idx = rand_indices(S, K, q_offset=q_offset, seed=seed, shuffle=True, holes=holes)
    _check(q, kv, idx, scale, q_offset, BF16_TOL)


def test_fwd_bf16_shuffled_slots_and_holes():
    S, H, K = 160, 128, 96
    q, kv, _, scale = attn_inputs(S, H, seed=7, logit_std=3.0)
    idx = rand_indices(S, K, seed=7, shuffle=True, holes=0.2)
    _check(q, kv, idx, scale, 0, BF16_TOL)


def test_fwd_bf16_rows_without_keys():
    S, H, K = 64, 32, 32
    q, kv, _, scale = attn_inputs(S, H, seed=5)
    idx = rand_indices(S, K, seed=5)
    idx[0, ::3] = -1  # every third row has no usable key
    out, smax, ssum = _run(q, kv, idx, scale)
    assert torch.all(out[0, ::3] == 0)
    assert torch.all(torch.isneginf(smax[0, ::3])) and torch.all(ssum[0, ::3] == 0)
    ref_out, _ = O.sparse_mla_fwd(q, kv, idx, scale)
    assert rel_err(out, ref_out) <= BF16_TOL


def test_fwd_bf16_large_logit_range_uses_fixup():
    """Logits growing by far more than the 2^64 headroom after the first block are recomputed exactly."""
    S, H, K = 64, 32, 64
    q, kv, _, scale = attn_inputs(S, H, seed=9)
    kv = kv.float()
    kv[0, 40:] *= 40.0  # later keys dominate by ~e^100
    kv = kv.to(torch.bfloat16)
    idx = rand_indices(S, K, seed=9)
    _check(q, kv, idx, scale, 0, BF16_TOL)


def test_fwd_dense_special_case_matches_sdpa():
    """K >= #valid keys reduces to dense causal SDPA (a library routine)."""
    S, H = 128, 32
    q, kv, _, scale = attn_inputs(S, H, seed=11)
    idx = rand_indices(S, S, seed=11)  # every causal key
    out, _, _ = _run(q, kv, idx, scale)
    qd = q.double().permute(0, 2, 1, 3)
    kd = kv.double().unsqueeze(1).expand(1, H, S, 576)
    vd = kd[..., :512]
    ref = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd, is_causal=True, scale=scale)
    assert rel_err(out, ref.permute(0, 2, 1, 3)) <= BF16_TOL


@pytest.mark.parametrize("S,H,K,dqk,dv", [(64, 4, 16, 576, 512), (48, 3, 24, 96, 64)])
def test_fwd_fp32_parity(S, H, K, dqk, dv):
    q, kv, _, scale = attn_inputs(S, H, seed=13, dtype=torch.float32, d_qk=dqk)
    idx = rand_indices(S, K, seed=13)
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    dev = torch.device("cuda:0")
    out, smax, ssum = ops.sparse_mla_fwd(q.to(dev), kv.to(dev), idx.to(dev), scale, d_v=dv)
    ref_out, ref_lse = O.sparse_mla_fwd(q, kv, idx, scale, d_v=dv)
    assert rel_err(out.cpu(), ref_out) <= FP32_TOL
    lse = smax.cpu().double() + torch.log(ssum.cpu().double())
    assert (lse - ref_lse).abs().max() <= 1e-5
