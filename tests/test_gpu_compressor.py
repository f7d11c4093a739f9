"""Parity of dsa_compressor_fwd (HIP) with the oracle's compressor_pool.

fp32 pooling: 1e-5 relative; RMSNorm epilogue written as bf16: 2e-2.  Shapes cover the
reference's ratios (4 with overlap, 128 without; model.py:150) and head dims 512 / 128.
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _inputs(B, S, D, r, overlap, seed, ape_std=0.02):
    g = torch.Generator().manual_seed(seed)
    coff = 2 if overlap else 1
    kv = torch.randn(B, S, coff * D, generator=g)
    score = torch.randn(B, S, coff * D, generator=g)
    ape = torch.randn(r, coff * D, generator=g) * ape_std
    return kv, score, ape


@pytest.mark.parametrize("B,S,D,r,overlap", [(1, 64, 512, 4, True), (2, 48, 128, 4, True), (1, 256, 512, 128, False),
                                             (1, 40, 128, 1, False), (1, 96, 64, 3, False), (1, 12, 1024, 4, True)])
def test_compressor_pool_parity(B, S, D, r, overlap):
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    kv, score, ape = _inputs(B, S, D, r, overlap, seed=S + D + r)
    got = ops.compressor_pool(kv.to(DEV), score.to(DEV), ape.to(DEV), r, overlap=overlap).cpu()
    ref = O.compressor_pool(kv.double(), score.double(), ape.double(), r, overlap=overlap)
    assert got.shape == (B, S // r, D)
    assert rel_err(got, ref) <= 1e-5


@pytest.mark.parametrize("D,r,overlap", [(512, 4, True), (128, 4, True), (512, 128, False)])
def test_compressor_rmsnorm_epilogue(D, r, overlap):
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    S = 4 * r
    kv, score, ape = _inputs(1, S, D, r, overlap, seed=D + r)
    w = torch.rand(D, generator=torch.Generator().manual_seed(7)) + 0.5
    got = ops.compressor_pool(kv.to(DEV), score.to(DEV), ape.to(DEV), r, overlap=overlap, norm_weight=w.to(DEV),
                              norm_eps=1e-6).cpu()
    assert got.dtype == torch.bfloat16
    ref = O.compressor_pool(kv, score, ape, r, overlap=overlap, norm_weight=w, norm_eps=1e-6,
                            out_dtype=torch.bfloat16)
    assert rel_err(got.float(), ref) <= 2e-2


def test_compressor_uniform_gates_is_mean_on_gpu():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    kv = torch.randn(1, 32, 256, generator=torch.Generator().manual_seed(3))
    got = ops.compressor_pool(kv.to(DEV), torch.zeros_like(kv).to(DEV), torch.zeros(4, 256).to(DEV), 4,
                              overlap=False).cpu()
    torch.testing.assert_close(got, kv.view(1, 8, 4, 256).mean(2), rtol=1e-6, atol=1e-6)


def test_compressor_rejects_bad_shapes():
    from torchtitan_npu_simulator_amd import DSAError
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    kv = torch.randn(1, 10, 128, device=DEV)
    with pytest.raises(DSAError):
        ops.compressor_pool(kv, kv, torch.zeros(4, 128, device=DEV), 4, overlap=False)  # 10 % 4 != 0
    kv = torch.randn(1, 8, 96, device=DEV)
    with pytest.raises(DSAError):
        ops.compressor_pool(kv, kv, torch.zeros(4, 96, device=DEV), 4, overlap=False)  # D not a power of two
