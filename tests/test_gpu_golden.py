"""HIP path against the committed golden fixtures (tests/golden/*.npz, written by the oracle).

The fixture inputs are bf16-exact, so the fp32 path is held to 1e-5 relative error and
the bf16 path to 2e-2; top-k indices are compared bit for bit.  The indexer KL gradients
take bf16 indexer inputs and round E = g w [S > 0] to bf16, hence 1e-2 for them.
"""

import pytest
import torch

from tests.dsa_cases import rel_err
from tests.golden.make_golden import CASES, load

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
FP32_TOL = 1e-5
BF16_TOL = 2e-2


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_indexer_and_topk(name):
    meta, z = load(name)
    ops = _ops()
    qo, K = meta["q_offset"], meta["K"]
    sc = ops.indexer_scores(z["q_idx"].to(DEV), z["k_idx"].to(DEV), z["w"].to(DEV), q_offset=qo).cpu()
    ref = z["scores"]
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(sc))
    assert rel_err(sc[fin], ref[fin]) <= FP32_TOL
    # selection is a pure function of the fp32 scores: bit-exact on the fixture's scores
    idx, _ = ops.topk_select(ref.to(DEV), K, q_offset=qo)
    assert torch.equal(idx.cpu(), z["indices"])


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("dtype,tol", [(torch.float32, FP32_TOL), (torch.bfloat16, BF16_TOL)])
def test_golden_attention_fwd_bwd(name, dtype, tol):
    meta, z = load(name)
    ops = _ops()
    qo, scale = meta["q_offset"], meta["scale"]
    q, kv, dout = (z[k].to(dtype).to(DEV) for k in ("q", "kv", "dout"))
    idx = z["indices"].to(DEV)
    out, smax, ssum = ops.sparse_mla_fwd(q, kv, idx, scale, q_offset=qo)
    dq, dkv = ops.sparse_mla_bwd(q, kv, idx, out, dout, smax, ssum, scale, q_offset=qo)
    mass = ops.attn_mass(q, kv, idx, smax, ssum, scale, q_offset=qo)
    torch.cuda.synchronize()
    lse = (smax.double() + torch.log(ssum.double())).cpu()
    assert rel_err(out.cpu(), z["out"]) <= tol
    assert rel_err(lse, z["lse"]) <= tol
    assert rel_err(dq.cpu(), z["dq"]) <= tol
    assert rel_err(dkv.cpu(), z["dkv"]) <= tol
    assert rel_err(mass.cpu(), z["mass"]) <= tol


@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_indexer_kl(name):
    meta, z = load(name)
    ops = _ops()
    dq, dk, dw, loss_rows = ops.indexer_kl_grad_from_mass(
        z["q_idx"].to(DEV), z["k_idx"].to(DEV), z["w"].to(DEV), z["indices"].to(DEV), z["mass"].to(DEV),
        q_offset=meta["q_offset"], loss_scale=meta["loss_scale"], eps=meta["eps"])
    torch.cuda.synchronize()
    loss = float(loss_rows.double().sum())
    ref = float(z["loss"][0])
    assert abs(loss - ref) <= 1e-4 * abs(ref)
    assert rel_err(dq.cpu(), z["dq_idx"]) <= 1e-2
    assert rel_err(dk.cpu(), z["dk_idx"]) <= 1e-2
    assert rel_err(dw.cpu(), z["dw"]) <= 1e-2
