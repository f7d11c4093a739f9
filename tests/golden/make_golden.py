"""Writes the committed golden fixtures of the DSA path from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no numeric known answers for this path (its tests mock the
fused ops), so the fixtures are the oracle's outputs on seeded inputs of the
BASELINE config-1 family at reduced size.  Inputs are stored as bf16 bit
patterns so that the fp32 and bf16 HIP paths see identical values; outputs are
fp32 (computed in fp64).  The pipeline mirrors converters/kernels/dsa.py:195-277
(indexer -> top-k -> sparse flash attention) and :140-192 (KL loss in backward).
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import dsa_oracle as O  # noqa: E402

CASES = {
    # config-1 family: 576/512 MLA, indexer 4 heads x 64, causal top-k
    "dsa_c1_tiny": dict(S=32, H=2, H_I=4, D_I=64, K=16, q_offset=0, seed=0),
    # one context-parallel shard: 24 query rows after a 16-token prefix
    "dsa_c1_shard": dict(S=24, H=2, H_I=4, D_I=64, K=12, q_offset=16, seed=1),
}


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).float()


def make_case(S, H, H_I, D_I, K, q_offset, seed):
    g = torch.Generator().manual_seed(seed)
    s_kv = S + q_offset
    q = torch.randn(1, S, H, 576, generator=g) / math.sqrt(576)
    kv = torch.randn(1, s_kv, 576, generator=g)
    q_idx = torch.randn(1, S, H_I, D_I, generator=g)
    k_idx = torch.randn(1, s_kv, D_I, generator=g)
    w = torch.rand(1, S, H_I, generator=g) * (H_I ** -0.5) * (D_I ** -0.5)
    dout = torch.randn(1, S, H, 512, generator=g)
    raw = dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, dout=dout)
    bits = {k: bf16_bits(v) for k, v in raw.items()}
    x = {k: from_bits(v) for k, v in bits.items()}  # bf16-exact fp32 values
    scale = 576 ** -0.5

    scores = O.indexer_scores(x["q_idx"], x["k_idx"], w, q_offset=q_offset)
    idx = O.topk_select(scores, K, q_offset=q_offset)
    out, lse = O.sparse_mla_fwd(x["q"], x["kv"], idx, scale, q_offset=q_offset)
    dq, dkv = O.sparse_mla_bwd(x["q"], x["kv"], idx, x["dout"], scale, q_offset=q_offset)
    mass = O.attn_mass(x["q"], x["kv"], idx, lse, scale, q_offset=q_offset)
    dqi, dki, dw, loss = O.indexer_kl_from_mass(x["q_idx"], x["k_idx"], w, idx, mass, q_offset=q_offset)

    arrays = {f"{k}_bf16": v for k, v in bits.items()}
    arrays.update(
        w=w.numpy().astype(np.float32),
        scores=scores.numpy().astype(np.float32),
        indices=idx.numpy().astype(np.int32),
        out=out.float().numpy(),
        lse=lse.float().numpy(),
        dq=dq.float().numpy(),
        dkv=dkv.float().numpy(),
        mass=mass.float().numpy(),
        dq_idx=dqi.float().numpy(),
        dk_idx=dki.float().numpy(),
        dw=dw.float().numpy(),
        loss=np.array([float(loss)], dtype=np.float64),
    )
    meta = dict(S=S, H=H, H_I=H_I, D_I=D_I, K=K, q_offset=q_offset, seed=seed, d_qk=576, d_v=512, scale=scale,
                loss_scale=1.0, eps=1e-8,
                note="q is N(0,1)/sqrt(576); w ~ U(0,1)*H_I^-0.5*D_I^-0.5; inputs rounded to bf16")
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    return arrays


def load(name):
    """Returns (meta dict, arrays dict with bf16 inputs decoded to fp32 tensors)."""
    z = np.load(os.path.join(HERE, name + ".npz"))
    meta = json.loads(bytes(z["meta"]).decode())
    out = {}
    for k in z.files:
        if k == "meta":
            continue
        if k.endswith("_bf16"):
            out[k[:-5]] = from_bits(z[k])
        else:
            out[k] = torch.from_numpy(z[k])
    return meta, out


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    for name, cfg in CASES.items():
        arrays = make_case(**cfg)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
        print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
