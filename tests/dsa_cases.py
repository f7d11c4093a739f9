"""Seeded input builders shared by the parity tests (CPU tensors; tests move them to the GPU)."""

from __future__ import annotations

import math

import torch


def rand_indices(S, K, *, q_offset=0, s_kv=None, seed=0, shuffle=False, holes=0.0, pad_invalid=True):
    """int32 [1,S,K]: per row, distinct causal keys t <= s + q_offset (ascending unless shuffle), -1 padded.

    holes: fraction of slots replaced by -1 anywhere in the row (tests arbitrary padding).
    pad_invalid: when False, rows with fewer than K causal keys repeat nothing and pad with -1 anyway.
    """
    g = torch.Generator().manual_seed(seed)
    s_kv = S + q_offset if s_kv is None else s_kv
    out = torch.full((1, S, K), -1, dtype=torch.int32)
    for s in range(S):
        lim = min(s + q_offset + 1, s_kv)
        c = min(K, lim)
        if c <= 0:
            continue
        sel = torch.randperm(lim, generator=g)[:c]
        if not shuffle:
            sel = torch.sort(sel).values
        row = torch.full((K,), -1, dtype=torch.int32)
        row[:c] = sel.to(torch.int32)
        if shuffle:
            row = row[torch.randperm(K, generator=g)]
        if holes > 0:
            m = torch.rand(K, generator=g) < holes
            row[m] = -1
        out[0, s] = row
    return out


def attn_inputs(S, H, *, s_kv=None, q_offset=0, seed=0, dtype=torch.bfloat16, d_qk=576, logit_std=1.0):
    """q [1,S,H,d_qk], kv [1,S_kv,d_qk], dout [1,S,H,512] ~ N(0,1), seeded; scale gives logit std ~ logit_std."""
    g = torch.Generator().manual_seed(seed)
    s_kv = S + q_offset if s_kv is None else s_kv
    q = torch.randn(1, S, H, d_qk, generator=g).to(dtype)
    kv = torch.randn(1, s_kv, d_qk, generator=g).to(dtype)
    dout = torch.randn(1, S, H, 512, generator=g).to(dtype)
    scale = logit_std / math.sqrt(d_qk)
    return q, kv, dout, scale


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))
