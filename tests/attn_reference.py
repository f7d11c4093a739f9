"""Full-output fp32 reference of the gathered attention on the GPU (test infrastructure).

A plain PyTorch fp32 restatement of the gathered sparse attention forward and backward -
``O = softmax(scale q K_sel^T) V_sel`` per (row, head), with an optional per-head sink logit
in the softmax that carries no value, and its gradients in closed form - run over the rows
in chunks so every row and every key of a full-size configuration can be compared with the
HIP kernels, not only sampled ones.  It shares nothing with the kernels but the slot
indices: its own gathers, its own softmax statistics and its own fp32 scatter-add of the
per-(row, slot) dKV contributions (``index_add_``).  Products run in fp32 on contiguous
operands.  The CPU oracle (fp64) pins the same closed form on small inputs
(tests/test_oracle.py), and the sampled-row / sampled-key checks hold the kernels to it at
full size as well.
"""

from __future__ import annotations

import torch


def attention_reference(q, kv, idx, dout, scale, *, d_v=512, q_offset=0, sinks=None, rows=64, on_rows=None):
    """fp32 out [S,H,d_v], lse [S,H] (natural log, sink included), mass [S,K] (head-summed P
    at the slots), dq [S,H,D], dkv [S_kv,D] and, with ``sinks``, d_sinks [H] of batch 0.

    q [1,S,H,D], kv [1,S_kv,D] (k = the whole row, v = its first d_v columns), idx [1,S,K]
    (slot j of row s is used iff 0 <= idx < S_kv and idx <= s + q_offset), dout [1,S,H,d_v].
    ``on_rows(r0, r1, chunk)`` instead receives each row chunk's out / lse / mass / dq as it is
    made (nothing of them is kept: the long configurations' fp32 rows would not fit), and
    only dkv and d_sinks are returned.
    """
    S, H, D = q.shape[1:]
    s_kv = kv.shape[1]
    K = idx.shape[-1]
    dev = q.device
    kv32 = kv[0].float()
    f32 = dict(device=dev, dtype=torch.float32)
    keep = on_rows is None
    out = torch.empty(S, H, d_v, **f32) if keep else None
    lse = torch.empty(S, H, **f32) if keep else None
    mass = torch.empty(S, K, **f32) if keep else None
    dq = torch.empty(S, H, D, **f32) if keep else None
    dkv = torch.zeros(s_kv, D, **f32)
    dsink = torch.zeros(H, **f32) if sinks is not None else None
    sk = sinks.float().view(1, H, 1) if sinks is not None else None
    for r0 in range(0, S, rows):
        r1 = min(S, r0 + rows)
        ii = idx[0, r0:r1].long()
        lim = torch.arange(r0, r1, device=dev).view(-1, 1) + q_offset
        valid = (ii >= 0) & (ii < s_kv) & (ii <= lim)
        iic = ii.clamp(0, s_kv - 1)
        kr = kv32[iic]  # [R,K,D]
        vr = kr[..., :d_v].contiguous()
        qr = q[0, r0:r1].float()
        do = dout[0, r0:r1].float()
        logits = torch.bmm(qr, kr.transpose(1, 2).contiguous()) * scale  # [R,H,K]
        logits = logits.masked_fill(~valid.unsqueeze(1), float("-inf"))
        if sk is not None:
            l = torch.logsumexp(torch.cat([logits, sk.expand(r1 - r0, H, 1)], dim=-1), dim=-1)
        else:
            l = torch.logsumexp(logits, dim=-1)
        p = torch.exp(logits - l.unsqueeze(-1)).nan_to_num(0.0)  # rows with no key: P = 0
        o = torch.bmm(p, vr)
        dp = torch.bmm(do, vr.transpose(1, 2).contiguous())
        delta = (do * o).sum(-1)
        ds = p * (dp - delta.unsqueeze(-1))
        dq_r = torch.bmm(ds, kr) * scale
        c = torch.bmm(ds.transpose(1, 2).contiguous(), qr) * scale  # [R,K,D]
        c[..., :d_v] += torch.bmm(p.transpose(1, 2).contiguous(), do)
        c = c * valid.unsqueeze(-1)
        dkv.index_add_(0, iic.reshape(-1), c.reshape(-1, D))
        if keep:
            out[r0:r1], lse[r0:r1], mass[r0:r1], dq[r0:r1] = o, l, p.sum(1), dq_r
        else:
            on_rows(r0, r1, dict(out=o, lse=l, mass=p.sum(1), dq=dq_r))
        if sk is not None:
            dsink -= (torch.exp(sk.view(1, H) - l).nan_to_num(0.0) * delta).sum(0)
    return dict(out=out, lse=lse, mass=mass, dq=dq, dkv=dkv, dsink=dsink)


def chunk_rel_errors(got, ref, dim0_chunk):
    """Relative errors ||got - ref|| / ||ref|| over consecutive chunks of the first axis
    (chunks whose reference is all zero are compared in absolute terms against 1e-30)."""
    errs = []
    for a in range(0, ref.shape[0], dim0_chunk):
        g = got[a:a + dim0_chunk].double()
        r = ref[a:a + dim0_chunk].double()
        errs.append(float((g - r).norm() / r.norm().clamp_min(1e-30)) if float(r.norm()) > 0 else float(g.norm()))
    return torch.tensor(errs)
