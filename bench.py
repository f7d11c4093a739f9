#!/usr/bin/env python3
"""DSA sparse-attention fwd+bwd throughput on one MI355X (tokens/s) with roofline accounting.

One step = one pass of the DeepSeek-V3.2 DSA hot path over one synthetic batch
(config C3 by default: B=1, S=8192, H=128, D_qk=576 / D_v=512, top-k 2048, indexer
64 heads x 128 with fp8-e4m3 per-token-scaled keys and queries):

  fp8 quantise q_I, k_I -> lightning indexer + top-k -> sparse MLA forward ->
  sparse MLA backward (dQ, dKV, and the head-summed attention mass the indexer loss
  needs, from the probabilities the backward recomputes) -> indexer KL loss gradients

Inputs are resident in HBM before the timed region.  Prints ONE JSON line.  The
library's kernel timing (HIP events around every kernel launch, on the stream the kernel
runs on) is on over the timed region: ``kernels_in_step`` lists every kernel with its
average launch duration, algorithmic bytes (or FLOPs) per launch and fraction of peak,
slowest first, and ``roofline`` is the dominant one (the most time per step).
``roofline_attention_fwd_bwd`` is the attention forward + backward as a whole.
``cpu_baseline`` times the CPU oracle (fp32, all host threads) on a bounded sample of the
same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", choices=("c3", "c3-op", "c4", "c5", "c5-long", "v4"), default="c3",
                   help="c3 (default, the headline): dense-KV step at S=8192; c4: compressed-KV step "
                        "(block compressor r=4, indexer and attention over S/4 compressed rows, S=32768); "
                        "c5: 8 packed sequences of U[1024,32768] tokens through the varlen entry points; "
                        "c5-long: one 131072-token sequence; v4: DeepSeek-V4 shared-KV attention (128-token "
                        "window + top-1024 of the S/4 compressed rows + per-head sink, 128 heads x 512) fwd+bwd; "
                        "c3-op: the C3 layer through the torch_npu op surface (bf16 indexer, the fused indexer "
                        "KL op recomputing its target mass)")
    p.add_argument("--seq", type=int, default=None, help="query tokens (default: 8192, or 32768 for c4, "
                                                          "131072 for c5-long)")
    p.add_argument("--heads", type=int, default=128)
    p.add_argument("--topk", type=int, default=2048)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--varlen-bounds", choices=("host", "device"), default="host",
                   help="c5: sequence bounds as a host list (one launch per sequence) or a device tensor (one "
                        "launch per op over the whole batch, no host read)")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="target CPU time of the baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run one 1 GiB device copy first (reference kernel for the PMC byte counters)")
    return p.parse_args()


def make_inputs(S, H, topk, seed, device, on_device=False):
    """Seeded synthetic inputs of one dense-KV step.  ``on_device`` draws them with a
    generator on the GPU (the long-sequence workloads; the host generator would spend
    minutes on tens of GB of normals)."""
    import torch

    if on_device:
        return _device_inputs(S, H, topk, seed, device, [S], [S])
    g = torch.Generator().manual_seed(seed)
    d_qk, d_v, h_i, d_i = 576, 512, 64, 128
    # fixed draw order: q, kv, q_idx, k_idx, w, dout
    q = torch.randn(1, S, H, d_qk, generator=g)
    kv = torch.randn(1, S, d_qk, generator=g)
    q_idx = torch.randn(1, S, h_i, d_i, generator=g)
    k_idx = torch.randn(1, S, d_i, generator=g)
    w = torch.rand(1, S, h_i, generator=g) * h_i ** -0.5 * d_i ** -0.5
    dout = torch.randn(1, S, H, d_v, generator=g)
    to = dict(device=device)
    return dict(
        q=q.to(torch.bfloat16).to(**to),
        kv=kv.to(torch.bfloat16).to(**to),
        q_idx=q_idx.to(torch.bfloat16).to(**to),
        k_idx=k_idx.to(torch.bfloat16).to(**to),
        w=w.to(**to),
        dout=dout.to(torch.bfloat16).to(**to),
        scale=d_qk ** -0.5,
        topk=topk,
    )


def _device_inputs(T, H, topk, seed, device, lens_q, lens_k, kv_rows=None):
    """Packed inputs drawn on the device: q [1,T,H,576], kv [1,kv_rows,576], q_idx
    [1,T,64,128], k_idx [1,kv_rows,128], w [1,T,64], dout [1,T,H,512] (same draw order as
    the host variant)."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    d_qk, d_v, h_i, d_i = 576, 512, 64, 128
    kv_rows = T if kv_rows is None else kv_rows
    bf = dict(device=device, dtype=torch.bfloat16, generator=g)
    q = torch.randn(1, T, H, d_qk, **bf)
    kv = torch.randn(1, kv_rows, d_qk, **bf)
    q_idx = torch.randn(1, T, h_i, d_i, **bf)
    k_idx = torch.randn(1, kv_rows, d_i, **bf)
    w = torch.rand(1, T, h_i, device=device, generator=g) * h_i ** -0.5 * d_i ** -0.5
    dout = torch.randn(1, T, H, d_v, **bf)
    return dict(q=q, kv=kv, q_idx=q_idx, k_idx=k_idx, w=w, dout=dout, scale=d_qk ** -0.5, topk=topk,
                lens_q=list(lens_q), lens_k=list(lens_k))


def compressor_inputs(S, D, ratio, seed, device):
    """Inputs of one block-compressor call (reference Compressor._forward_bsnd): the wkv and
    wgate projections [1,S,coff*D] fp32 (gate logits ~N(0,1)), ape ~N(0,0.02) [ratio,coff*D],
    RMSNorm weight [D]; coff = 2 (overlapping blocks) when ratio == 4."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    coff = 2 if ratio == 4 else 1
    f = dict(device=device, dtype=torch.float32, generator=g)
    kv = torch.randn(1, S, coff * D, **f)
    score = torch.randn(1, S, coff * D, **f)
    ape = torch.randn(ratio, coff * D, **f) * 0.02
    norm_w = 1.0 + 0.1 * torch.randn(D, **f)
    return dict(kv=kv, score=score, ape=ape, norm_w=norm_w, ratio=ratio, D=D, coff=coff, S=S)


def compressor_bytes(c):
    """Algorithmic bytes of one compressor call: both fp32 projections read once, ape, and the
    bf16 output rows."""
    S, D, r, coff = c["S"], c["D"], c["ratio"], c["coff"]
    return 2 * S * coff * D * 4 + r * coff * D * 4 + (S // r) * D * 2


def time_ms(torch, fn, reps=10):
    """Average duration (ms) of ``fn`` over ``reps`` back-to-back calls, HIP events on the
    current stream (the one every op here launches on), after one untimed call."""
    fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


class PhaseTimer:
    """HIP events on the current stream around each phase; averages over timed steps."""

    def __init__(self, torch):
        self.torch = torch
        self.events = {}
        self.enabled = False

    def __call__(self, name):
        timer = self

        class _Ctx:
            def __enter__(self_inner):
                if timer.enabled:
                    self_inner.e0 = timer.torch.cuda.Event(enable_timing=True)
                    self_inner.e1 = timer.torch.cuda.Event(enable_timing=True)
                    self_inner.e0.record()

            def __exit__(self_inner, *exc):
                if timer.enabled:
                    self_inner.e1.record()
                    timer.events.setdefault(name, []).append((self_inner.e0, self_inner.e1))

        return _Ctx()

    def averages_ms(self):
        out = {}
        for k, evs in self.events.items():
            out[k] = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
        return out


def dsa_step(inp, ops, timer):
    """One DSA layer forward + backward; returns the tensors a trainer would consume."""
    with timer("quantize"):
        q8, qs = ops.quantize_fp8_per_row(inp["q_idx"])
        k8, ks = ops.quantize_fp8_per_row(inp["k_idx"])
    with timer("indexer_topk"):
        idx, _ = ops.npu_lightning_indexer(q8, k8, inp["w"], sparse_count=inp["topk"], sparse_mode=3,
                                           query_scale=qs, key_scale=ks)
        idx = idx[:, :, 0]
    with timer("attn_fwd"):
        out, smax, ssum = ops.sparse_mla_fwd(inp["q"], inp["kv"], idx, inp["scale"])
    with timer("attn_bwd"):
        dq, dkv, mass = ops.sparse_mla_bwd(inp["q"], inp["kv"], idx, out, inp["dout"], smax, ssum, inp["scale"],
                                           return_mass=True)
    with timer("indexer_kl_grad"):
        dq_i, dk_i, dw, loss_rows = ops.indexer_kl_grad_from_mass(inp["q_idx"], inp["k_idx"], inp["w"], idx, mass)
    return dict(idx=idx, out=out, dq=dq, dkv=dkv, dq_i=dq_i, dk_i=dk_i, dw=dw, loss=loss_rows)


def c3_op_step(inp, ops, timer):
    """The C3 layer through the op surface that a converter written against torch_npu calls
    (reference converters/kernels/dsa.py:159-177, :217-253): the bf16 lightning indexer with
    its fused top-k, the sparse attention forward and backward, and the fused indexer KL op,
    which recomputes its target mass from the forward statistics (dsa_attn_mass) as the
    reference's npu_sparse_lightning_indexer_grad_kl_loss does."""
    with timer("indexer_topk"):
        idx, _ = ops.npu_lightning_indexer(inp["q_idx"], inp["k_idx"], inp["w"], sparse_count=inp["topk"],
                                           sparse_mode=3)
        idx = idx[:, :, 0]
    with timer("attn_fwd"):
        out, smax, ssum = ops.sparse_mla_fwd(inp["q"], inp["kv"], idx, inp["scale"])
    with timer("attn_bwd"):
        dq, dkv = ops.sparse_mla_bwd(inp["q"], inp["kv"], idx, out, inp["dout"], smax, ssum, inp["scale"])
    with timer("indexer_kl_grad"):
        dq_i, dk_i, dw, loss = ops.npu_sparse_lightning_indexer_grad_kl_loss(
            inp["q"], inp["kv"], inp["q_idx"], inp["k_idx"], inp["w"], idx, smax, ssum, inp["scale"])
    return dict(idx=idx, out=out, dq=dq, dkv=dkv, dq_i=dq_i, dk_i=dk_i, dw=dw, loss=loss)


def c4_step(inp, comp, comp_i, ops, timer):
    """One compressed-KV layer (config C4): block compressor (r=4, overlapping blocks,
    RMSNorm epilogue) for the 512-column KV and the 128-column indexer keys -> fp8
    indexer + top-k over the S/4 compressed rows (valid: t < (s+1)//4) -> gathered
    attention forward + backward over the selected compressed rows -> indexer KL
    gradients.  Compressed rows have 512 columns (k = v = the row, as in
    SparseAttention), and the attention runs on the kernels' 512-column variant with
    512-column queries."""
    with timer("compressor"):
        ckv = ops.compressor_pool(comp["kv"], comp["score"], comp["ape"], 4, norm_weight=comp["norm_w"])
        cki = ops.compressor_pool(comp_i["kv"], comp_i["score"], comp_i["ape"], 4, norm_weight=comp_i["norm_w"])
    with timer("quantize"):
        q8, qs = ops.quantize_fp8_per_row(inp["q_idx"])
        k8, ks = ops.quantize_fp8_per_row(cki)
    with timer("indexer_topk"):
        idx, _ = ops.npu_lightning_indexer(q8, k8, inp["w"], sparse_count=inp["topk"], sparse_mode=3, cmp_ratio=4,
                                           query_scale=qs, key_scale=ks)
        idx = idx[:, :, 0]
    nm = ops._NO_MASK_OFFSET  # validity is already in the indices (-1 past (s+1)//4)
    with timer("attn_fwd"):
        out, smax, ssum = ops.sparse_mla_fwd(inp["q"], ckv, idx, inp["scale"], q_offset=nm)
    with timer("attn_bwd"):
        dq, dkv, mass = ops.sparse_mla_bwd(inp["q"], ckv, idx, out, inp["dout"], smax, ssum, inp["scale"],
                                           q_offset=nm, return_mass=True)
    with timer("indexer_kl_grad"):
        dq_i, dk_i, dw, loss_rows = ops.indexer_kl_grad_from_mass(inp["q_idx"], cki, inp["w"], idx, mass,
                                                                  q_offset=nm)
    return dict(idx=idx, out=out, dq=dq, dkv=dkv, dq_i=dq_i, dk_i=dk_i, dw=dw, loss=loss_rows)


def c5_step(inp, ops, timer):
    """One layer over a packed varlen batch (config C5 ii) through the ``_varlen`` entry
    points: each sequence attends causally to its own tokens only.  The sequence bounds are a
    device tensor (``inp["cu_dev"]``, the form a trainer's packed batch carries them in: the ops
    then read them on the device; ``--varlen-bounds device``) or a host list (the ops schedule
    one launch per sequence; the default)."""
    cu = inp.get("cu_dev")
    if cu is None:
        cu = [0]
        for n in inp["lens_q"]:
            cu.append(cu[-1] + n)
    q, kv, qi, ki, w, do = (inp[k][0] for k in ("q", "kv", "q_idx", "k_idx", "w", "dout"))
    with timer("quantize"):
        q8, qs = ops.quantize_fp8_per_row(qi)
        k8, ks = ops.quantize_fp8_per_row(ki)
    with timer("indexer_topk"):
        idx, _ = ops.lightning_indexer_varlen(q8, k8, w, cu, cu, inp["topk"], query_scale=qs, key_scale=ks)
    with timer("attn_fwd"):
        out, smax, ssum = ops.sparse_mla_fwd_varlen(q, kv, idx, inp["scale"], cu, cu)
    with timer("attn_bwd"):
        dq, dkv, mass = ops.sparse_mla_bwd_varlen(q, kv, idx, out, do, smax, ssum, inp["scale"], cu, cu,
                                                  return_mass=True)
    with timer("indexer_kl_grad"):
        dq_i, dk_i, dw, loss_rows = ops.indexer_kl_grad_from_mass_varlen(qi, ki, w, idx, mass, cu, cu)
    return dict(idx=idx, out=out, dq=dq, dkv=dkv, dq_i=dq_i, dk_i=dk_i, dw=dw, loss=loss_rows)


def v4_inputs(S, H, topk, seed, device, ratio=4):
    """DeepSeek-V4 attention layer inputs drawn on the device: query [1,S,H,512], window
    rows ori_kv [1,S,512], compressed rows cmp_kv [1,S/r,512], indexer q_I [1,S,64,128],
    compressed indexer keys [1,S/r,128], w [1,S,64], sinks [H] ~ N(0,1), dout."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    bf = dict(device=device, dtype=torch.bfloat16, generator=g)
    n_c = S // ratio
    return dict(q=torch.randn(1, S, H, 512, **bf), ori=torch.randn(1, S, 512, **bf),
                cmp=torch.randn(1, n_c, 512, **bf), q_idx=torch.randn(1, S, 64, 128, **bf),
                k_idx=torch.randn(1, n_c, 128, **bf),
                w=torch.rand(1, S, 64, device=device, generator=g) * 64 ** -0.5 * 128 ** -0.5,
                sinks=torch.randn(H, device=device, generator=g), dout=torch.randn(1, S, H, 512, **bf),
                scale=512 ** -0.5, topk=topk, ratio=ratio, window=128)


def v4_step(inp, ops, timer):
    """One DeepSeek-V4 attention layer (SparseAttention with the NPU op's layout): fp8
    indexer + top-k over the compressed rows (valid t < (s+1)//4), then the shared-KV
    attention over the 128-token window and the selected compressed rows with the per-head
    sink, forward and backward (gradients to query, both KV sets and the sinks)."""
    import torch

    S = inp["q"].shape[1]
    with timer("quantize"):
        q8, qs = ops.quantize_fp8_per_row(inp["q_idx"])
        k8, ks = ops.quantize_fp8_per_row(inp["k_idx"])
    with timer("indexer_topk"):
        idx, _ = ops.npu_lightning_indexer(q8, k8, inp["w"], sparse_count=inp["topk"], sparse_mode=3,
                                           cmp_ratio=inp["ratio"], query_scale=qs, key_scale=ks)
        idx = idx[:, :, 0]
        idx = torch.where(idx >= 0, idx + S, idx)  # rows of cat(ori_kv, cmp_kv)
    leaves = [inp[k].detach().requires_grad_(True) for k in ("q", "ori", "cmp", "sinks")]
    with timer("attn_fwd"):
        out = ops.npu_sparse_attn_shared_kv(leaves[0], leaves[1], leaves[2], idx, leaves[3], inp["scale"],
                                            inp["ratio"], ori_win_left=inp["window"] - 1)
    with timer("attn_bwd"):
        out.backward(inp["dout"])
    return dict(idx=idx, out=out, dq=leaves[0].grad, d_ori=leaves[1].grad, d_cmp=leaves[2].grad,
                dsink=leaves[3].grad)


def algorithmic_work(S, H, topk, idx, d_qk=576, d_v=512, h_i=64, d_i=128, causal_pairs=None, sum_keff=None):
    """Algorithmic bytes and FLOPs of the DSA path per step.

    sum_keff = number of valid (row, slot) pairs; every head of a row shares its gathered
    KV rows, so each row's keys are counted once; dKV is counted as an fp32 scatter-add
    payload (4 bytes per element per pair).  ``causal_pairs`` = the (query, key) pairs the
    indexer scores (default: one causal sequence of S tokens).
    """
    if sum_keff is None:
        sum_keff = int((idx >= 0).sum().item())
    if causal_pairs is None:
        causal_pairs = S * (S + 1) // 2
    K = topk
    fwd_bytes = 2 * H * d_qk * S + 2 * d_qk * sum_keff + 4 * K * S + 2 * H * d_v * S + 4 * H * S
    bwd_bytes = (2 * H * d_qk * S * 2 + 2 * H * d_v * S * 2 + 4 * H * S + 4 * K * S + 2 * d_qk * sum_keff
                 + 4 * d_qk * sum_keff)
    return dict(
        sum_keff=sum_keff,
        attn_fwd_bytes=fwd_bytes,
        attn_bwd_bytes=bwd_bytes,
        attn_fwd_flops=2 * H * (d_qk + d_v) * sum_keff,
        attn_bwd_flops=2 * H * (3 * d_qk + 2 * d_v) * sum_keff,
        indexer_flops=2 * h_i * d_i * causal_pairs,
        topk_bytes=4 * causal_pairs + 4 * K * S,
    )


def measured_traffic(kernel, S, H, K):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 PMC summary, or None.

    profiles/hbm_traffic_c3.json holds FETCH_SIZE and WRITE_SIZE per dispatch, each
    already divided by the factor the same counter reads on a copy of known size.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic_c3.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    wl = data.get("workload", {})
    if (wl.get("seq_len"), wl.get("heads"), wl.get("topk")) != (S, H, K):
        return None
    k = data.get("kernels", {}).get(kernel)
    if not k:
        return None
    return k["fetch_bytes"] + k["write_bytes"]


def step_kernel_work(S, H, K, P, pairs, s_kv, s_ki=None, h_i=64, d_i=128, d_qk=576, k_attn=None, sink=False):
    """Algorithmic work of one launch-set per step of every kernel in the DSA step, keyed by
    the name the library's kernel timing reports (dsa_kernel_timing).

    S query rows, H heads, K top-k slots, P = valid (row, slot) pairs of the attention,
    ``pairs`` = causal (query, key) pairs the indexer scores, s_kv attention keys, s_ki
    indexer keys (default s_kv), d_qk the attention row width (576: latent + rope; 512: the
    rope-less DeepSeek-V4 rows, whose kernels report a ``<512>`` name), k_attn the attention
    slots per row (default K; V4: the 128-token window + K), ``sink`` whether the attention
    has a per-head sink (then a separate pass forms delta = rowsum(dO o O) for the score
    kernel; without one the score kernel reads O itself).  Returns name -> (bound, bytes,
    flops, intermediate_bytes):

    * ``bytes``: the operands of the op contract that the kernel must move once, counted as
      the per-unit formulas of the survey's measurement table count them (Q, dO, O, the
      gathered KV rows per pair, indices, row statistics, dQ, dKV; no cache hits assumed).
      The dKV scatter-add payload (4 bytes per element and pair) is what the backward's
      contribution rows cost here: written once in bf16 by the contribution kernel and read
      once by the key-major reduction (2 + 2 bytes per element and pair);
    * ``intermediate_bytes``: what this design adds between its kernels and the op contract
      does not have: G (dS and P per head, bf16) written by the score kernel and read back by
      the dQ and contribution kernels, the per-row delta, the head-summed mass handed to the
      indexer loss, and the CSR pair lists;
    * ``flops``: the MFMA products.
    """
    s_ki = s_kv if s_ki is None else s_ki
    Ka = K if k_attn is None else k_attn
    dq, dv, gw = d_qk, 512, 256  # row width, latent width, G row (dS | P) x 128 heads
    w = {
        "quantize_fp8_kernel": ("hbm", (S * h_i + s_ki) * (2 * d_i + d_i + 4), 0, 0),
        "indexer_lin_pieces_kernel<64>": ("hbm", 0, 0, S * (h_i * d_i + 4 * h_i + 4 * h_i + 4 * d_i + 16)),
        "indexer_tile_kernel<fp8, 4, split>": ("mfma", 0, 2 * h_i * d_i * pairs, 0),
        # bf16 indexer (the op surface without quantisation): against the fp8 peak x 1/2
        "indexer_tile_kernel": ("mfma_bf16", 0, 2 * h_i * d_i * pairs, 0),
        # Q, gathered rows, indices, row statistics | mass written (the KL op's target)
        "attn_mass_bf16_kernel": ("hbm", 2 * H * dq * S + 2 * dq * P + 4 * Ka * S + 8 * H * S, 2 * H * dq * P,
                                  4 * Ka * S),
        "topk_kernel": ("hbm", 4 * pairs + 4 * K * S, 0, 0),
        "sparse_mla_fwd_bf16_kernel": ("hbm", 2 * H * dq * S + 2 * dq * P + 4 * Ka * S + 2 * H * dv * S + 8 * H * S,
                                       2 * H * (dq + dv) * P, 0),
        "sparse_mla_fwd_exact_kernel<fixup>": ("hbm", 4 * H * S, 0, 0),
        # O, dO | delta written
        "bwd_delta_kernel": ("hbm", 2 * (2 * H * dv * S), 0, 4 * H * S),
        # Q, dO, O (delta formed here when there is no sink), gathered rows, indices, row
        # statistics | G written, mass written, delta read (with a sink)
        "bwd_sdp_kernel": ("hbm", 2 * H * dq * S + 2 * H * dv * S * (1 if sink else 2) + 2 * dq * P + 4 * Ka * S
                           + 8 * H * S, 2 * H * (dq + dv) * P, 2 * gw * P + 4 * Ka * S + (4 * H * S if sink else 0)),
        # gathered rows, indices, dQ written | dS half of G read
        "bwd_dqk_kernel": ("hbm", 2 * dq * P + 4 * Ka * S + 2 * H * dq * S, 2 * H * dq * P, 2 * (gw // 2) * P),
        # X = [Q; dO], indices, contribution rows written (half the scatter payload) | G read
        "bwd_contrib_kernel<2>": ("hbm", 2 * H * (dq + dv) * S + 4 * Ka * S + 2 * dq * P,
                                  2 * P * (gw * dv + (gw // 2) * (dq - dv)), 2 * gw * P),
        "zero_i32_kernel": ("hbm", 0, 0, 4 * (s_kv + 1) + 4 * (s_ki + 1)),
        "csr_count_kernel<count>": ("hbm", 0, 0, 8 * Ka * S),
        "csr_count_kernel<fill>": ("hbm", 0, 0, 8 * Ka * S + 8 * P),
        # (the same list, staged per key in LDS and written as 32-byte sectors)
        "csr_fill_staged_kernel": ("hbm", 0, 0, 8 * Ka * S + 8 * P),
        "csr_count_kernel<fill, repair>": ("hbm", 0, 0, 0),
        "csr_scan_kernel": ("hbm", 0, 0, 12 * (s_kv + s_ki)),
        "csr_seg_key_kernel": ("hbm", 0, 0, 8 * (s_kv + s_ki)),
        # contribution rows read (the other half of the scatter payload), fp32 dKV written | pair list
        "dkv_reduce_kernel<72>": ("hbm", 2 * dq * P + 4 * dq * s_kv, 0, 4 * P),
        # q_I, gathered k_I rows, weights, dq_I (fp32), dk_I contributions (half the dk_I scatter
        # payload), dw, loss | mass read, the key rows' second gather (the gradient pass)
        "indexer_kl_mfma_kernel": ("hbm", S * (2 * h_i * d_i + 4 * h_i + 4 * h_i * d_i + 4 * h_i + 4)
                                   + P * (2 * d_i + 2 * d_i), 2 * P * h_i * d_i * 3, 4 * K * S + 2 * d_i * P),
        # dk_I contributions read (the other half of the payload), fp32 dk_I written | pair list
        "dkv_reduce_kernel<16>": ("hbm", 2 * d_i * P + 4 * d_i * s_ki, 0, 4 * P),
        "compressor_kernel": ("hbm", 0, 0, 0),  # per-call bytes depend on the block geometry; see kernels
    }
    if dq != 576:  # the rope-less variants' names
        for name in ("sparse_mla_fwd_bf16_kernel", "bwd_sdp_kernel", "bwd_dqk_kernel", "attn_mass_bf16_kernel"):
            w[f"{name}<{dq}>"] = w.pop(name)
        w[f"bwd_contrib_kernel<2,{dq}>"] = w.pop("bwd_contrib_kernel<2>")
        w[f"dkv_reduce_kernel<{dq // 8}>"] = w.pop("dkv_reduce_kernel<72>")
    return w


def kernel_table(ktimes, work, steps, traffic_of=None):
    """Per-kernel roofline rows, slowest first: average launch duration and launches per step
    from the kernel timing, the algorithmic bytes (or FLOPs for MFMA-bound kernels) per launch,
    achieved rate and ``frac`` of peak on those bytes alone; the design-intermediate bytes per
    launch and ``frac_with_intermediates`` on both; the MFMA fraction of the bf16 peak where
    the kernel runs MFMAs, and the counter bytes per launch when a PMC summary has the kernel."""
    rows = []
    for name, (total_ms, launches) in ktimes.items():
        per_step = launches / steps
        avg = total_ms / launches
        row = dict(kernel=name, avg_launch_ms=avg, launches_per_step=per_step, ms_per_step=total_ms / steps)
        if name in work:
            bound, nbytes, flops, inter = work[name]
            b1, f1, i1 = nbytes / per_step, flops / per_step, inter / per_step
            if bound in ("mfma", "mfma_bf16"):
                ach = f1 / (avg * 1e-3) / 1e12
                peak = FP8_PEAK_TFLOPS if bound == "mfma" else BF16_PEAK_TFLOPS
                row.update(bound="mfma", algorithmic_flops=f1, achieved=ach, peak=peak, unit="TFLOP/s",
                           frac=ach / peak)
            elif nbytes or inter:
                ach = b1 / (avg * 1e-3) / 1e9
                row.update(bound="hbm", algorithmic_bytes=b1, achieved=ach, peak=HBM_PEAK_GBPS, unit="GB/s",
                           frac=ach / HBM_PEAK_GBPS)
                if flops:
                    row["mfma_frac_bf16"] = f1 / (avg * 1e-3) / 1e12 / BF16_PEAK_TFLOPS
            if inter and bound not in ("mfma", "mfma_bf16"):
                row["intermediate_bytes"] = i1
                row["frac_with_intermediates"] = (b1 + i1) / (avg * 1e-3) / 1e9 / HBM_PEAK_GBPS
        if traffic_of is not None:
            t = traffic_of(name)
            if t is not None:
                row["traffic"] = t
                row["traffic_gbps"] = t / (avg * 1e-3) / 1e9
        rows.append(row)
    rows.sort(key=lambda r: -r["ms_per_step"])
    return rows


def time_indexer_kernel(inp, ops, torch, reps=10):
    """Average duration (ms) of the lightning-indexer scores alone (dsa_indexer_fwd_ws, fp8
    queries and keys, causal: the linear-split pre-pass plus the score kernel), timed with HIP
    events on the stream they run on, outside the timed steps.  The step's indexer phase also
    includes the top-k selection."""
    q8, qs = ops.quantize_fp8_per_row(inp["q_idx"])
    k8, ks = ops.quantize_fp8_per_row(inp["k_idx"])
    S = q8.shape[1]
    out = torch.empty(1, S, k8.shape[1], dtype=torch.float32, device=q8.device)

    ms = time_ms(torch, lambda: ops.indexer_scores(q8, k8, inp["w"], q_scale=qs, k_scale=ks, q_offset=0, out=out),
                 reps)
    del out
    return ms


def copy_calibration(torch, device, nbytes=1 << 30):
    """One elementwise copy kernel of known size (reads and writes ``nbytes`` once each), for
    scaling the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def cpu_baseline(inp_gpu, S, H, topk, seconds):
    """Time the CPU oracle (fp32, all host threads) on the last rows of the same workload."""
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import dsa_oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    threads = torch.get_num_threads()
    cpu = {k: (v.cpu() if hasattr(v, "cpu") else v) for k, v in inp_gpu.items()}
    q, kv, qi, ki, w, do = (cpu[k].float() for k in ("q", "kv", "q_idx", "k_idx", "w", "dout"))
    qi8, qis = O.quantize_e4m3_per_row(qi)
    ki8, kis = O.quantize_e4m3_per_row(ki)
    qid = qi8.float() * qis.unsqueeze(-1)
    kid = ki8.float() * kis.unsqueeze(-1)

    def run(rows):
        r0 = S - rows
        # the last `rows` query rows against the full KV prefix (q_offset = r0)
        sc = O.indexer_scores(qid[:, r0:], kid, w[:, r0:], q_offset=r0)
        idx = O.topk_select(sc, topk, q_offset=r0)
        out, lse = O.sparse_mla_fwd(q[:, r0:], kv, idx, cpu["scale"], q_offset=r0, dtype=torch.float32, chunk=8)
        O.indexer_kl_loss_grad(q[:, r0:], kv, qi[:, r0:], ki, w[:, r0:], idx, lse, cpu["scale"], q_offset=r0,
                               dtype=torch.float32)
        O.sparse_mla_bwd_closed_form(q[:, r0:], kv, idx, out, lse, do[:, r0:], cpu["scale"], q_offset=r0,
                                     dtype=torch.float32)

    rows = 4
    run(rows)  # warm-up
    t0 = time.perf_counter()
    run(rows)
    dt = time.perf_counter() - t0
    rows = max(4, min(256, S, int(rows * seconds / max(dt, 1e-3) / 3)))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(rows)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[1]
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(
        value=rows / med,
        unit="tokens/s",
        cores=threads,
        kind="port",
        sample=(f"fp32 CPU oracle of the full step (fp8-dequantised indexer, top-k, attention fwd, "
                f"indexer KL grads, attention bwd) on the last {rows} of {S} query rows against the "
                f"full KV prefix, median of 3 runs; host CPU: {model}"),
    )


def kernel_rooflines(inp, ops, torch, dev, S, K, seed, with_topk):
    """Per-kernel roofline entries measured outside the timed steps: the block compressor at
    config C4's shape (32768 tokens, r = 4 with overlapping blocks, D = 512 and the indexer's
    D_I = 128; HBM-bound) and, for a dense-KV workload, the top-k selection over the full
    causal score matrix (HBM-bound: scores read once, indices written)."""
    out = {}
    comp = [compressor_inputs(32768, d, 4, seed + 1 + i, dev) for i, d in enumerate((512, 128))]

    def run_comp():
        for c in comp:
            ops.compressor_pool(c["kv"], c["score"], c["ape"], 4, norm_weight=c["norm_w"])

    ms = time_ms(torch, run_comp)
    nbytes = sum(compressor_bytes(c) for c in comp)
    out["compressor"] = dict(kernel="compressor_kernel (D=512 and D=128 launches)", bound="hbm",
                             shape="C4: 32768 tokens, r=4, overlap, RMSNorm epilogue, bf16 out",
                             algorithmic_bytes=nbytes, avg_launch_ms=ms,
                             achieved=nbytes / (ms * 1e-3) / 1e9, peak=HBM_PEAK_GBPS, unit="GB/s",
                             frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS)
    del comp
    # the indexer input producer at the C3 indexer shape: RoPE (V3.2 layout) + Hadamard +
    # fp8 of q_I [1,S,64,128] and k_I [1,S,128]; per 128-feature row 256 B read, 256 B bf16
    # + 128 B fp8 + 4 B scale written
    g = torch.Generator(device=dev).manual_seed(seed + 3)
    qi = torch.randn(1, S, 64, 128, device=dev, dtype=torch.bfloat16, generator=g)
    ki = torch.randn(1, S, 128, device=dev, dtype=torch.bfloat16, generator=g)
    inv = 1.0 / (10000.0 ** (torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    ang = torch.outer(torch.arange(S, dtype=torch.float64), inv)
    fc = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(dev)

    def run_prep():
        ops.indexer_prep(qi, fc)
        ops.indexer_prep(ki, fc)

    ms = time_ms(torch, run_prep)
    nbytes = S * 65 * (256 + 256 + 128 + 4)
    out["indexer_prep"] = dict(kernel="indexer_prep_kernel (q_I and k_I launches)", bound="hbm",
                               shape=f"S={S}: q_I [1,S,64,128] + k_I [1,S,128] bf16, RoPE + Hadamard + fp8",
                               algorithmic_bytes=nbytes, avg_launch_ms=ms, achieved=nbytes / (ms * 1e-3) / 1e9,
                               peak=HBM_PEAK_GBPS, unit="GB/s", frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS)
    del qi, ki
    # the MLA absorb kernels at the C3 attention shape (128 heads): q_nope [1,S,H,128] . w_uk ->
    # the 576-wide query with q_pe appended, and the [1,S,H,512] output . w_uv_t -> [1,S,H,128]
    H = 128
    qn = torch.randn(1, S, H, 128, device=dev, dtype=torch.bfloat16, generator=g)
    qp = torch.randn(1, S, H, 64, device=dev, dtype=torch.bfloat16, generator=g)
    wuk = torch.randn(H, 128, 512, device=dev, dtype=torch.bfloat16, generator=g)
    ao = torch.randn(1, S, H, 512, device=dev, dtype=torch.bfloat16, generator=g)
    wuv = torch.randn(H, 512, 128, device=dev, dtype=torch.bfloat16, generator=g)
    wuk_t, wuv_tt = wuk.transpose(1, 2).contiguous(), wuv.transpose(1, 2).contiguous()

    def run_absorb():
        ops.mla_absorb(qn, wuk_t, append=qp)
        ops.mla_absorb(ao, wuv_tt)

    ms = time_ms(torch, run_absorb)
    nbytes = S * H * 2 * ((128 + 64 + 576) + (512 + 128)) + 2 * H * 128 * 512 * 2
    out["mla_absorb"] = dict(kernel="mla_absorb_kernel<128,512> + <512,128>", bound="hbm",
                             shape=f"S={S}, H={H}: q absorb (128 -> 512, q_pe appended) + output absorb (512 -> 128)",
                             algorithmic_bytes=nbytes, avg_launch_ms=ms, achieved=nbytes / (ms * 1e-3) / 1e9,
                             peak=HBM_PEAK_GBPS, unit="GB/s", frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                             flops=4 * S * H * 128 * 512)
    del qn, qp, wuk, ao, wuv, wuk_t, wuv_tt
    if with_topk:
        q8, qs = ops.quantize_fp8_per_row(inp["q_idx"])
        k8, ks = ops.quantize_fp8_per_row(inp["k_idx"])
        scores = ops.indexer_scores(q8, k8, inp["w"], q_scale=qs, k_scale=ks, q_offset=0)
        ms = time_ms(torch, lambda: ops.topk_select(scores, K, q_offset=0))
        nbytes = 4 * (S * (S + 1) // 2) + 4 * K * S
        out["topk"] = dict(kernel="dsa_topk", bound="hbm", algorithmic_bytes=nbytes, avg_launch_ms=ms,
                           achieved=nbytes / (ms * 1e-3) / 1e9, peak=HBM_PEAK_GBPS, unit="GB/s",
                           frac=nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS)
        del scores
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the DSA path shards by query rows; multi-GPU runs are not part of this build)", file=sys.stderr)
        sys.exit(2)
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from torchtitan_npu_simulator_amd import _lib
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    dev = torch.device("cuda:0")
    wl = args.workload
    H, K = args.heads, args.topk
    S = args.seq or {"c3": 8192, "c3-op": 8192, "c4": 32768, "c5": 0, "c5-long": 131072, "v4": 8192}[wl]
    if args.copy_calibration:
        copy_calibration(torch, dev)
    pairs = None
    if wl == "c3":
        inp = make_inputs(S, H, K, args.seed, dev)
        step = lambda t: dsa_step(inp, ops, t)  # noqa: E731
        cfg = dict(workload="C3: DeepSeek-V3.2 DSA layer fwd+bwd", batch=1, seq_len=S)
    elif wl == "c3-op":
        inp = make_inputs(S, H, K, args.seed, dev)
        step = lambda t: c3_op_step(inp, ops, t)  # noqa: E731
        cfg = dict(workload="C3 through the torch_npu op surface: bf16 indexer + top-k, attention fwd+bwd, fused "
                            "indexer KL op recomputing its target mass", batch=1, seq_len=S)
    elif wl == "c5-long":
        inp = make_inputs(S, H, K, args.seed, dev, on_device=True)
        step = lambda t: dsa_step(inp, ops, t)  # noqa: E731
        cfg = dict(workload="C5(i): one long sequence, DSA layer fwd+bwd, indexer chunked by query rows",
                   batch=1, seq_len=S)
    elif wl == "c4":
        inp = _device_inputs(S, H, K, args.seed, dev, [S], [S // 4], kv_rows=0)
        inp["q"] = inp["q"][..., :512].contiguous()  # 512-column rows: k = v = the compressed row
        inp["scale"] = 512 ** -0.5
        comp = compressor_inputs(S, 512, 4, args.seed + 1, dev)
        comp_i = compressor_inputs(S, 128, 4, args.seed + 2, dev)
        step = lambda t: c4_step(inp, comp, comp_i, ops, t)  # noqa: E731
        pairs = sum((s + 1) // 4 for s in range(S))
        cfg = dict(workload="C4: compressed KV (r=4, overlap) compressor + indexer + attention fwd+bwd",
                   batch=1, seq_len=S, compressed_rows=S // 4, cmp_ratio=4)
    elif wl == "v4":
        inp = v4_inputs(S, H, K if args.topk != 2048 else 1024, args.seed, dev)
        step = lambda t: v4_step(inp, ops, t)  # noqa: E731
        pairs = sum((s + 1) // 4 for s in range(S))
        K = inp["topk"]
        cfg = dict(workload="DeepSeek-V4 shared-KV attention fwd+bwd (window 128 + compressed r=4 top-k + sink)",
                   batch=1, seq_len=S, window=128, cmp_ratio=4, compressed_rows=S // 4)
    else:  # c5: packed varlen batch
        g = torch.Generator().manual_seed(args.seed)
        lens = torch.randint(1024, 32769, (8,), generator=g).tolist()
        S = sum(lens)
        inp = _device_inputs(S, H, K, args.seed, dev, lens, lens)
        if args.varlen_bounds == "device":
            bounds = [0]
            for n in lens:
                bounds.append(bounds[-1] + n)
            inp["cu_dev"] = torch.tensor(bounds, dtype=torch.int32, device=dev)
        step = lambda t: c5_step(inp, ops, t)  # noqa: E731
        pairs = sum(n * (n + 1) // 2 for n in lens)
        cfg = dict(workload="C5(ii): 8 packed sequences (TND), varlen entry points, fwd+bwd", tokens=S,
                   seq_lens=lens, seq_bounds=args.varlen_bounds)
    timer = PhaseTimer(torch)
    for _ in range(args.warmup):
        res = step(timer)
    torch.cuda.synchronize()
    timer.enabled = True
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    # HIP events around every library kernel launch inside the timed region, on the stream
    # each kernel runs on (the library's own timing; a few microseconds per step)
    with _lib.kernel_timing() as ktimer:
        t0.record()
        for _ in range(args.steps):
            res = step(timer)
        t1.record()
        torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    ktimes = ktimer.summary()
    phases = timer.averages_ms()
    if wl == "v4":
        # slots per row: the window (min(128, s + 1) rows) plus the valid compressed picks;
        # rows are 512 wide (the kernels' rope-less variant)
        win = sum(min(128, s + 1) for s in range(S))
        work = algorithmic_work(S, H, K, res["idx"], causal_pairs=pairs, d_qk=512)
        work = algorithmic_work(S, H, K + 128, None, causal_pairs=pairs, sum_keff=work["sum_keff"] + win, d_qk=512)
    else:
        work = algorithmic_work(S, H, K, res["idx"], causal_pairs=pairs, d_qk=512 if wl == "c4" else 576)
    del res

    fwd_ms = phases["attn_fwd"]
    bwd_ms = phases["attn_bwd"]
    if wl == "v4":
        kwork = step_kernel_work(S, H, K, work["sum_keff"], pairs, S + S // 4, S // 4, d_qk=512, k_attn=K + 128,
                                 sink=True)
    else:
        s_kv = S // 4 if wl == "c4" else S
        kwork = step_kernel_work(S, H, K, work["sum_keff"], pairs if pairs is not None else S * (S + 1) // 2, s_kv,
                                 d_qk=512 if wl == "c4" else 576)
    traffic_of = (lambda name: measured_traffic(name, S, H, K)) if wl == "c3" else None
    ktable = kernel_table(ktimes, kwork, args.steps, traffic_of)
    # Dominant kernel: the kernel with the most time per step that has an algorithmic
    # roofline (every kernel of the step has one except the compressor's per-call geometry)
    dom = next((r for r in ktable if "frac" in r), None)
    if dom is not None:
        roof = dict(bound=dom["bound"], kernel=dom["kernel"], achieved=dom["achieved"], peak=dom["peak"],
                    unit=dom["unit"], frac=dom["frac"], traffic=dom.get("traffic"),
                    avg_launch_ms=dom["avg_launch_ms"], launches_per_step=dom["launches_per_step"],
                    share_of_step=dom["ms_per_step"] / ms_per_step)
        if dom["bound"] == "hbm":
            roof["algorithmic_bytes"] = dom["algorithmic_bytes"]
            if "intermediate_bytes" in dom:  # the design's own intermediates, outside `achieved`
                roof["intermediate_bytes"] = dom["intermediate_bytes"]
                roof["frac_with_intermediates"] = dom["frac_with_intermediates"]
        else:
            roof["algorithmic_flops"] = dom["algorithmic_flops"]
    else:  # (v4: the attention forward as a whole)
        roof = dict(bound="hbm", kernel="dsa_sparse_mla_fwd", achieved=work["attn_fwd_bytes"] / (fwd_ms * 1e-3) / 1e9,
                    peak=HBM_PEAK_GBPS, unit="GB/s", algorithmic_bytes=work["attn_fwd_bytes"], avg_launch_ms=fwd_ms,
                    traffic=None)
        roof["frac"] = roof["achieved"] / roof["peak"]
    attn_bytes = work["attn_fwd_bytes"] + work["attn_bwd_bytes"]
    roof_pair = dict(
        bound="hbm",
        ops="dsa_sparse_mla_fwd + dsa_sparse_mla_bwd",
        achieved=attn_bytes / ((fwd_ms + bwd_ms) * 1e-3) / 1e9,
        peak=HBM_PEAK_GBPS,
        unit="GB/s",
        algorithmic_bytes=attn_bytes,
    )
    roof_pair["frac"] = roof_pair["achieved"] / roof_pair["peak"]
    cfg.update(heads=H, d_qk=512 if wl in ("v4", "c4") else 576, d_v=512, topk=K, index_heads=64, index_dim=128, sum_k_eff=work["sum_keff"],
               indexer_pairs=pairs if pairs is not None else S * (S + 1) // 2)
    metric = "sparse-attn fwd+bwd tokens/s @S=8K,top-k 2048; % HBM / MFMA roofline"
    if wl != "c3":
        metric = f"sparse-attn fwd+bwd tokens/s, workload {wl}; % HBM / MFMA roofline"
    line = dict(
        metric=metric,
        value=S / (ms_per_step * 1e-3),
        unit="tokens/s",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
        ms_per_step=ms_per_step,
        higher_is_better=True,
        scaling="weak",
        vs_baseline=None,
        dtype="bf16 (attention), fp8-e4m3 (indexer)",
        data="synthetic, seeded N(0,1) inputs",
        config=cfg,
        roofline=roof,
        roofline_attention_fwd_bwd=roof_pair,
        kernels_in_step=[{k: (round(v, 6) if isinstance(v, float) else v) for k, v in r.items()} for r in ktable],
        phases_ms={k: round(v, 4) for k, v in phases.items()},
        attn_mfma=dict(fwd_tflops=work["attn_fwd_flops"] / (fwd_ms * 1e-3) / 1e12,
                       bwd_tflops=work["attn_bwd_flops"] / (bwd_ms * 1e-3) / 1e12, peak_tflops=BF16_PEAK_TFLOPS),
    )
    idx_ms = phases["indexer_topk"]
    line["indexer_topk"] = dict(flops=work["indexer_flops"], ms_with_topk=idx_ms,
                                tflops_with_topk=work["indexer_flops"] / (idx_ms * 1e-3) / 1e12)
    if wl == "c3":
        # the step's own indexer kernels (fused indexer + top-k: the linear-split pre-pass and
        # the score kernel, masked spans left unwritten), from the in-step event timing; the
        # standalone dsa_indexer_fwd_ws call (which also writes -inf over the masked spans) is
        # reported beside it
        in_step = [r for r in ktable if r["kernel"].startswith(("indexer_lin_pieces_kernel", "indexer_tile_kernel"))]
        step_idx_ms = sum(r["ms_per_step"] for r in in_step)
        idx_kernel_ms = time_indexer_kernel(inp, ops, torch)
        line["indexer_mfma"] = dict(kernel=" + ".join(r["kernel"] for r in in_step), bound="mfma",
                                    flops=work["indexer_flops"], ms_per_step=step_idx_ms,
                                    achieved_tflops=work["indexer_flops"] / (step_idx_ms * 1e-3) / 1e12,
                                    peak_tflops=FP8_PEAK_TFLOPS,
                                    frac=work["indexer_flops"] / (step_idx_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS,
                                    standalone_fwd_ws_ms=idx_kernel_ms,
                                    standalone_frac=work["indexer_flops"] / (idx_kernel_ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS,
                                    ms_with_topk=idx_ms)
    if wl in ("c3", "c4"):
        line["kernels"] = kernel_rooflines(inp, ops, torch, dev, S, K, args.seed, with_topk=wl == "c3")
    if wl == "c3" and not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(inp, S, H, K, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
