"""bench.py's host-side contract: the one-GPU guard and the algorithmic byte / FLOP
accounting behind its roofline figures, checked against the closed forms of the
measured configurations (S=8192 causal with top-k 2048; the C4 compressor shapes)."""

import os
import subprocess
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def _causal_indices(S, K, valid_of_row):
    s = torch.arange(S).unsqueeze(1)
    j = torch.arange(K).unsqueeze(0)
    n = valid_of_row(s)
    return torch.where(j < n, j, torch.full_like(j, -1)).unsqueeze(0)


def test_c3_attention_bytes_match_closed_form():
    S, H, K = 8192, 128, 2048
    idx = _causal_indices(S, K, lambda s: torch.clamp(s + 1, max=K))
    w = bench.algorithmic_work(S, H, K, idx)
    # sum over rows of min(K, s + 1): 2048*2049/2 + (8192 - 2048) * 2048
    assert w["sum_keff"] == K * (K + 1) // 2 + (S - K) * K == 14_681_088
    assert round(w["attn_fwd_bytes"] / 1e10, 3) == 1.927
    assert round(w["attn_bwd_bytes"] / 1e10, 3) == 5.537
    assert round((w["attn_fwd_bytes"] + w["attn_bwd_bytes"]) / 1e10, 3) == 7.464
    assert w["indexer_flops"] == 2 * 64 * 128 * S * (S + 1) // 2
    assert w["topk_bytes"] == 4 * S * (S + 1) // 2 + 4 * K * S
    assert w["attn_fwd_flops"] == 2 * H * (576 + 512) * w["sum_keff"]


def test_compressed_pairs_and_keff():
    # C4: row s sees the (s + 1) // 4 whole compressed blocks; top-k 2048 of them
    S, K = 32768, 2048
    pairs = sum((s + 1) // 4 for s in range(S))
    assert pairs == sum(min(c, S // 4) for c in ((s + 1) // 4 for s in range(S)))
    keff = sum(min(K, (s + 1) // 4) for s in range(S))
    assert round(keff / 1e7, 2) == 5.87


def test_compressor_bytes_c4():
    # wkv and wgate projections read once (fp32, coff = 2), ape, bf16 rows out; D = 512 + 128
    total = 0
    for D in (512, 128):
        c = dict(S=32768, D=D, ratio=4, coff=2)
        b = bench.compressor_bytes(c)
        assert b == 2 * 32768 * 2 * D * 4 + 4 * 2 * D * 4 + 8192 * D * 2
        total += b
    assert round(total / 1e8, 2) == 3.46


def test_kernel_table_rooflines_per_bound():
    """Per-kernel rows: HBM kernels against 8 TB/s, the fp8 indexer against the fp8 peak, the
    bf16 indexer against the bf16 peak; the attention mass kernel's bytes follow its formula
    (Q, the gathered rows, indices, row statistics, mass) and the 512-column names map."""
    S, H, K, P, pairs = 8192, 128, 2048, 14_681_088, 8192 * 8193 // 2
    w = bench.step_kernel_work(S, H, K, P, pairs, S)
    bound, nbytes, flops, inter = w["attn_mass_bf16_kernel"]
    assert bound == "hbm" and flops == 2 * H * 576 * P
    assert nbytes == 2 * H * 576 * S + 2 * 576 * P + 4 * K * S + 8 * H * S and inter == 4 * K * S
    w512 = bench.step_kernel_work(S, H, K, P, pairs, S, d_qk=512)
    assert "attn_mass_bf16_kernel<512>" in w512 and w512["attn_mass_bf16_kernel<512>"][2] == 2 * H * 512 * P
    ktimes = {"indexer_tile_kernel<fp8, 4, split>": (0.5, 2), "indexer_tile_kernel": (1.0, 2),
              "attn_mass_bf16_kernel": (4.0, 2)}
    rows = {r["kernel"]: r for r in bench.kernel_table(ktimes, w, steps=2)}
    fp8, b16, mass = rows["indexer_tile_kernel<fp8, 4, split>"], rows["indexer_tile_kernel"], rows["attn_mass_bf16_kernel"]
    assert fp8["peak"] == bench.FP8_PEAK_TFLOPS and b16["peak"] == bench.BF16_PEAK_TFLOPS
    assert abs(b16["frac"] - 2 * 64 * 128 * pairs / 0.5e-3 / 1e12 / bench.BF16_PEAK_TFLOPS) < 1e-9
    assert mass["unit"] == "GB/s" and abs(mass["achieved"] - nbytes / 2e-3 / 1e9) < 1e-6
    assert abs(mass["frac_with_intermediates"] - (nbytes + inter) / 2e-3 / 1e9 / bench.HBM_PEAK_GBPS) < 1e-9
    assert rows["attn_mass_bf16_kernel"]["ms_per_step"] == 2.0


def test_backward_bytes_split_into_contract_and_intermediate():
    """The attention backward's per-kernel bytes: the survey's formula counts Q and dQ, O and
    dO, the row statistics, the indices, the gathered rows and a 4-byte-per-element dKV
    scatter payload; here the payload is the bf16 contribution rows written by the
    contribution kernel and read by the reduction (2 + 2 bytes).  G (dS | P per head), the
    delta, the mass and the pair lists are design intermediates, kept out of ``frac``."""
    S, H, K, P, pairs = 8192, 128, 2048, 14_681_088, 8192 * 8193 // 2
    w = bench.step_kernel_work(S, H, K, P, pairs, S)
    G = 2 * 256 * P  # bf16 dS and P of 128 heads per (row, slot)
    # with no sink the score kernel forms delta from O itself: O is its contract read, no
    # delta buffer; with a sink the delta pass reads O and dO and the score kernel the delta
    assert w["bwd_sdp_kernel"][3] == G + 4 * K * S
    assert w["bwd_sdp_kernel"][1] == 2 * H * 576 * S + 2 * 2 * H * 512 * S + 2 * 576 * P + 4 * K * S + 8 * H * S
    ws = bench.step_kernel_work(S, H, K, P, pairs, S, sink=True)
    assert ws["bwd_sdp_kernel"][3] == G + 4 * K * S + 4 * H * S
    assert ws["bwd_sdp_kernel"][1] + ws["bwd_delta_kernel"][1] == w["bwd_sdp_kernel"][1] + 2 * H * 512 * S
    assert w["bwd_dqk_kernel"][3] == G // 2
    assert w["bwd_contrib_kernel<2>"][3] == G
    assert w["bwd_contrib_kernel<2>"][1] == 2 * H * (576 + 512) * S + 4 * K * S + 2 * 576 * P
    assert w["dkv_reduce_kernel<72>"][1] == 2 * 576 * P + 4 * 576 * S
    # the two halves of the contribution round trip are exactly the survey's scatter payload
    payload = (w["bwd_contrib_kernel<2>"][1] - 2 * H * (576 + 512) * S - 4 * K * S) + \
        (w["dkv_reduce_kernel<72>"][1] - 4 * 576 * S)
    assert payload == 4 * 576 * P
    assert all(w[k][1] == 0 for k in ("csr_count_kernel<count>", "csr_count_kernel<fill>", "csr_fill_staged_kernel",
                                      "csr_scan_kernel"))
    ktimes = {"bwd_contrib_kernel<2>": (5.0, 1), "csr_count_kernel<fill>": (0.2, 1)}
    rows = {r["kernel"]: r for r in bench.kernel_table(ktimes, w, steps=1)}
    beta = rows["bwd_contrib_kernel<2>"]
    assert beta["frac"] < beta["frac_with_intermediates"]
    assert abs(beta["frac"] - w["bwd_contrib_kernel<2>"][1] / 5e-3 / 1e9 / bench.HBM_PEAK_GBPS) < 1e-9
    assert rows["csr_count_kernel<fill>"]["frac"] == 0.0
