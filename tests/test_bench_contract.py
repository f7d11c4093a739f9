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
    bound, nbytes, flops = w["attn_mass_bf16_kernel"]
    assert bound == "hbm" and flops == 2 * H * 576 * P
    assert nbytes == 2 * H * 576 * S + 2 * 576 * P + 8 * K * S + 8 * H * S
    w512 = bench.step_kernel_work(S, H, K, P, pairs, S, d_qk=512)
    assert "attn_mass_bf16_kernel<512>" in w512 and w512["attn_mass_bf16_kernel<512>"][2] == 2 * H * 512 * P
    ktimes = {"indexer_tile_kernel<fp8, 4, split>": (0.5, 2), "indexer_tile_kernel": (1.0, 2),
              "attn_mass_bf16_kernel": (4.0, 2)}
    rows = {r["kernel"]: r for r in bench.kernel_table(ktimes, w, steps=2)}
    fp8, b16, mass = rows["indexer_tile_kernel<fp8, 4, split>"], rows["indexer_tile_kernel"], rows["attn_mass_bf16_kernel"]
    assert fp8["peak"] == bench.FP8_PEAK_TFLOPS and b16["peak"] == bench.BF16_PEAK_TFLOPS
    assert abs(b16["frac"] - 2 * 64 * 128 * pairs / 0.5e-3 / 1e12 / bench.BF16_PEAK_TFLOPS) < 1e-9
    assert mass["unit"] == "GB/s" and abs(mass["achieved"] - nbytes / 2e-3 / 1e9) < 1e-6
    assert rows["attn_mass_bf16_kernel"]["ms_per_step"] == 2.0
