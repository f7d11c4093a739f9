"""The indexer input producer (dsa_indexer_prep) and the compressor's RoPE epilogue on the
GPU, against the oracle.

bf16 outputs, stage by stage: the kernel computes in fp32 where the oracle is exact, so a
value may land one bf16 ulp away next to a rounding boundary, or, where the exact result
cancels, within the kernel's fp32 rounding of the operands' magnitude (2^-18 of it); at
most 1 in 1000 values differ.  The RoPE output is checked against the oracle's RoPE, and
the full output against the oracle's Hadamard rotation of the kernel's own RoPE output (a
flipped rounding in the first stage moves every output of its row).  fp8: the bytes and scales equal the oracle's
quantize_e4m3_per_row of the kernel's own bf16 output (bit-exact).  Compressor: fp32 1e-5,
bf16 2e-2 relative (its usual bars), the RoPE at the blocks' positions included.
"""

import pytest
import torch

from oracle import dsa_oracle as O
from tests.dsa_cases import rel_err

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _ops():
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    return ops


def _freqs(n_pos, rope_dim=64, base=10000.0):
    inv = 1.0 / (base ** (torch.arange(0, rope_dim, 2, dtype=torch.float64) / rope_dim))
    ang = torch.outer(torch.arange(n_pos, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang).to(torch.complex64)


def _bf16_check(got, ref, scale, what):
    """Each value within one bf16 ulp of the oracle, or within 2^-18 of ``scale`` (the
    magnitude the kernel's fp32 arithmetic works at, which bounds its rounding where the
    exact result cancels); at most 1 in 1000 values off at all."""
    g, r = got.float().cpu(), ref.float().cpu()
    exp = torch.frexp(r.abs().clamp_min(1e-30))[1]
    ulp = torch.ldexp(torch.ones_like(r), exp - 8)  # bf16 has 8 significant bits
    d = (g - r).abs()
    ok = (d <= ulp * (1 + 1e-6)) | (d <= scale.expand_as(d) * 2.0 ** -18)
    bad = int((~ok).sum())
    frac = float((d > 0).float().mean())
    assert bad == 0, f"{what}: {bad} values beyond the bound (worst {float((d / ulp).max()):.1f} ulp)"
    assert frac <= 1e-3, f"{what}: {frac:.2e} of the values differ"
    return frac


def _check_prep(ops, x, freqs, positions, pos_offset, pos_flat, layout, **kw):
    """Two stages: the kernel's RoPE output against the oracle's RoPE, then the kernel's full
    output against the oracle's Hadamard of the kernel's own RoPE output; fp8 bit-exact."""
    n = pos_flat.numel()
    rows_shape = (n, *x.shape[(2 if layout == "BSND" else 1):])
    p = None if positions is None else positions.to(DEV)
    r_gpu, _, _ = ops.indexer_prep(x.to(DEV), freqs, positions=p, pos_offset=pos_offset, hadamard=False, fp8=False,
                                   layout=layout, **kw)
    y, q8, sc = ops.indexer_prep(x.to(DEV), freqs, positions=p, pos_offset=pos_offset, layout=layout, **kw)
    torch.cuda.synchronize()
    xt = x.reshape(rows_shape)
    r_gpu = r_gpu.reshape(rows_shape).cpu()
    f1 = 0.0
    if freqs is not None:
        r_ref = O.rope_rotate(xt, freqs, pos_flat, rope_start=kw["rope_start"], interleaved=kw["interleaved"])
        f1 = _bf16_check(r_gpu, r_ref, 2 * xt.float().abs().amax(-1, keepdim=True), "rope")
    y_ref = O.hadamard_rotate(r_gpu)
    f2 = _bf16_check(y.reshape(rows_shape), y_ref, r_gpu.float().abs().sum(-1, keepdim=True) * 128 ** -0.5,
                     "hadamard")
    rq, rs = O.quantize_e4m3_per_row(y.float().cpu())
    assert torch.equal(q8.cpu().view(torch.uint8), rq.view(torch.uint8)), "fp8 bytes"
    assert torch.equal(sc.cpu(), rs), "fp8 scales"
    return f1, f2


@pytest.mark.parametrize("variant", ["v32", "v4", "hadamard_only"])
def test_indexer_prep_parity(variant):
    ops = _ops()
    B, S, H = 2, 96, 64
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, S, H, 128, generator=g).bfloat16()
    k = torch.randn(B, S, 128, generator=g).bfloat16()
    fc = _freqs(512)
    kw = dict(v32=dict(rope_start=0, interleaved=False), v4=dict(rope_start=64, interleaved=True),
              hadamard_only=dict(rope_start=0, interleaved=False))[variant]
    freqs = None if variant == "hadamard_only" else fc
    positions = torch.randint(0, 512, (B, S), generator=g) if variant == "v4" else None
    pos = positions.reshape(-1) if positions is not None else (torch.arange(S) + 3).repeat(B)
    for x in (q, k):
        f1, f2 = _check_prep(ops, x, freqs, positions, 3, pos, "BSND", **kw)
        print(f"[prep] {variant} {tuple(x.shape)}: rope {f1:.2e}, hadamard {f2:.2e} of the values differ", flush=True)


def test_indexer_prep_packed_rows_and_outputs():
    ops = _ops()
    T = 75
    g = torch.Generator().manual_seed(12)
    x = torch.randn(T, 64, 128, generator=g).bfloat16()
    pos = torch.randint(0, 100, (T,), generator=g)
    keep = torch.arange(T) != 5
    fc = _freqs(100)
    _check_prep(ops, x[keep], fc, pos[keep], 0, pos[keep], "TND", rope_start=0, interleaved=False)
    pos[5] = 200  # outside the table: that row keeps its features (no rotation)
    r_gpu, _, _ = ops.indexer_prep(x.to(DEV), fc, positions=pos.to(DEV), layout="TND", hadamard=False, fp8=False)
    assert torch.equal(r_gpu[5].cpu(), x[5])
    y, q8, sc = ops.indexer_prep(x.to(DEV), fc, positions=pos.to(DEV), layout="TND", fp8=False)
    assert q8 is None and sc is None
    y2, q82, sc2 = ops.indexer_prep(x.to(DEV), fc, positions=pos.to(DEV), layout="TND", return_bf16=False)
    assert y2 is None
    rq, rs = O.quantize_e4m3_per_row(y.float().cpu())
    assert torch.equal(q82.cpu().view(torch.uint8), rq.view(torch.uint8)) and torch.equal(sc2.cpu(), rs)


@pytest.mark.parametrize("D,r,norm", [(512, 4, True), (128, 4, True), (512, 128, True), (128, 4, False)])
def test_compressor_rope_epilogue(D, r, norm):
    ops = _ops()
    B, S = 2, 64 * r // 4 if r == 4 else 256
    g = torch.Generator().manual_seed(D + r)
    coff = 2 if r == 4 else 1
    kv = torch.randn(B, S, coff * D, generator=g)
    sc = torch.randn(B, S, coff * D, generator=g)
    ape = torch.randn(r, coff * D, generator=g) * 0.02
    w = torch.rand(D, generator=g) + 0.5 if norm else None
    fc = _freqs(S)
    positions = torch.randint(0, S, (B, S), generator=g)
    for pos in (None, positions):
        got = ops.compressor_pool(kv.to(DEV), sc.to(DEV), ape.to(DEV), r, norm_weight=None if w is None else w.to(DEV),
                                  freqs_cis=fc, positions=None if pos is None else pos.to(DEV)).cpu()
        ref = O.compressor_pool(kv.double() if not norm else kv, sc.double() if not norm else sc,
                                ape.double() if not norm else ape, r, norm_weight=w,
                                out_dtype=torch.bfloat16 if norm else None, freqs_cis=fc, positions=pos)
        tol = 2e-2 if norm else 1e-5
        assert rel_err(got.float(), ref) <= tol, rel_err(got.float(), ref)


def test_compressor_tnd_rope_epilogue():
    from torchtitan_npu_simulator_amd import tnd

    ops = _ops()
    D, r = 128, 4
    pos = torch.cat([torch.arange(5, 5 + 23), torch.arange(0, 10), torch.arange(0, 41)])
    T = pos.numel()
    g = torch.Generator().manual_seed(17)
    kv = torch.randn(T, 2 * D, generator=g)
    sc = torch.randn(T, 2 * D, generator=g)
    ape = torch.randn(r, 2 * D, generator=g) * 0.02
    w = torch.rand(D, generator=g) + 0.5
    bs = tnd.compressed_block_starts(pos, r)
    fc = _freqs(64)
    got = ops.compressor_pool_tnd(kv.to(DEV), sc.to(DEV), ape.to(DEV), r, bs.to(DEV), pos.to(DEV),
                                  norm_weight=w.to(DEV), freqs_cis=fc).cpu()
    ref = O.compressor_pool_tnd(kv, sc, ape, r, bs, pos, norm_weight=w, out_dtype=torch.bfloat16, freqs_cis=fc)
    assert rel_err(got.float(), ref) <= 2e-2
