"""Pins of the oracle's indexer input producer and the compressor's RoPE epilogue (CPU).

Each check is independent of the oracle's own formula: explicit per-pair loops for the
rotary embedding in both pair layouts, the algebra of the Hadamard matrix (orthogonal,
symmetric, one-hot columns), and compositions of those with the reference's bf16
rounding points.
"""

import math

import numpy as np
import pytest
import torch
from scipy.linalg import hadamard

from oracle import dsa_oracle as O


def _freqs(n_pos, rope_dim, base=10000.0, dtype=torch.complex64):
    inv = 1.0 / (base ** (torch.arange(0, rope_dim, 2, dtype=torch.float64) / rope_dim))
    ang = torch.outer(torch.arange(n_pos, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang).to(dtype)


def _rope_loop(x, fc, pos, rope_dim, rope_start, interleaved):
    """Pair i of token n rotated by fc[pos[n], i], one pair at a time (fp64)."""
    out = x.to(torch.float64).clone()
    half = rope_dim // 2
    for n in range(x.shape[0]):
        for i in range(half):
            if interleaved:
                ia, ib = rope_start + 2 * i, rope_start + 2 * i + 1
            else:
                ia, ib = rope_start + i, rope_start + i + half
            c, s = float(fc[pos[n], i].real), float(fc[pos[n], i].imag)
            a, b = x[n, ..., ia].double(), x[n, ..., ib].double()
            out[n, ..., ia] = a * c - b * s
            out[n, ..., ib] = a * s + b * c
    return out


@pytest.mark.parametrize("interleaved,rope_start", [(False, 0), (True, 64), (True, 0)])
def test_rope_matches_pair_loops(interleaved, rope_start):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(6, 3, 128, generator=g, dtype=torch.float64)
    fc = _freqs(40, 64)
    pos = torch.tensor([0, 5, 39, 7, 7, 12])
    got = O.rope_rotate(x, fc, pos, rope_dim=64, rope_start=rope_start, interleaved=interleaved,
                        out_dtype=torch.float64)
    ref = _rope_loop(x, fc, pos, 64, rope_start, interleaved)
    torch.testing.assert_close(got, ref, rtol=1e-6, atol=1e-6)  # fc is complex64


def test_rope_identity_inverse_and_norms():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 128, generator=g, dtype=torch.float64)
    fc = _freqs(16, 64, dtype=torch.complex128)
    zero = torch.zeros(5, dtype=torch.long)
    torch.testing.assert_close(O.rope_rotate(x, fc, zero, out_dtype=torch.float64), x, rtol=0, atol=0)
    pos = torch.tensor([1, 3, 15, 8, 2])
    y = O.rope_rotate(x, fc, pos, rope_dim=64, rope_start=64, interleaved=True, out_dtype=torch.float64)
    back = O.rope_rotate(y, fc.conj(), pos, rope_dim=64, rope_start=64, interleaved=True, out_dtype=torch.float64)
    torch.testing.assert_close(back, x, rtol=1e-12, atol=1e-12)
    pairs_x = x[:, 64:].reshape(5, 32, 2).norm(dim=-1)
    pairs_y = y[:, 64:].reshape(5, 32, 2).norm(dim=-1)
    torch.testing.assert_close(pairs_y, pairs_x, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(y[:, :64], x[:, :64], rtol=0, atol=0)  # features outside the rope part


def test_hadamard_algebra():
    H = torch.tensor(hadamard(128), dtype=torch.float64)
    assert torch.equal(H, H.T) and torch.equal(H @ H, 128 * torch.eye(128, dtype=torch.float64))
    g = torch.Generator().manual_seed(3)
    x = torch.randn(7, 128, generator=g, dtype=torch.float64)
    y = O.hadamard_rotate(x, out_dtype=torch.float64)
    torch.testing.assert_close(O.hadamard_rotate(y, out_dtype=torch.float64), x, rtol=1e-12, atol=1e-12)
    e = torch.zeros(1, 128, dtype=torch.float64)
    e[0, 37] = 1.0
    torch.testing.assert_close(O.hadamard_rotate(e, out_dtype=torch.float64)[0], H[:, 37] / math.sqrt(128))
    # Sylvester order: H[i][j] = (-1)^popcount(i & j)
    i = torch.arange(128)
    pc = torch.tensor([[bin(a & b).count("1") for b in range(128)] for a in range(128)])
    assert torch.equal(H, (1 - 2 * (pc % 2)).double())
    del i


@pytest.mark.parametrize("interleaved,rope_start", [(False, 0), (True, 64)])
def test_indexer_prep_composition(interleaved, rope_start):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4, 2, 128, generator=g).bfloat16()
    fc = _freqs(8, 64)
    pos = torch.tensor([0, 3, 7, 1])
    y, q8, sc = O.indexer_prep(x, fc, pos, rope_start=rope_start, interleaved=interleaved)
    r = _rope_loop(x, fc, pos, 64, rope_start, interleaved).bfloat16()  # rope output in the model dtype
    h = (r.double() @ torch.tensor(hadamard(128), dtype=torch.float64).T).bfloat16()  # bf16 linear
    ref = (h.float() * np.float32(128 ** -0.5)).bfloat16()  # bf16 * python float
    assert torch.equal(y, ref)
    rq, rs = O.quantize_e4m3_per_row(ref.float())
    assert torch.equal(q8.view(torch.uint8), rq.view(torch.uint8)) and torch.equal(sc, rs)


def test_compressor_rope_epilogue_rotates_block_positions():
    g = torch.Generator().manual_seed(5)
    B, S, D, r = 2, 32, 128, 4
    kv = torch.randn(B, S, 2 * D, generator=g)
    sc = torch.randn(B, S, 2 * D, generator=g)
    ape = torch.randn(r, 2 * D, generator=g) * 0.02
    w = torch.rand(D, generator=g) + 0.5
    fc = _freqs(S, 64)
    base = O.compressor_pool(kv, sc, ape, r, norm_weight=w, out_dtype=torch.bfloat16)
    got = O.compressor_pool(kv, sc, ape, r, norm_weight=w, out_dtype=torch.bfloat16, freqs_cis=fc)
    for b in range(B):
        pos = torch.arange(S // r) * r
        ref = _rope_loop(base[b].bfloat16(), fc, pos, 64, D - 64, True)
        torch.testing.assert_close(got[b], ref, rtol=1e-6, atol=1e-6)
    # TND: block c at positions[block_starts[c]]
    positions = torch.cat([torch.arange(0, 12), torch.arange(0, 20)])
    bs = O.tnd_compressed_block_starts(positions, r)
    kt, st = kv[0], sc[0]
    base_t = O.compressor_pool_tnd(kt, st, ape, r, bs, positions, norm_weight=w, out_dtype=torch.bfloat16)
    got_t = O.compressor_pool_tnd(kt, st, ape, r, bs, positions, norm_weight=w, out_dtype=torch.bfloat16,
                                  freqs_cis=fc)
    ref_t = _rope_loop(base_t.bfloat16(), fc, positions[bs], 64, D - 64, True)
    torch.testing.assert_close(got_t, ref_t, rtol=1e-6, atol=1e-6)


def test_mla_absorb_oracle_against_loops_and_non_absorbed_attention():
    g = torch.Generator().manual_seed(9)
    B, S, H, R = 1, 6, 3, 32
    q_nope = torch.randn(B, S, H, 16, generator=g, dtype=torch.float64)
    q_pe = torch.randn(B, S, H, 8, generator=g, dtype=torch.float64)
    w_uk = torch.randn(H, 16, R, generator=g, dtype=torch.float64)
    q = O.mla_absorb_q(q_nope, q_pe, w_uk)
    for h in range(H):
        torch.testing.assert_close(q[0, :, h, :R], q_nope[0, :, h] @ w_uk[h])
    torch.testing.assert_close(q[..., R:], q_pe)
    # absorbed scores == explicit keys k_nope = kv_latent w_uk^T (plus the rope part)
    kv = torch.randn(B, S, R, generator=g, dtype=torch.float64)
    k_pe = torch.randn(B, S, 8, generator=g, dtype=torch.float64)
    scores = torch.einsum("bshd,btd->bhst", q, torch.cat([kv, k_pe], -1))
    k_nope = torch.einsum("btr,hqr->bhtq", kv, w_uk)
    explicit = torch.einsum("bshq,bhtq->bhst", q_nope, k_nope) + torch.einsum("bshp,btp->bhst", q_pe, k_pe)
    torch.testing.assert_close(scores, explicit)
    # absorbed output (P kv) w_uv == P (kv w_uv)
    P = torch.softmax(scores, dim=-1)
    w_uv_t = torch.randn(H, R, 10, generator=g, dtype=torch.float64)
    o_lat = torch.einsum("bhst,btr->bshr", P, kv)
    v = torch.einsum("btr,hrv->bhtv", kv, w_uv_t)
    torch.testing.assert_close(O.mla_absorb_out(o_lat, w_uv_t), torch.einsum("bhst,bhtv->bshv", P, v))
