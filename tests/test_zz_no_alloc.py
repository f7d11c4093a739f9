"""dsa_indexer_fwd_noalloc (the entry point that allocates nothing) through the C ABI.

Its scores must equal dsa_indexer_fwd_ws's with a caller workspace bit for bit (the same
kernels; only where the linear-split pieces live differs), on two calls in a row with the
second smaller than the first (the static scratch keeps the first call's pieces), and a
request above the scratch's row limit must be refused before anything is launched.
"""

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _lib():
    from torchtitan_npu_simulator_amd import _lib as L

    return L, L.load_library()


def _case(S, s_k, seed, fp8=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(1, S, 64, 128, device=DEV, generator=g)
    k = torch.randn(1, s_k, 128, device=DEV, generator=g)
    w = torch.randn(1, S, 64, device=DEV, generator=g) * 64 ** -0.5 * 128 ** -0.5
    if not fp8:
        return q.bfloat16(), None, k.bfloat16(), None, w
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    q8, qs = ops.quantize_fp8_per_row(q)
    k8, ks = ops.quantize_fp8_per_row(k)
    return q8, qs, k8, ks, w


def _scores(L, lib, q, qs, k, ks, w, q_offset, noalloc):
    S, s_k = q.shape[1], k.shape[1]
    out = torch.full((1, S, s_k), float("nan"), device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    dt = L.dtype_code(q.dtype)
    args = (L.ptr(q), L.ptr(qs), L.ptr(k), L.ptr(ks), L.ptr(w), L.ptr(out), dt, 1, S, s_k, 64, 128, s_k, q_offset, 1)
    if noalloc:
        rc = lib.dsa_indexer_fwd_noalloc(*args, st)
        L.check(rc, "dsa_indexer_fwd_noalloc")
    else:
        ws_bytes = int(lib.dsa_indexer_fwd_workspace_size(1, S, 64, 128, dt))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        L.check(lib.dsa_indexer_fwd_ws(*args, L.ptr(ws) if ws_bytes else None, ws_bytes, st), "dsa_indexer_fwd_ws")
    torch.cuda.synchronize()
    return out


def test_noalloc_equals_workspace_entry_point_twice():
    L, lib = _lib()
    assert lib.dsa_indexer_fwd_noalloc_max_rows() == (32 << 20) // (4 * 128 + 16)
    for S, s_k, q_off, seed in ((3000, 3000, 0, 1), (517, 2100, 1583, 2)):  # second call smaller
        q, qs, k, ks, w = _case(S, s_k, seed)
        got = _scores(L, lib, q, qs, k, ks, w, q_off, noalloc=True)
        ref = _scores(L, lib, q, qs, k, ks, w, q_off, noalloc=False)
        assert not bool(torch.isnan(got).any()), f"S={S}: scores left unwritten"
        assert torch.equal(got, ref), f"S={S}: noalloc scores differ from dsa_indexer_fwd_ws"
        # and the oracle's selection on them is the op's (one row block, bit-exact top-k)
        nv = [O.valid_key_count(s, q_off, 1, s_k) for s in range(S)]
        assert torch.equal(torch.isfinite(got[0]).sum(-1).cpu(), torch.tensor(nv))


def test_noalloc_other_shapes_run_the_plain_kernels():
    L, lib = _lib()
    q, qs, k, ks, w = _case(200, 200, 3, fp8=False)
    got = _scores(L, lib, q, qs, k, ks, w, 0, noalloc=True)
    ref = _scores(L, lib, q, qs, k, ks, w, 0, noalloc=False)
    assert torch.equal(got, ref)


def test_noalloc_refuses_rows_beyond_its_scratch():
    from torchtitan_npu_simulator_amd import DSAError

    L, lib = _lib()
    rows = int(lib.dsa_indexer_fwd_noalloc_max_rows()) + 1
    q = torch.empty(1, rows, 64, 128, dtype=torch.float8_e4m3fn, device=DEV)
    k = torch.empty(1, 16, 128, dtype=torch.float8_e4m3fn, device=DEV)
    w = torch.empty(1, rows, 64, device=DEV)
    out = torch.empty(1, rows, 16, device=DEV)
    rc = lib.dsa_indexer_fwd_noalloc(L.ptr(q), None, L.ptr(k), None, L.ptr(w), L.ptr(out), L.DSA_FP8_E4M3, 1, rows,
                                     16, 64, 128, 16, 0, 1, torch.cuda.current_stream().cuda_stream)
    assert rc == 1  # DSA_ERR_INVALID_ARG
    with pytest.raises(DSAError, match="static scratch"):
        L.check(rc, "dsa_indexer_fwd_noalloc")
