"""The C-ABI library builds for gfx950, loads, and exports every symbol include/dsa_mi355x.h declares.

No compute entry point is called here (there is no GPU in the CPU suite); the host
op layer is checked to refuse CPU tensors instead of falling back to any CPU path.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dsa_mi355x.h"


def header_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from torchtitan_npu_simulator_amd import _lib

    if not _lib.LIB_PATH.exists():
        from torchtitan_npu_simulator_amd import build

        build.build()
    return _lib.load_library()


def test_header_declares_the_entry_points():
    syms = header_symbols()
    for name in ("dsa_indexer_fwd", "dsa_topk", "dsa_sparse_mla_fwd", "dsa_sparse_mla_bwd",
                 "dsa_indexer_kl_grad", "dsa_compressor_fwd", "dsa_last_error"):
        assert name in syms


def test_library_exports_every_header_symbol(lib):
    from torchtitan_npu_simulator_amd import _lib

    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in header_symbols() if not hasattr(raw, s)]
    assert not missing, missing
    # the ctypes signature table covers exactly the header
    assert sorted(_lib.exported_symbols()) == header_symbols()


def test_abi_version_and_error_text(lib):
    from torchtitan_npu_simulator_amd import _lib

    assert lib.dsa_abi_version() == _lib.ABI_VERSION
    assert isinstance(lib.dsa_last_error(), bytes)


def test_ops_refuse_cpu_tensors(lib):
    from torchtitan_npu_simulator_amd import DSAError
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    q = torch.zeros(1, 4, 2, 576, dtype=torch.bfloat16)
    kv = torch.zeros(1, 4, 576, dtype=torch.bfloat16)
    idx = torch.zeros(1, 4, 2, dtype=torch.int32)
    with pytest.raises(DSAError):
        ops.sparse_mla_fwd(q, kv, idx, 0.1)
    with pytest.raises(DSAError):
        ops.indexer_scores(torch.zeros(1, 4, 2, 8), torch.zeros(1, 4, 8), torch.zeros(1, 4, 2))


def test_indexer_workspace_size(lib):
    """The linear-split workspace (four fp8 pieces of 128 bytes and their fp32 scales per
    query row) is sized for fp8 with H_I=64, D_I=128 only; other shapes need none."""
    from torchtitan_npu_simulator_amd import _lib

    fp8, bf16 = _lib.dtype_code(torch.float8_e4m3fn), _lib.dtype_code(torch.bfloat16)
    assert lib.dsa_indexer_fwd_workspace_size(2, 8192, 64, 128, fp8) == 2 * 8192 * (4 * 128 + 4 * 4)
    assert lib.dsa_indexer_fwd_workspace_size(1, 8192, 64, 128, bf16) == 0
    assert lib.dsa_indexer_fwd_workspace_size(1, 8192, 32, 128, fp8) == 0
    assert lib.dsa_indexer_fwd_workspace_size(1, 0, 64, 128, fp8) == 0


@pytest.mark.parametrize("B,S,s_k", [(2, 700, 700), (8, 512, 4096), (1, 700, 700)])
def test_lightning_indexer_workspace_respects_the_score_budget(lib, B, S, s_k):
    """The fused indexer's workspace stays within the score budget when all batches do not
    fit at once (the C entry then goes batch by batch): scores of one budget's worth of rows
    plus the fp8 split pieces of those rows."""
    from torchtitan_npu_simulator_amd import _lib
    from torchtitan_npu_simulator_amd import torch_npu_ops as ops

    fp8 = _lib.dtype_code(torch.float8_e4m3fn)
    budget = S * s_k * 4  # exactly one batch of score rows
    ws = ops.lightning_indexer_workspace_bytes(lib, B, S, s_k, 64, 128, fp8, budget=budget)
    pieces = lib.dsa_indexer_fwd_workspace_size(1, S, 64, 128, fp8)
    assert ws <= budget + 256 + pieces
    if B > 1:
        small = ops.lightning_indexer_workspace_bytes(lib, B, S, s_k, 64, 128, fp8, budget=budget - 4 * s_k)
        assert small <= budget - 4 * s_k + 256 + pieces
    big = ops.lightning_indexer_workspace_bytes(lib, B, S, s_k, 64, 128, fp8, budget=B * S * s_k * 4)
    assert big >= B * S * s_k * 4  # everything in one pass when it fits
