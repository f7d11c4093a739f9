"""The committed golden fixtures still agree with the oracle and with independent checks."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O
from tests.golden.make_golden import CASES, load
from tests.test_oracle import _brute_topk


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_reproduced_by_oracle(name):
    meta, z = load(name)
    qo = meta["q_offset"]
    scores = O.indexer_scores(z["q_idx"], z["k_idx"], z["w"], q_offset=qo)
    assert torch.equal(scores, z["scores"])
    idx = O.topk_select(scores, meta["K"], q_offset=qo)
    assert torch.equal(idx, z["indices"])
    out, lse = O.sparse_mla_fwd(z["q"], z["kv"], idx, meta["scale"], q_offset=qo)
    torch.testing.assert_close(out.float(), z["out"], rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(lse.float(), z["lse"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_topk_is_brute_force_selection(name):
    meta, z = load(name)
    S, K, qo = meta["S"], meta["K"], meta["q_offset"]
    sc = z["scores"][0].numpy()
    for s in range(S):
        assert list(z["indices"][0, s].numpy()) == _brute_topk(sc[s].tolist(), K, s + qo + 1)


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_gradient_checksums(name):
    meta, z = load(name)
    # sum_j kv_j . dKV_j == sum q . dQ + sum O . dO (k_nope and v alias the latent)
    lhs = (z["kv"].double() * z["dkv"].double()).sum()
    rhs = (z["q"].double() * z["dq"].double()).sum() + (z["out"].double() * z["dout"].double()).sum()
    assert abs(float(lhs - rhs)) <= 1e-4 * max(1.0, abs(float(rhs)))
    # the head-summed mass never exceeds the head count and is zero on -1 slots
    m = z["mass"]
    assert float(m.sum(-1).max()) <= meta["H"] + 1e-5
    assert float(m.masked_select(z["indices"] < 0).abs().sum()) == 0.0
    assert np.isfinite(float(z["loss"][0])) and float(z["loss"][0]) >= 0.0
