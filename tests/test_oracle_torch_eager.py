"""Pins oracle/torch_eager.py (the reference's CPU PyTorch step, timed as the CPU baseline).

With integer ranks and B in multiples of 1/64 every dot product is exact under
any summation order, so the torch bf16 path must reproduce the numpy oracle's
eager bf16 restatement id for id, and the fp32 path the fused argmax's ids
wherever the top-2 margin pins them.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_eager


def _case(seed, M=6, d=64, r=32, V=3001):
    rng = np.random.default_rng(seed)
    h = rng.integers(-1, 2, (M, d)).astype(np.float32)
    A = (rng.integers(-1, 2, (r, d)) * (rng.random((r, d)) < 0.1)).astype(np.float32)
    B = (rng.integers(-64, 65, (V, r)) / 64).astype(np.float32)
    base = oracle.bf16_round((rng.standard_normal((M, V)) * 3).astype(np.float32))
    prior = oracle.bf16_round(np.log(rng.dirichlet(np.ones(V))).astype(np.float32))
    alpha = rng.uniform(0.05, 0.6, M).astype(np.float32)
    beta = rng.uniform(0.05, 0.6, M).astype(np.float32)
    beta[1] = 0.0
    return h, A, B, base, prior, alpha, beta


@pytest.mark.parametrize("seed,act", [(0, "identity"), (1, "silu"), (2, "identity")])
def test_eager_bf16_matches_numpy_restatement(seed, act):
    h, A, B, base, prior, alpha, beta = _case(seed)
    t = torch.from_numpy
    ids = torch_eager.eager_step_bf16(t(h), t(A), t(B), t(base), t(prior), t(alpha), t(beta), act).numpy()
    rank = oracle.rank_proj(h, A, None, act)
    want = oracle.eager_argmax_bf16(rank, B, base, prior, alpha, beta)
    np.testing.assert_array_equal(ids, want)
    # without a prior the beta term drops out entirely
    ids0 = torch_eager.eager_step_bf16(t(h), t(A), t(B), t(base), None, t(alpha), t(beta), act).numpy()
    np.testing.assert_array_equal(ids0, oracle.eager_argmax_bf16(rank, B, base, None, alpha, beta))


@pytest.mark.parametrize("seed", [3, 4])
def test_fp32_step_matches_fused_argmax(seed):
    h, A, B, base, prior, alpha, beta = _case(seed, M=12)
    t = torch.from_numpy
    ids = torch_eager.step_fp32(t(h), t(A), t(B), t(base), t(prior), t(alpha), t(beta)).numpy()
    rank = oracle.rank_proj(h, A)
    rid, rsc, rsec = oracle.fused_argmax(rank, B, base, prior, alpha, beta)
    res = oracle.check_parity(ids, None, rid, rsc, rsec)
    assert res["id_mismatch_pinned"] == 0 and res["pinned"] >= 10, res
