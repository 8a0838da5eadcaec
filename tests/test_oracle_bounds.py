"""Pins oracle/bounds.py: the error bounds behind the fp8-vs-bf16 and eager-vs-fused id checks.

Two sides.  Domination: on random cases (several magnitudes, with and without
a prior, cancelling dot products) every entry's true difference between the
two paths' scores -- each computed by the oracle's own pinned functions, the
eager one by torch -- is within the bound.  Tightness: on constructed cases
whose rounding errors all point the same way the true difference reaches the
bound to within 1 %, so dropping or shrinking any term of the bound that
matters there (the rank term, the B term, their product, the alpha factor)
would break domination on that case.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import bounds, torch_eager

F32 = np.float32


def _scores_bf16(rank, B, base, prior, alpha, beta):
    """fp32-semantics scores of every (row, vocabulary) entry, through the oracle's score_at."""
    M, V = base.shape
    return np.stack([oracle.score_at(rank, B, base, prior, alpha, beta, np.full(M, v)) for v in range(V)], axis=1)


def _scores_fp8(rank8, Bq, sB, base, prior, alpha, beta):
    M, V = base.shape
    return np.stack([oracle.score_at_fp8(rank8, Bq, sB, base, prior, alpha, beta, np.full(M, v)) for v in range(V)],
                    axis=1)


def _bound_matrix_fp8(rank_b, rank8, B, Bq, sB, base, prior, alpha, beta):
    M, V = base.shape
    return np.stack([bounds.fp8_bound_at(rank_b, rank8, B, Bq, sB, base, prior, alpha, beta, np.full(M, v))
                     for v in range(V)], axis=1)


@pytest.mark.parametrize("seed,scale,with_prior", [(0, 0.02, True), (1, 1.0, False), (2, 30.0, True),
                                                   (3, 0.02, False)])
def test_fp8_bound_dominates(seed, scale, with_prior):
    rng = np.random.default_rng(seed)
    M, d, r, V = 7, 96, 64, 257
    h = oracle.bf16_round(rng.standard_normal((M, d)).astype(F32))
    A = oracle.bf16_round((rng.standard_normal((r, d)) * scale).astype(F32))
    B = oracle.bf16_round((rng.standard_normal((V, r)) * scale).astype(F32))
    A[3, :] = 0.0                                     # an all-zero channel (scale 1)
    base = (rng.standard_normal((M, V)) * 3).astype(F32)
    prior = np.log(rng.dirichlet(np.ones(V))).astype(F32) if with_prior else None
    alpha = rng.uniform(0.0, 2.0, M).astype(F32)
    beta = rng.uniform(0.0, 0.6, M).astype(F32)
    beta[0] = 0.0
    rank_b = oracle.rank_proj(h, A)
    Aq, sA = oracle.quantize_rows_e4m3(A)
    rank8 = oracle.rank_proj_fp8(h, Aq, sA)
    Bq, sB = oracle.quantize_rows_e4m3(B)
    diff = np.abs(_scores_fp8(rank8, Bq, sB, base, prior, alpha, beta).astype(np.float64)
                  - _scores_bf16(rank_b, B, base, prior, alpha, beta))
    E = _bound_matrix_fp8(rank_b, rank8, B, Bq, sB, base, prior, alpha, beta)
    assert (diff <= E).all(), float((diff - E).max())
    # the vocabulary-wide maximum agrees with the per-entry bound
    Emax = bounds.fp8_error_bound(rank_b, rank8, B, Bq, sB, base, prior, alpha, beta, chunk=100)
    np.testing.assert_allclose(Emax, E.max(axis=1), rtol=1e-12)
    # the bound is not vacuous: it stays within a small multiple of the worst true difference
    assert E.max() < 20 * diff.max() + 1e-6


# rank rows and B rows whose e4m3 rounding errs upwards: 0.68 -> 320/448 after absmax scaling
_UP = float(oracle.bf16_round(np.array([0.68], F32))[0])


@pytest.mark.parametrize("rank_row,B_row,alpha", [
    ([0.0, 1.0], [1.0, _UP], 1.7),      # B's rounding only (the rank is e4m3-exact)
    ([1.0, _UP], [0.0, 1.0], 1.7),      # the rank's rounding only (B is e4m3-exact)
    ([1.0, _UP], [1.0, _UP], 1.7),      # both, aligned: the product term eR.eB is needed as well
    ([1.0, _UP], [1.0, _UP], 0.3),
])
def test_fp8_bound_is_tight_on_aligned_errors(rank_row, B_row, alpha):
    rank = np.array([rank_row], F32)
    B = np.array([B_row, [1.0, 1.0]], F32)
    Bq, sB = oracle.quantize_rows_e4m3(B)
    base = np.zeros((1, 2), F32)
    a = np.array([alpha], F32)
    b = np.zeros(1, F32)
    s8 = _scores_fp8(rank, Bq, sB, base, None, a, b)[0, 0]
    sb = _scores_bf16(rank, B, base, None, a, b)[0, 0]
    E = bounds.fp8_bound_at(rank, rank, B, Bq, sB, base, None, a, b, np.array([0]))[0]
    diff = abs(float(s8) - float(sb))
    assert diff > 0.0
    assert diff <= E and diff >= 0.99 * E, (diff, E)


def _eager_case(seed, M=6, d=64, r=48, V=400, scale=0.02, with_prior=True):
    rng = np.random.default_rng(seed)
    h = oracle.bf16_round(rng.standard_normal((M, d)).astype(F32))
    A = oracle.bf16_round((rng.standard_normal((r, d)) * scale).astype(F32))
    B = oracle.bf16_round((rng.standard_normal((V, r)) * scale).astype(F32))
    base = (rng.standard_normal((M, V)) * 3).astype(F32)
    prior = np.log(rng.dirichlet(np.ones(V))).astype(F32) if with_prior else None
    alpha = rng.uniform(0.0, 2.0, M).astype(F32)
    beta = rng.uniform(0.0, 0.6, M).astype(F32)
    beta[1] = 0.0
    return h, A, B, base, prior, alpha, beta


def _eager_vs_fused(h, A, B, base, prior, alpha, beta):
    t = torch.from_numpy
    fin = torch_eager.eager_logits_bf16(t(h), t(A), t(B), t(base), None if prior is None else t(prior), t(alpha),
                                        t(beta)).float().numpy()
    rank = oracle.rank_proj(h, A)
    s = _scores_bf16(rank, B, base, prior, alpha, beta)
    M, V = base.shape
    E = np.stack([bounds.eager_bound_at(rank, B, base, prior, alpha, beta, np.full(M, v)) for v in range(V)], axis=1)
    return np.abs(fin.astype(np.float64) - s), E, rank


@pytest.mark.parametrize("seed,scale,with_prior", [(0, 0.02, True), (1, 0.5, False), (2, 3.0, True)])
def test_eager_bound_dominates(seed, scale, with_prior):
    h, A, B, base, prior, alpha, beta = _eager_case(seed, scale=scale, with_prior=with_prior)
    diff, E, rank = _eager_vs_fused(h, A, B, base, prior, alpha, beta)
    assert (diff <= E).all(), float((diff - E).max())
    Emax = bounds.eager_bf16_error_bound(rank, B, base, prior, alpha, beta, chunk=128)
    np.testing.assert_allclose(Emax, E.max(axis=1), rtol=1e-12)


@pytest.mark.parametrize("which", ["base", "low_rank", "prior", "cancelling"])
def test_eager_bound_covers_each_source_alone(which):
    """One rounding source at a time, the others switched off: the bound must cover each."""
    h, A, B, base, prior, alpha, beta = _eager_case(7, M=8, V=500, scale=0.5)
    if which == "base":                      # fp32 base cast to bf16 (alpha = 0, no prior)
        alpha[:] = 0.0
        prior = None
    elif which == "low_rank":                # bf16(short), bf16(alpha short): base 0, no prior
        base[:] = 0.0
        prior = None
    elif which == "prior":                   # bf16(beta bf16(prior)): base 0, alpha 0
        base[:] = 0.0
        alpha[:] = 0.0
        beta[:] = 0.45
    else:                                    # dot products that cancel: only accumulation order is left
        base[:] = 0.0
        prior = None
        h[:, :] = 1.0
        A[:, :] = 0.0
        A[:, 0] = 1.0
        B[:, 0::2] = oracle.bf16_round(np.full_like(B[:, 0::2], 1.0 + 2.0 ** -7))
        B[:, 1::2] = -oracle.bf16_round(np.full_like(B[:, 1::2], 1.0 + 2.0 ** -7))
        B[:, 1] = 2.0 ** -30
    diff, E, _ = _eager_vs_fused(h, A, B, base, prior, alpha, beta)
    assert (diff <= E).all(), float((diff - E).max())
    if which != "cancelling":
        assert diff.max() > 0.0              # the source really rounds in this case


def test_pick_consistent_flags_a_wrong_pick():
    s_ref = np.array([5.0, 5.0, 5.0])
    s_other = np.array([4.99, 4.0, 5.0])
    e = np.array([0.01, 0.01, 0.0])
    ok = bounds.pick_consistent(s_ref, s_other, e, e)
    assert ok.tolist() == [True, False, True]


@pytest.mark.parametrize("seed", [11, 12])
def test_eager_bound_with_rank_slack_covers_a_differently_rounded_rank(seed):
    """The other path's rank one bf16 ulp away (signs aligned with B's row of the entry
    checked, the worst case for it): the bound with ``rank_order_slack`` still covers it."""
    h, A, B, base, prior, alpha, beta = _eager_case(seed, M=5, V=300, scale=0.05)
    base[:] = 0.0                  # the rank shift is then the largest source of difference
    prior = None
    rank = oracle.rank_proj(h, A)
    D = bounds.rank_order_slack(h, A, rank)
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(rank), 2.0 ** -126))[1] - 8)
    assert (D >= ulp).all()
    M, V = base.shape
    rng = np.random.default_rng(seed)
    v_star = rng.integers(0, V, M)
    step = (np.sign(B[v_star]) * ulp).astype(F32)               # one ulp towards a larger dot with B[v_star]
    rank_p = (rank + step).astype(F32)
    assert (oracle.bf16_round(rank_p) == rank_p).all()
    t = torch.from_numpy
    eye = torch.eye(rank.shape[1])
    fin = torch_eager.eager_logits_bf16(t(rank_p), eye, t(B), t(base), None, t(alpha), t(beta)).float().numpy()
    s = _scores_bf16(rank, B, base, prior, alpha, beta)
    E = np.stack([bounds.eager_bound_at(rank, B, base, prior, alpha, beta, np.full(M, v), rank_slack=D)
                  for v in range(V)], axis=1)
    diff = np.abs(fin.astype(np.float64) - s)
    assert (diff <= E).all(), float((diff - E).max())
    # without the slack the shifted rank escapes the bound at the aligned entries of some row
    E0 = np.stack([bounds.eager_bound_at(rank, B, base, prior, alpha, beta, np.full(M, v)) for v in range(V)], axis=1)
    assert (diff > E0).any()
