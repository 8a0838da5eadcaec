"""Pins the oracle's rank projection and fused argmax.

Independent checks: torch library routines (F.linear, F.silu, torch.matmul,
torch.argmax), closed forms that remove one term at a time, a pure-Python
brute force on tiny shapes, planted maxima/ties, and permutation invariance.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _bf16(rng, shape, std=1.0):
    return oracle.bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def _case(seed, M=5, d=48, r=32, V=700):
    rng = np.random.default_rng(seed)
    h = _bf16(rng, (M, d))
    A = _bf16(rng, (r, d), 0.1)
    B = _bf16(rng, (V, r), 0.1)
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    prior = np.log(rng.dirichlet(np.ones(V))).astype(np.float32)
    alpha = rng.uniform(0, 0.6, M).astype(np.float32)
    beta = rng.uniform(0, 0.6, M).astype(np.float32)
    return h, A, B, base, prior, alpha, beta


# ---------------------------------------------------------------- rank projection

@pytest.mark.parametrize("act", ["identity", "silu"])
@pytest.mark.parametrize("bias", [False, True])
def test_rank_proj_matches_torch_linear(act, bias):
    rng = np.random.default_rng(3)
    h, A = _bf16(rng, (7, 64)), _bf16(rng, (40, 64), 0.1)
    b = _bf16(rng, (40,), 0.5) if bias else None
    got = oracle.rank_proj(h, A, b, act)
    # torch in float64: exact dot, then the two bf16 roundings the reference applies
    pre = F.linear(torch.from_numpy(h).double(), torch.from_numpy(A).double(),
                   None if b is None else torch.from_numpy(b).double())
    ref = pre.float().to(torch.bfloat16)
    if act == "silu":
        ref = F.silu(ref)  # torch's own bf16 silu (fp32 math, one rounding)
    np.testing.assert_array_equal(got, ref.float().numpy())


def test_rank_proj_rejects_unknown_activation():
    with pytest.raises(ValueError, match="Unsupported DeLS rank_activation"):
        oracle.rank_proj(np.zeros((1, 8), np.float32), np.zeros((8, 8), np.float32), act="gelu")


# ---------------------------------------------------------------- closed forms

def test_alpha_beta_zero_reduces_to_argmax_of_base():
    h, A, B, base, prior, _, _ = _case(4)
    rank = oracle.rank_proj(h, A)
    ids, score, second = oracle.fused_argmax(rank, B, base, prior, 0.0, 0.0)
    tb = torch.from_numpy(base)
    np.testing.assert_array_equal(ids, torch.argmax(tb, dim=1).numpy())
    np.testing.assert_array_equal(score, tb.max(dim=1).values.numpy())
    np.testing.assert_array_equal(second, torch.topk(tb, 2, dim=1).values[:, 1].numpy())


def test_zero_lm_head_reduces_to_base_minus_beta_prior():
    h, A, B, base, prior, alpha, beta = _case(5)
    rank = oracle.rank_proj(h, A)
    ids, score, _ = oracle.fused_argmax(rank, np.zeros_like(B), base, prior, alpha, beta)
    ref = torch.from_numpy(base) - torch.from_numpy(beta)[:, None] * torch.from_numpy(prior)[None, :]
    np.testing.assert_array_equal(ids, torch.argmax(ref, dim=1).numpy())
    np.testing.assert_allclose(score, ref.max(dim=1).values.numpy(), rtol=0, atol=1e-5)


def test_constant_base_no_prior_reduces_to_lowrank_logits():
    h, A, B, base, prior, alpha, _ = _case(6)
    rank = oracle.rank_proj(h, A)
    ids, score, _ = oracle.fused_argmax(rank, B, np.full_like(base, 2.5), prior, alpha, 0.0)
    logits = torch.matmul(torch.from_numpy(rank).double(), torch.from_numpy(B).double().T)
    ref = logits * torch.from_numpy(alpha).double()[:, None] + 2.5
    np.testing.assert_array_equal(ids, torch.argmax(ref, dim=1).numpy())
    np.testing.assert_allclose(score, ref.max(dim=1).values.numpy(), rtol=1e-6, atol=1e-6)


def test_prior_skipped_when_beta_zero_or_absent():
    h, A, B, base, prior, alpha, beta = _case(7)
    rank = oracle.rank_proj(h, A)
    beta = beta.copy()
    beta[::2] = 0.0
    inf_prior = prior.copy()
    inf_prior[10] = np.inf   # would poison rows whose beta is used
    ids, score, _ = oracle.fused_argmax(rank, B, base, inf_prior, alpha, beta)
    ids_np, score_np, _ = oracle.fused_argmax(rank, B, base, None, alpha, beta)
    np.testing.assert_array_equal(ids[::2], ids_np[::2])
    np.testing.assert_array_equal(score[::2], score_np[::2])
    assert np.all(np.isneginf(score[1::2]) | (ids[1::2] != 10))


# ---------------------------------------------------------------- brute force

def _round_f32_exact(x: Fraction) -> np.float32:
    """A rational rounded to the nearest float32 (ties to even), by integer arithmetic."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    ax = abs(x)
    e = ax.numerator.bit_length() - ax.denominator.bit_length()   # 2**e <= ax < 2**(e+2)
    if Fraction(2) ** e > ax:
        e -= 1
    elif Fraction(2) ** (e + 1) <= ax:
        e += 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    q = ax / quantum
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(n * quantum))


def _fma_exact(a, b, c) -> np.float32:
    """``a * b + c`` of float32 values in exact rational arithmetic, rounded once to float32."""
    return _round_f32_exact(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _brute_force(rank, B, base, prior, alpha, beta):
    """Element-by-element evaluation with Python loops (tiny shapes only): the dot in
    exact rational arithmetic rounded once to fp32, the combine as two exact fmas."""
    f32 = np.float32
    M, V = base.shape
    ids, best = [], []
    for m in range(M):
        bv, bi = None, None
        for v in range(V):
            dot = _round_f32_exact(sum(Fraction(float(rank[m, k])) * Fraction(float(B[v, k]))
                                       for k in range(rank.shape[1])))
            s = _fma_exact(dot, f32(alpha[m]), f32(base[m, v]))
            if prior is not None and beta[m] != 0:
                s = _fma_exact(-f32(beta[m]), f32(prior[v]), s)
            if bv is None or s > bv:
                bv, bi = s, v
        ids.append(bi)
        best.append(bv)
    return np.array(ids), np.array(best, np.float32)


def test_fma_f32_is_correctly_rounded():
    """oracle.fma_f32 against exact rational arithmetic, on random operands with
    cancellation and on a constructed case that only a correct second rounding
    gets right: 1 + (2**-24 + 2**-60) lies just above the float32 midpoint
    between 1 and 1 + 2**-23 but rounds to the midpoint in float64."""
    rng = np.random.default_rng(5)
    n = 4000
    a = (rng.uniform(1, 2, n) * 2.0 ** rng.integers(-8, 8, n)).astype(np.float32)
    b = (rng.uniform(-2, 2, n) * 2.0 ** rng.integers(-8, 8, n)).astype(np.float32)
    c = (-(a.astype(np.float64) * b) * rng.uniform(0.5, 1.5, n)).astype(np.float32)   # cancellation
    a[:4] = [1 + 2.0 ** -12, 1.0, 3.0, np.float32(np.inf)]
    b[:4] = [np.float32(2.0 ** -24 * (1 - 2.0 ** -12 + 2.0 ** -24)), 1.0, 0.5, 1.0]
    c[:4] = [1.0, -1.0, 0.25, 1.0]
    got = oracle.fma_f32(a, b, c)
    exact = np.array([_fma_exact(x, y, z) if np.isfinite(x) else np.float32(np.inf) for x, y, z in zip(a, b, c)],
                     np.float32)
    np.testing.assert_array_equal(got, exact)
    assert got[0] == np.float32(1 + 2.0 ** -23)
    two_step = ((a * b).astype(np.float32) + c).astype(np.float32)
    assert two_step[0] == np.float32(1.0)              # separate roundings land on the other neighbour
    assert np.count_nonzero(two_step[4:] != exact[4:]) > 50   # the cases distinguish fma from two roundings


@pytest.mark.parametrize("seed", [10, 11, 12])
def test_fused_argmax_matches_brute_force(seed):
    h, A, B, base, prior, alpha, beta = _case(seed, M=3, d=16, r=8, V=97)
    rank = oracle.rank_proj(h, A)
    ids, score, _ = oracle.fused_argmax(rank, B, base, prior, alpha, beta, chunk=13)
    bi, bs = _brute_force(rank, B, base, prior, alpha, beta)
    np.testing.assert_array_equal(ids, bi)
    np.testing.assert_array_equal(score, bs)


# ---------------------------------------------------------------- planted cases

def test_planted_tail_maximum_and_cross_chunk_ties():
    h, A, B, base, prior, alpha, beta = _case(13, M=4, V=1000)
    rank = oracle.rank_proj(h, A)
    base = base.copy()
    base[0, 999] = 1e4                       # last index (tail of the vocabulary)
    base[1, 100] = base[1, 900] = 1e4        # tie across chunks -> lower index
    base[2, 5] = base[2, 6] = 1e4            # tie within a chunk -> lower index
    B = B.copy()
    B[[999, 100, 900, 5, 6]] = 0.0
    prior = prior.copy()
    prior[[999, 100, 900, 5, 6]] = 0.0
    ids, score, second = oracle.fused_argmax(rank, B, base, prior, alpha, beta, chunk=256)
    assert ids[0] == 999 and ids[1] == 100 and ids[2] == 5
    assert score[1] == second[1] == np.float32(1e4)


def test_all_neg_inf_row_returns_zero():
    _, _, B, base, prior, alpha, beta = _case(14, M=2, V=300)
    rank = np.zeros((2, B.shape[1]), np.float32)
    base = base.copy()
    base[1] = -np.inf
    ids, score, _ = oracle.fused_argmax(rank, B, base, prior, alpha, beta, chunk=64)
    assert ids[1] == 0 and np.isneginf(score[1])


def test_permutation_invariance():
    h, A, B, base, prior, alpha, beta = _case(15, V=500)
    rank = oracle.rank_proj(h, A)
    perm = np.random.default_rng(0).permutation(500)
    ids, score, _ = oracle.fused_argmax(rank, B, base, prior, alpha, beta)
    pid, pscore, _ = oracle.fused_argmax(rank, B[perm], base[:, perm], prior[perm], alpha, beta)
    np.testing.assert_array_equal(perm[pid], ids)
    np.testing.assert_array_equal(pscore, score)


def test_score_at_agrees_with_argmax():
    h, A, B, base, prior, alpha, beta = _case(16)
    rank = oracle.rank_proj(h, A)
    ids, score, _ = oracle.fused_argmax(rank, B, base, prior, alpha, beta)
    np.testing.assert_array_equal(oracle.score_at(rank, B, base, prior, alpha, beta, ids), score)


# ---------------------------------------------------------------- eager bf16 semantics

def test_eager_bf16_matches_torch_bf16_ops():
    # Inputs chosen so every dot product is exact in fp32: then torch's bf16
    # F.linear and the oracle agree bit-for-bit and the remaining ops are
    # torch's own bf16 elementwise arithmetic.
    rng = np.random.default_rng(17)
    M, r, V = 4, 16, 2000
    rank = (rng.integers(-8, 8, (M, r)) / 8).astype(np.float32)
    B = (rng.integers(-8, 8, (V, r)) / 16).astype(np.float32)
    base = oracle.bf16_round((rng.standard_normal((M, V)) * 3).astype(np.float32))
    prior = oracle.bf16_round(np.log(rng.dirichlet(np.ones(V))).astype(np.float32))
    alpha, beta = 0.3, 0.45
    got = oracle.eager_argmax_bf16(rank, B, base, prior, alpha, beta)
    tb = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)  # noqa: E731
    short = F.linear(tb(rank), tb(B))
    final = tb(base) + alpha * short
    final = final - beta * tb(prior).view(1, -1)
    np.testing.assert_array_equal(got, torch.argmax(final, dim=-1).numpy())


def test_check_parity_rule():
    ref_ids = np.array([3, 4, 5])
    ref_sc = np.array([10.0, 10.0, 10.0], np.float32)
    ref_sec = np.array([9.0, 9.9999, 9.0], np.float32)   # row 1 is within 1e-3 relative
    dev_ids = np.array([3, 7, 6])
    res = oracle.check_parity(dev_ids, ref_sc, ref_ids, ref_sc, ref_sec)
    assert res["pinned"] == 2 and res["id_mismatch_pinned"] == 1 and res["bad_rows"] == [2]
    res = oracle.check_parity(ref_ids, ref_sc + np.float32(0.02), ref_ids, ref_sc, ref_sec)
    assert res["score_bad"] == 3
