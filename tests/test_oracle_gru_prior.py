"""Pins the oracle's GRU step, input table, rollout and unigram prior."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _bf16(rng, shape, std=1.0):
    return oracle.bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


@pytest.mark.parametrize("with_bias", [False, True])
def test_gru_cell_matches_torch_gru(with_bias):
    rng = np.random.default_rng(20)
    nb, E, G = 5, 24, 32
    x = _bf16(rng, (nb, E))
    h = _bf16(rng, (nb, G), 0.5)
    W_ih, W_hh = _bf16(rng, (3 * G, E), 0.3), _bf16(rng, (3 * G, G), 0.3)
    b_ih = _bf16(rng, (3 * G,), 0.2) if with_bias else None
    b_hh = _bf16(rng, (3 * G,), 0.2) if with_bias else None
    gi = oracle.gru_input_table(x, W_ih, b_ih)
    got = oracle.gru_cell(gi, h, W_hh, b_hh)
    # torch.nn.GRU (gate order r, z, n) in float64 as the mathematical reference
    gru = torch.nn.GRU(E, G, num_layers=1, batch_first=True, bias=with_bias).double()
    with torch.no_grad():
        gru.weight_ih_l0.copy_(torch.from_numpy(W_ih))
        gru.weight_hh_l0.copy_(torch.from_numpy(W_hh))
        if with_bias:
            gru.bias_ih_l0.copy_(torch.from_numpy(b_ih))
            gru.bias_hh_l0.copy_(torch.from_numpy(b_hh))
        _, ref = gru(torch.from_numpy(x).double().unsqueeze(1), torch.from_numpy(h).double().unsqueeze(0))
    ref = ref[0].numpy()
    # bf16 roundings of gi, gh and h' separate the two: a few bf16 ulps
    assert np.max(np.abs(got - ref)) < 3e-2
    assert np.mean(np.abs(got - ref)) < 3e-3
    # a swapped update rule ((1 - z) * h + z * n) is far off
    gh = F.linear(torch.from_numpy(h).double(), torch.from_numpy(W_hh).double()).numpy()
    gir, giz, gin = np.split(gi.astype(np.float64), 3, axis=1)
    ghr, ghz, ghn = np.split(gh, 3, axis=1)
    sig = lambda v: 1 / (1 + np.exp(-v))  # noqa: E731
    if not with_bias:
        rg, zg = sig(gir + ghr), sig(giz + ghz)
        swapped = (1 - zg) * h + zg * np.tanh(gin + rg * ghn)
        assert np.max(np.abs(got - swapped)) > 0.1


def test_gru_input_table_matches_linear():
    rng = np.random.default_rng(21)
    E, W, b = _bf16(rng, (50, 16)), _bf16(rng, (24, 16), 0.3), _bf16(rng, (24,), 0.3)
    ref = F.linear(torch.from_numpy(E).double(), torch.from_numpy(W).double(), torch.from_numpy(b).double())
    np.testing.assert_array_equal(oracle.gru_input_table(E, W, b),
                                  ref.float().to(torch.bfloat16).float().numpy())


def test_rollout_matches_step_by_step_composition():
    rng = np.random.default_rng(22)
    nb, steps, V, E, G, r = 2, 5, 300, 16, 24, 16
    E_w = _bf16(rng, (V, E))
    W_ih, W_hh = _bf16(rng, (3 * G, E), 0.3), _bf16(rng, (3 * G, G), 0.3)
    A, Bw = _bf16(rng, (r, G), 0.3), _bf16(rng, (V, r), 0.3)
    gi_table = oracle.gru_input_table(E_w, W_ih)
    base = (rng.standard_normal((nb, steps, V)) * 3).astype(np.float32)
    prior = np.log(rng.dirichlet(np.ones(V))).astype(np.float32)
    alphas, betas = [0.3] * steps, [0.1, 0.0, 0.2, 0.3, 0.4]
    prefix = np.array([3, 250])
    ids, scores, _ = oracle.rollout(prefix, base, gi_table=gi_table, W_hh=W_hh, b_hh=None, A=A, rank_bias=None,
                                    act="silu", B=Bw, prior=prior, alphas=alphas, betas=betas)
    # the same recurrence written with torch.nn.GRUCell / F.linear / torch.argmax (float64)
    cell = torch.nn.GRUCell(E, G, bias=False).double()
    with torch.no_grad():
        cell.weight_ih.copy_(torch.from_numpy(W_ih))
        cell.weight_hh.copy_(torch.from_numpy(W_hh))
    emb = torch.from_numpy(E_w).double()
    torch.set_grad_enabled(False)
    h = cell(emb[torch.from_numpy(prefix)], torch.zeros(nb, G, dtype=torch.float64))
    for s in range(steps):
        rank = F.silu(F.linear(h, torch.from_numpy(A).double()))
        logits = F.linear(rank, torch.from_numpy(Bw).double()) * alphas[s] + torch.from_numpy(base[:, s])
        if betas[s] != 0:
            logits = logits - betas[s] * torch.from_numpy(prior).double()
        top2 = torch.topk(logits, 2, dim=1).values
        margin = ((top2[:, 0] - top2[:, 1]) / top2[:, 0].abs()).numpy()
        tok = torch.argmax(logits, dim=1)
        # bf16 rounding of the recurrent state may only flip near-ties
        ok = (tok.numpy() == ids[:, s]) | (margin < 1e-2)
        assert ok.all(), (s, tok, ids[:, s], margin)
        tok = torch.from_numpy(ids[:, s])      # follow the oracle's own path
        h = cell(emb[tok], h)
    torch.set_grad_enabled(True)


def test_unigram_prior_closed_form():
    got = oracle.unigram_log_prior([1, 3], vocab_size=4, smoothing=1.0)
    np.testing.assert_allclose(got, np.log([2 / 8, 4 / 8, 1 / 8, 1 / 8]), rtol=0, atol=1e-15)
    got = oracle.unigram_log_prior([2, 0, 6], vocab_size=3, smoothing=0.0)
    np.testing.assert_allclose(got, [math.log(2 / 8), math.log(2 / 8), math.log(6 / 8)], atol=1e-15)
    assert np.isclose(np.exp(oracle.unigram_log_prior(np.arange(10), 12, 0.5)).sum(), 1.0)
    with pytest.raises(ValueError, match="exceeds runtime vocab"):
        oracle.unigram_log_prior([1, 2, 3], vocab_size=2)
    with pytest.raises(ValueError, match="no positive counts"):
        oracle.unigram_log_prior([0, 0], vocab_size=2, smoothing=0.0)
    with pytest.raises(ValueError, match="non-negative"):
        oracle.unigram_log_prior([1], vocab_size=2, smoothing=-1.0)


def test_fp8_oracle_reduces_to_bf16_with_unit_scales():
    # weights already on the e4m3 grid with row absmax 448 -> scale 1, quantisation is the identity
    rng = np.random.default_rng(23)
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    grid = grid[np.isfinite(grid) & (np.abs(grid) <= 448) & (np.abs(grid) >= 2 ** -6)]
    M, d, r, V = 3, 32, 16, 200
    A = rng.choice(grid, (r, d)).astype(np.float32)
    A[:, 0] = 448.0
    Bq = rng.choice(grid, (V, r)).astype(np.float32)
    Bq[:, 0] = 448.0
    h = _bf16(rng, (M, d), 1e-3)
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    qa, sa = oracle.quantize_rows_e4m3(A)
    qb, sb = oracle.quantize_rows_e4m3(Bq)
    np.testing.assert_array_equal(qa, A)
    np.testing.assert_array_equal(sa, 1.0)
    rank, ids, score, _ = oracle.lowrank_argmax_fp8(h, qa, sa, None, "identity", qb, sb, base, None, 1e-6, 0.0)
    np.testing.assert_array_equal(rank, oracle.rank_proj(h, A))
    # scaling each B row by 2^k moves its scale, not the result
    k = rng.integers(-3, 4, V).astype(np.float32)
    qb2, sb2 = oracle.quantize_rows_e4m3(Bq * np.exp2(k)[:, None])
    np.testing.assert_array_equal(qb2, qb)
    np.testing.assert_array_equal(sb2, np.exp2(k).astype(np.float32))
    _, ids2, score2, _ = oracle.lowrank_argmax_fp8(h, qa, sa, None, "identity", qb2, sb2, base, None, 1e-6, 0.0)
    raw = oracle.fused_argmax(rank, Bq * np.exp2(k)[:, None], base, None, 1e-6, 0.0)
    # the fp8 path quantises rank per row; with alpha tiny the base term dominates both
    np.testing.assert_array_equal(ids2, raw[0])


# ------------------------------------------------------------------ Markov rollout

def test_markov_rollout_follows_the_chain():
    """Rows of E orthonormal and B[pi(t)] = 10 E[t]: from token t the low-rank logit is 10 at
    pi(t) and 0 elsewhere, so with a small base every step moves t -> pi(t) and the rollout
    visits pi^(s+1)(prev) -- a rollout feeding the wrong token (the previous one, or the
    step's own input) would not."""
    rng = np.random.default_rng(4)
    V, r, nb, steps = 50, 64, 3, 6
    Q, _ = np.linalg.qr(rng.standard_normal((r, r)))
    E = Q[:V].astype(np.float32)
    pi = rng.permutation(V)
    B = np.zeros((V, r), np.float32)
    B[pi] = 10 * E
    base = (rng.standard_normal((nb, steps, V)) * 0.1).astype(np.float32)
    prior = np.log(rng.dirichlet(np.ones(V))).astype(np.float32) * 0.01
    prev = np.array([0, 7, 49])
    ids, scores, _ = oracle.markov_rollout(prev, base, E=E, B=B, prior=prior, alphas=[1.0] * steps,
                                           betas=[0.2] * steps)
    want = np.zeros((nb, steps), np.int64)
    t = prev.copy()
    for s in range(steps):
        t = pi[t]
        want[:, s] = t
    np.testing.assert_array_equal(ids, want)
    assert np.all(scores > 9.0)
    # teacher forcing: each step starts from the forced token
    forced = rng.integers(0, V, (nb, steps))
    fids, _, _ = oracle.markov_rollout(prev, base, E=E, B=B, prior=prior, alphas=[1.0] * steps,
                                       betas=[0.2] * steps, forced_ids=forced)
    np.testing.assert_array_equal(fids[:, 0], pi[prev])
    np.testing.assert_array_equal(fids[:, 1:], pi[forced[:, :-1]])
